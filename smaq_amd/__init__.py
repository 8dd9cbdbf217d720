"""smaq_amd -- MI355X-native (gfx950) SMAQ quantized-KV hot path.

Drop-in for the ``smaq`` package's hot-path API: the key codecs
(``SMAQQuantizer``, ``RotationAdapter``, ``SMAQBlockVQ``), the value codec
(``quantize_values`` / ``dequantize_values``), the strategies, the
compressed store and ``compute_hybrid_attention``.  The arithmetic runs in
hand-written HIP kernels (libsmaq_hip.so, C ABI in include/smaq_hip.h).
"""

from smaq_amd.integration.vllm import (MODE_CAPTURE_ONLY, MODE_FULL_SMAQ, MODE_HYBRID, MODE_OFF, free_kv_cache,
                                       get_mode, get_stats, install_hooks, set_mode)
from smaq_amd.backends import HipHybridAttentionBackend, TorchHybridAttentionBackend
from smaq_amd.block_vq import BlockVQQuantized, SMAQBlockVQ
from smaq_amd.calibration import IdentityCalibrationProvider, StaticCalibrationProvider
from smaq_amd.capture import KVCaptureEngine, RingBuffer
from smaq_amd.core import (AttentionBackend, CacheBackend, CacheCapabilities, CalibrationProvider, LayoutInfo,
                           MetricStrategy, ModelLayoutAdapter, QuantizationStrategy)
from smaq_amd.layout import (GemmaModelLayoutAdapter, GenericModelLayoutAdapter, QwenModelLayoutAdapter,
                             infer_model_layout_adapter)
from smaq_amd.kv_cache import SMAQKVCache, ValueQuantized, dequantize_values, quantize_values, unpack_values
from smaq_amd.quantizer import SMAQQuantized, SMAQQuantizer
from smaq_amd.score import MIN_HISTORY_FOR_SMAQ, HybridAttentionBackend, compute_hybrid_attention
from smaq_amd.store import CompressedKVStore, FlatCache
from smaq_amd.strategies import (ExactShadowStrategy, IdentityMetricStrategy, IdentityScalarStrategy,
                                 SMAQBlockVQStrategy, SMAQDiagonalMetricState, SMAQDiagonalMetricStrategy,
                                 SMAQFullMetricScalarStrategy, SMAQFullMetricStrategy)
from smaq_amd.weighted_scalar import (RotationAdapter, SMAQWeightedRotationQuantizer,
                                      build_block_diagonal_metric_scales, build_codebook,
                                      build_rotated_diagonal_metric_scales)

__version__ = "0.1.0"
