"""The reference's import paths resolve: every name ``smaq/__init__.py``
exports (smaq/__init__.py:1-43), and the module paths its callers and its
own modules import from -- ``smaq.score``, ``smaq.store``, ``smaq.kv_cache``,
the kernel seam ``smaq.triton_kernels`` (smaq/quantizer.py:172), the vLLM
shim and adapter (smaq/vllm_attn_backend.py, smaq/integration/vllm.py).
CPU only: nothing here launches a kernel."""

from __future__ import annotations

import importlib

import pytest

# smaq/__init__.py:1-43, module by module
REFERENCE_EXPORTS = {
    "smaq.backends": ["TorchHybridAttentionBackend"],
    "smaq.calibration": ["IdentityCalibrationProvider", "StaticCalibrationProvider"],
    "smaq.block_vq": ["BlockVQQuantized", "SMAQBlockVQ"],
    "smaq.core": ["AttentionBackend", "CacheBackend", "CacheCapabilities", "CalibrationProvider", "LayoutInfo",
                  "MetricStrategy", "ModelLayoutAdapter", "QuantizationStrategy"],
    "smaq.capture": ["KVCaptureEngine", "RingBuffer"],
    "smaq.kv_cache": ["SMAQKVCache"],
    "smaq.layout": ["GemmaModelLayoutAdapter", "GenericModelLayoutAdapter", "QwenModelLayoutAdapter",
                    "infer_model_layout_adapter"],
    "smaq.quantizer": ["SMAQQuantized", "SMAQQuantizer"],
    "smaq.score": ["compute_hybrid_attention"],
    "smaq.strategies": ["ExactShadowStrategy", "IdentityMetricStrategy", "IdentityScalarStrategy",
                        "SMAQBlockVQStrategy", "SMAQDiagonalMetricState", "SMAQDiagonalMetricStrategy",
                        "SMAQFullMetricScalarStrategy", "SMAQFullMetricStrategy"],
    "smaq.store": ["CompressedKVStore"],
    "smaq.weighted_scalar": ["RotationAdapter", "SMAQWeightedRotationQuantizer",
                             "build_rotated_diagonal_metric_scales", "build_block_diagonal_metric_scales",
                             "build_codebook"],
}

# module-level names the reference's modules import from each other or that
# its documented callers use
MODULE_NAMES = {
    "smaq.kv_cache": ["ValueQuantized", "quantize_values", "dequantize_values", "unpack_values"],
    "smaq.score": ["MIN_HISTORY_FOR_SMAQ", "HybridAttentionBackend"],
    "smaq.store": ["FlatCache"],
    "smaq.ssf": ["ssf_log", "build_smaq_metric"],
    "smaq.triton_kernels": ["smaq_attention_scores"],
    "smaq.vllm_attn_backend": ["MODE_SHADOW", "MODE_ACCUMULATE", "MODE_ACTIVE", "set_mode", "get_mode",
                               "install_smaq_hooks", "enable_no_alloc", "free_kv_cache"],
    "smaq.integration": ["install_hooks", "get_stats", "set_mode", "get_mode", "free_kv_cache"],
    "smaq.integration.vllm": ["MODE_OFF", "MODE_CAPTURE_ONLY", "MODE_HYBRID", "MODE_FULL_SMAQ", "LayerConfig",
                              "LayerState", "install_hooks", "free_kv_cache", "get_stats", "set_mode", "get_mode"],
}


@pytest.mark.parametrize("module", sorted(set(REFERENCE_EXPORTS) | set(MODULE_NAMES)))
def test_module_path_resolves(module):
    mod = importlib.import_module(module)
    for name in REFERENCE_EXPORTS.get(module, []) + MODULE_NAMES.get(module, []):
        assert hasattr(mod, name), f"{module}.{name} missing"


def test_package_exports_and_identity():
    import smaq
    import smaq_amd
    for module, names in REFERENCE_EXPORTS.items():
        for name in names:
            assert getattr(smaq, name) is getattr(importlib.import_module(module), name)
    assert smaq.__version__ == "0.1.0"
    # one implementation: aliases share module objects (and module state)
    import smaq.integration.vllm as adapter
    assert adapter is smaq_amd.integration.vllm and smaq.score is smaq_amd.score
    from smaq.triton_kernels import smaq_attention_scores
    from smaq_amd.kernels import smaq_attention_scores as seam
    assert smaq_attention_scores is seam
