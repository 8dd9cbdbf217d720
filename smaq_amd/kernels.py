"""Score kernel entry point (replaces smaq/triton_kernels.py).

``smaq_attention_scores`` keeps the reference's name and contract
(smaq/triton_kernels.py:190-208): unscaled fp32 scores
(q @ E_inv^T) . c[code] * norm for any query shape, computed by the HIP score
kernel.  There is no fallback path: failures raise.
"""

from __future__ import annotations

import logging

import torch

from smaq_amd.quantizer import SMAQQuantized, scores_from_codes

# the reference's logger name for this seam (smaq/triton_kernels.py:20)
logger = logging.getLogger("smaq.triton")


def smaq_attention_scores(quantizer, query: torch.Tensor, quantized_key: SMAQQuantized) -> torch.Tensor:
    if logger.isEnabledFor(logging.DEBUG):
        logger.debug("HIP score kernel: query %s, %s keys", tuple(query.shape), tuple(quantized_key.indices.shape))
    q_rot = quantizer.rotate_query(query)
    return scores_from_codes(q_rot, quantized_key.indices, quantized_key.norms, quantized_key.bits,
                             quantizer.centroids, None, torch.float32)
