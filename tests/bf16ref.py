"""numpy bfloat16 rounding model used to pin the oracle's per-op rounding
independently of torch: every elementwise op computed in float32, then
rounded to the nearest bf16 (ties to even)."""

import numpy as np


def bf16_round(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    out = u.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out)
