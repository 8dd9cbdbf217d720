// Internal declarations shared by the key encoders (not part of the C ABI).
#pragma once

#include "smaq_common.h"

namespace smaq {

// Number of decision boundaries strictly below y (searchsorted, left side);
// NaN maps to the top code.  `ties` counts values within 1e-6 relative of a
// boundary (possible argmin / rounding ties against the reference).
__device__ __forceinline__ int count_below(const float* bounds, int nb, float y, unsigned* ties) {
  if (y != y) return nb;
  int c = 0;
  bool tie = false;
  for (int i = 0; i < nb; ++i) {
    const float b = bounds[i];
    c += (b < y) ? 1 : 0;
    const float tol = 1e-6f * fmaxf(fmaxf(fabsf(b), fabsf(y)), 1e-6f);
    tie |= fabsf(y - b) <= tol;
  }
  *ties += tie ? 1u : 0u;
  return c;
}

// Matrix-core scalar encoder (scalar_encode_mfma.hip): D = 128, 2/3/4-bit
// codes, at most 15 boundaries, 16-byte aligned key and code rows.
bool encode_scalar_mfma_supported(int D, int bits, int nb, const void* codes_out, const void* k,
                                  int kdtype, long long s_outer, long long s_inner);
int launch_encode_scalar_mfma(int kdtype, const void* k, RowMap map, int64_t rows, const float* Mt,
                              const float* cs, const float* bounds, int nb, int bits, void* codes,
                              void* norms, unsigned long long* ties, hipStream_t st);

// Matrix-core block-VQ encoder (blockvq_encode_mfma.hip): 8-dim blocks, 256
// centroids, at most 16 blocks, 16-byte aligned key rows.
bool encode_blockvq_mfma_supported(int nb, int bd, int nc, const void* k, int kdtype,
                                   long long s_outer, long long s_inner);
size_t encode_blockvq_mfma_lds(int nb);
int launch_encode_blockvq_mfma(int kdtype, const void* k, RowMap map, int64_t rows, int nb,
                               const float* E_blocks, const float* C, uint8_t* idx,
                               unsigned long long* ties, hipStream_t st);

}  // namespace smaq
