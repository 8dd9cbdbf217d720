// Block-VQ key codec: encoder (nearest codeword under the per-block SMAQ
// metric) and the pre-decoded-centroid dequantiser.
//
// Bit-exactness against torch-CPU (smaq/block_vq.py:216-244):
//  * x_i = sum_d k_d * E_b[i][d], sequential FMA over d (sgemm order).
//  * |x|^2 and |c|^2: sequential multiply-then-add (x.pow(2).sum(-1)).
//  * cdist takes its matmul form: d2 = fma-chain over k of (-2 x_k) * c_k,
//    then + |x|^2, then + |c|^2 (the [-2x, |x|^2, 1] . [c, 1, |c|^2] row
//    product, k = 0..bd+1), clamp_min(0), sqrt, first-index argmin.
//  * The argmin is over sqrt(d2).  sqrt is monotone, so the winner is the
//    first index whose d2 shares the smallest sqrt value; two d2 values can
//    only share one when they are within ~2^-22 of each other, so the exact
//    sqrt comparison is only evaluated for such near-equal records.  (torch's
//    vectorised sqrt is itself not correctly rounded; where that decides the
//    winner the two distances are within 1 ulp -- a counted tie.)
#include "encode_internal.h"

namespace smaq {

constexpr int kVqMaxBlockDim = 16;
constexpr int kVqMaxCentroids = 256;
constexpr int kVqThreads = 256;

template <typename T>
__global__ __launch_bounds__(kVqThreads) void encode_blockvq_kernel(
    const T* __restrict__ k, RowMap map, int64_t rows, int nb, int bd, int nc,
    const float* __restrict__ E_blocks, const float* __restrict__ C, uint8_t* __restrict__ idx_out,
    unsigned long long* tie_count) {
  extern __shared__ float csq[];  // [nb][nc]
  for (int i = threadIdx.x; i < nb * nc; i += blockDim.x) {
    const float* c = C + (int64_t)i * bd;
    float s = 0.0f;
    for (int e = 0; e < bd; ++e) s = s + c[e] * c[e];
    csq[i] = s;
  }
  __syncthreads();
  unsigned ties = 0;
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row < rows) {
    const T* kr = k + map.offset(row);
    for (int b = 0; b < nb; ++b) {
      float kb[kVqMaxBlockDim];
      float x[kVqMaxBlockDim];
#pragma unroll
      for (int d = 0; d < kVqMaxBlockDim; ++d) kb[d] = d < bd ? Num<T>::to_f(kr[b * bd + d]) : 0.f;
      const float* E = E_blocks + (int64_t)b * bd * bd;
      float xsq = 0.0f;
#pragma unroll
      for (int i = 0; i < kVqMaxBlockDim; ++i) {
        if (i < bd) {
          float a = 0.0f;
#pragma unroll
          for (int d = 0; d < kVqMaxBlockDim; ++d)
            if (d < bd) a = fmaf(kb[d], E[i * bd + d], a);
          x[i] = -2.0f * a;  // exact
          xsq = xsq + a * a;
        } else {
          x[i] = 0.f;
        }
      }
      const float* Cb = C + (int64_t)b * nc * bd;
      const float* cq = csq + b * nc;
      float best = __builtin_inff();  // smallest d2 seen
      float lo_cut = best;            // below this a record is surely a new sqrt class
      float second = __builtin_inff();
      int best_i = 0;
      bool seen_nan = false;
      for (int c = 0; c < nc; ++c) {
        const float* cc = Cb + c * bd;
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < kVqMaxBlockDim; ++e)
          if (e < bd) a = fmaf(x[e], cc[e], a);
        a = a + xsq;
        a = a + cq[c];
        a = a < 0.0f ? 0.0f : a;  // clamp_min(0); NaN passes
        if (seen_nan) continue;    // torch argmin returns the first NaN
        if (a != a) {
          best_i = c;
          seen_nan = true;
          continue;
        }
        if (a < best) {
          if (a < lo_cut || sqrtf(a) < sqrtf(best)) {
            second = best;
            best_i = c;
          } else {
            second = fminf(second, a);  // same sqrt value: the earlier index stays
          }
          best = a;
          lo_cut = best * (1.0f - 0x1p-19f);
        } else {
          second = fminf(second, a);
        }
      }
      if (!seen_nan && second <= best * (1.0f + 2e-6f)) ++ties;
      idx_out[map.out_row(row) * nb + b] = (uint8_t)best_i;
    }
  }
  add_count(tie_count, ties);
}

__global__ __launch_bounds__(256) void dequant_blockvq_kernel(const uint8_t* __restrict__ idx,
                                                              int64_t rows, int nb, int bd, int nc,
                                                              const float* __restrict__ decoded,
                                                              float* __restrict__ out) {
  const int D = nb * bd;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * D) return;
  const int64_t r = i / D;
  const int d = (int)(i - r * D);
  const int b = d / bd;
  const int c = min((int)idx[r * nb + b], nc - 1);
  out[i] = decoded[((int64_t)b * nc + c) * bd + (d - b * bd)];
}

}  // namespace smaq

using namespace smaq;

extern "C" int smaq_encode_blockvq(const void* k, int kdtype, long long n_outer, long long n_inner,
                                   long long s_outer, long long s_inner, long long out_outer, int n_blocks,
                                   int block_dim, int n_centroids, const float* E_blocks,
                                   const float* centroids, void* idx_out,
                                   unsigned long long* tie_count, void* stream) {
  SMAQ_REQUIRE(k && E_blocks && centroids && idx_out, "smaq_encode_blockvq: null pointer");
  SMAQ_REQUIRE(block_dim >= 1 && block_dim <= kVqMaxBlockDim,
               "smaq_encode_blockvq: block_dim must be in [1, %d], got %d", kVqMaxBlockDim,
               block_dim);
  SMAQ_REQUIRE(n_centroids >= 1 && n_centroids <= kVqMaxCentroids,
               "smaq_encode_blockvq: n_centroids must be in [1, 256], got %d", n_centroids);
  SMAQ_REQUIRE(n_blocks >= 1 && n_blocks * n_centroids * 4 <= 65536,
               "smaq_encode_blockvq: codebook too large (%d blocks x %d centroids)", n_blocks,
               n_centroids);
  SMAQ_REQUIRE(n_outer >= 0 && n_inner > 0, "smaq_encode_blockvq: bad row shape");
  SMAQ_REQUIRE(out_outer == 0 || out_outer >= n_inner, "smaq_encode_blockvq: output rows overlap "
               "(out_outer %lld < n_inner %lld)", out_outer, n_inner);
  const int64_t rows = (int64_t)n_outer * n_inner;
  if (rows == 0) return SMAQ_OK;
  RowMap map{n_inner, s_outer, s_inner, out_outer ? out_outer : n_inner};
  hipStream_t st = (hipStream_t)stream;
  if (encode_blockvq_mfma_supported(n_blocks, block_dim, n_centroids, k, kdtype, s_outer, s_inner))
    return launch_encode_blockvq_mfma(kdtype, k, map, rows, n_blocks, E_blocks, centroids,
                                      (uint8_t*)idx_out, tie_count, st);
  const size_t lds = (size_t)n_blocks * n_centroids * sizeof(float);
  const unsigned grid = (unsigned)((rows + kVqThreads - 1) / kVqThreads);
  switch (kdtype) {
    case SMAQ_F32:
      hipLaunchKernelGGL(encode_blockvq_kernel<float>, dim3(grid), dim3(kVqThreads), lds, st,
                         (const float*)k, map, rows, n_blocks, block_dim, n_centroids, E_blocks,
                         centroids, (uint8_t*)idx_out, tie_count);
      return launch_status("smaq_encode_blockvq");
    case SMAQ_F16:
      hipLaunchKernelGGL(encode_blockvq_kernel<_Float16>, dim3(grid), dim3(kVqThreads), lds, st,
                         (const _Float16*)k, map, rows, n_blocks, block_dim, n_centroids, E_blocks,
                         centroids, (uint8_t*)idx_out, tie_count);
      return launch_status("smaq_encode_blockvq");
    case SMAQ_BF16:
      hipLaunchKernelGGL(encode_blockvq_kernel<bf16>, dim3(grid), dim3(kVqThreads), lds, st,
                         (const bf16*)k, map, rows, n_blocks, block_dim, n_centroids, E_blocks,
                         centroids, (uint8_t*)idx_out, tie_count);
      return launch_status("smaq_encode_blockvq");
  }
  set_error("smaq_encode_blockvq: unsupported dtype %d", kdtype);
  return SMAQ_EUNSUPPORTED;
}

extern "C" int smaq_dequant_blockvq(const void* idx, long long rows, int n_blocks, int block_dim,
                                    int n_centroids, const float* decoded, float* out,
                                    void* stream) {
  SMAQ_REQUIRE(idx && decoded && out, "smaq_dequant_blockvq: null pointer");
  SMAQ_REQUIRE(n_blocks >= 1 && block_dim >= 1 && n_centroids >= 1 && n_centroids <= 256,
               "smaq_dequant_blockvq: bad codebook shape");
  if (rows <= 0) return SMAQ_OK;
  const int64_t n = (int64_t)rows * n_blocks * block_dim;
  hipLaunchKernelGGL(dequant_blockvq_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)idx, (int64_t)rows, n_blocks, block_dim,
                     n_centroids, decoded, out);
  return launch_status("smaq_dequant_blockvq");
}
