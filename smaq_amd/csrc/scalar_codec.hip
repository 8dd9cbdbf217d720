// Scalar key codec: SMAQ metric encoder (and RotationAdapter variant), the row
// transform used by rotate_query / dequantize, the dequantiser and the
// score kernel.
//
// Bit-exactness of the encoder against torch-CPU (pinned by probes on the
// reference's torch build):
//  * ||k|| (fp32, bf16): 8 partial sums, element d into partial d % 8 with
//    FMA, partials added left to right, tail elements (past the last multiple
//    of 8 for fp32, of 16 for bf16) FMA'd into the total; fp16: one
//    sequential sum.  Then a correctly rounded sqrt, rounded to the key dtype.
//  * u = rnd(k / rnd(n + 1e-10)) in the key dtype.
//  * y_j = sum_d u_d * M[j][d] as one sequential FMA chain d = 0..D-1 starting
//    from 0 (the MKL sgemm micro-kernel order for >= 6 rows).
//  * code = number of boundaries strictly below y (searchsorted, left); NaN
//    maps to the top code.
#include <type_traits>

#include "encode_internal.h"
#include "rotate128.h"

namespace smaq {

constexpr int kEncRows = 8;     // rows per tile
constexpr int kEncThreads = 256;
constexpr int kMaxDim = 256;
constexpr int kMaxBounds = 255;

template <typename T>
__global__ __launch_bounds__(kEncThreads) void encode_scalar_kernel(
    const T* __restrict__ k, RowMap map, int64_t rows, int D, const float* __restrict__ Mt,
    const float* __restrict__ coord_scales, const float* __restrict__ bounds_g, int nb, int bits,
    uint8_t* __restrict__ codes_out, T* __restrict__ norms_out, unsigned long long* tie_count) {
  __shared__ float xs[kEncRows][kMaxDim];
  __shared__ float us[kEncRows][kMaxDim];
  __shared__ uint8_t cs[kEncRows][kMaxDim];
  __shared__ float part[kEncRows][8];
  __shared__ float nprime[kEncRows];
  __shared__ float bounds[kMaxBounds];

  const int tid = threadIdx.x;
  for (int i = tid; i < nb; i += kEncThreads) bounds[i] = bounds_g[i];
  // torch-CPU norm order: fp32 and bf16 take the vectorised last-dim path
  // (8 FMA partials), fp16 the generic sequential reduction
  constexpr bool kSequentialNorm = sizeof(T) == 2 && !std::is_same<T, bf16>::value;
  const int vec = (sizeof(T) == 4) ? 8 : 16;
  const int main_end = D - D % vec;
  const int vpb = (8 / bits) > 1 ? 8 / bits : 1;
  const int P = (D + vpb - 1) / vpb;
  const int row_sets = kEncThreads / D;  // D <= 256
  unsigned ties = 0;

  for (int64_t tile = blockIdx.x; tile * kEncRows < rows; tile += gridDim.x) {
    const int64_t r0 = tile * kEncRows;
    const int nr = (int)min((int64_t)kEncRows, rows - r0);
    for (int i = tid; i < nr * D; i += kEncThreads) {
      const int r = i / D, d = i - r * D;
      xs[r][d] = Num<T>::to_f(k[map.offset(r0 + r) + d]);
    }
    __syncthreads();
    if (kSequentialNorm) {
      // fp16: torch's generic reduction, one sequential sum (products exact)
      if (tid < nr) {
        float a = 0.0f;
        for (int d = 0; d < D; ++d) a = fmaf(xs[tid][d], xs[tid][d], a);
        part[tid][0] = a;
      }
    } else if (tid < nr * 8) {
      const int r = tid >> 3, l = tid & 7;
      float a = 0.0f;
      for (int d = l; d < main_end; d += 8) a = fmaf(xs[r][d], xs[r][d], a);
      part[r][l] = a;
    }
    __syncthreads();
    if (tid < nr) {
      const int r = tid;
      float b = part[r][0];
      if (!kSequentialNorm) {
        for (int l = 1; l < 8; ++l) b = b + part[r][l];
        for (int d = main_end; d < D; ++d) b = fmaf(xs[r][d], xs[r][d], b);
      }
      const float n = Num<T>::round(sqrtf(b));
      norms_out[map.out_row(r0 + r)] = Num<T>::from_f(n);
      nprime[r] = Num<T>::round(n + 1e-10f);
    }
    __syncthreads();
    for (int i = tid; i < nr * D; i += kEncThreads) {
      const int r = i / D, d = i - r * D;
      us[r][d] = Num<T>::round(xs[r][d] / nprime[r]);
    }
    __syncthreads();
    if (tid < row_sets * D) {
      const int j = tid % D;
      const int rs = tid / D;
      float acc[kEncRows];
#pragma unroll
      for (int q = 0; q < kEncRows; ++q) acc[q] = 0.0f;
      for (int d = 0; d < D; ++d) {
        const float m = Mt[(int64_t)d * D + j];
#pragma unroll
        for (int q = 0; q < kEncRows; ++q) {
          const int r = rs + q * row_sets;
          if (q * row_sets < kEncRows && r < nr) acc[q] = fmaf(us[r][d], m, acc[q]);
        }
      }
      const float cscale = coord_scales ? coord_scales[j] : 1.0f;
#pragma unroll
      for (int q = 0; q < kEncRows; ++q) {
        const int r = rs + q * row_sets;
        if (q * row_sets < kEncRows && r < nr) {
          const float y = coord_scales ? acc[q] * cscale : acc[q];
          cs[r][j] = (uint8_t)count_below(bounds, nb, y, &ties);
        }
      }
    }
    __syncthreads();
    for (int i = tid; i < nr * P; i += kEncThreads) {
      const int r = i / P, p = i - r * P;
      uint32_t byte = 0;
      for (int e = 0; e < vpb; ++e) {
        const int d = p * vpb + e;
        if (d < D) byte += (uint32_t)cs[r][d] << (e * bits);
      }
      codes_out[map.out_row(r0 + r) * P + p] = (uint8_t)byte;
    }
    __syncthreads();
  }
  add_count(tie_count, ties);
}

// out[r][j] = (sum_d x[r][d] * Mt[d][j]) [* s[j]], one sequential fmaf chain
// over d per output.  A block holds
// kRotRows rows in LDS and one thread per column j; each Mt element loaded
// feeds kRotRows independent chains.
constexpr int kRotRows = 8;

// The same product for head_dim 128: rotate128_block (rotate128.h), one
// memory round trip for the matrix and a fixed summation tree per output.
template <int ROWS>
__global__ __launch_bounds__(256) void rotate_rows128_kernel(const void* __restrict__ x, int xdtype, int64_t rows,
                                                             const float* __restrict__ Mt,
                                                             const float* __restrict__ s,
                                                             float* __restrict__ out) {
  __shared__ Rot128Lds<ROWS> lds;
  rotate128_block<ROWS>(lds, x, xdtype, rows, Mt, s, out, blockIdx.x, threadIdx.x);
}

template <typename T>
__global__ __launch_bounds__(1024) void rotate_rows_kernel(const T* __restrict__ x, int64_t rows,
                                                           int D, const float* __restrict__ Mt,
                                                           const float* __restrict__ s,
                                                           float* __restrict__ out) {
  extern __shared__ float xs[];  // [kRotRows][D]
  const int j = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * kRotRows;
  const int nr = (int)min((int64_t)kRotRows, rows - r0);
  for (int i = 0; i < kRotRows; ++i)
    xs[i * D + j] = i < nr ? Num<T>::to_f(x[(r0 + i) * D + j]) : 0.0f;
  __syncthreads();
  float acc[kRotRows];
#pragma unroll
  for (int i = 0; i < kRotRows; ++i) acc[i] = 0.0f;
#pragma unroll 4
  for (int d = 0; d < D; ++d) {
    const float m = Mt[(int64_t)d * D + j];
#pragma unroll
    for (int i = 0; i < kRotRows; ++i) acc[i] = fmaf(xs[i * D + d], m, acc[i]);
  }
  const float sj = s ? s[j] : 1.0f;
  for (int i = 0; i < nr; ++i) out[(r0 + i) * D + j] = s ? acc[i] * sj : acc[i];
}

__device__ __forceinline__ uint32_t scalar_code(const uint8_t* row, int d, int bits, int vpb) {
  const uint32_t byte = row[d / vpb];
  return (byte >> ((d % vpb) * bits)) & ((1u << bits) - 1u);
}

template <typename TN, typename TO>
__global__ __launch_bounds__(256) void dequant_scalar_kernel(
    const uint8_t* __restrict__ codes, const TN* __restrict__ norms, int64_t rows, int D, int bits,
    const float* __restrict__ centroids, const float* __restrict__ inv_scales,
    const float* __restrict__ Mt, TO* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * D) return;
  const int64_t r = idx / D;
  const int j = (int)(idx - r * D);
  const int vpb = (8 / bits) > 1 ? 8 / bits : 1;
  const int P = (D + vpb - 1) / vpb;
  const uint8_t* cr = codes + r * P;
  float acc = 0.0f;
  for (int i = 0; i < D; ++i) {
    float yh = centroids[scalar_code(cr, i, bits, vpb)];
    if (inv_scales) yh = yh * inv_scales[i];
    acc = fmaf(yh, Mt[(int64_t)i * D + j], acc);
  }
  out[idx] = Num<TO>::from_f(acc * Num<TN>::to_f(norms[r]));
}

// out[b][r][t] = ((qrot[b][r] . c[code[b][t]]) * norm[b][t]) [* scale]
template <typename TN, typename TO>
__global__ __launch_bounds__(256) void scores_scalar_kernel(
    const float* __restrict__ qrot, int64_t nq, int64_t N, int D, const uint8_t* __restrict__ codes,
    int bits, const TN* __restrict__ norms, const float* __restrict__ centroids, int has_scale,
    float scale, TO* __restrict__ out) {
  __shared__ float lut[256];
  const int b = blockIdx.z;
  const int ncent = 1 << bits;
  for (int i = threadIdx.x; i < ncent; i += blockDim.x) lut[i] = centroids[i];
  __syncthreads();
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t r = blockIdx.y;
  if (t >= N) return;
  const int vpb = (8 / bits) > 1 ? 8 / bits : 1;
  const int P = (D + vpb - 1) / vpb;
  const uint8_t* cr = codes + ((int64_t)b * N + t) * P;
  const float* q = qrot + ((int64_t)b * nq + r) * D;
  float acc = 0.0f;
  for (int d = 0; d < D; ++d) acc = fmaf(q[d], lut[scalar_code(cr, d, bits, vpb)], acc);
  float s = acc * Num<TN>::to_f(norms[(int64_t)b * N + t]);
  if (has_scale) s = s * scale;
  out[((int64_t)b * nq + r) * N + t] = Num<TO>::from_f(s);
}

template <typename T>
static int launch_encode(const void* k, RowMap map, int64_t rows, int D, const float* Mt,
                         const float* cs, const float* bounds, int nb, int bits, void* codes,
                         void* norms, unsigned long long* ties, hipStream_t st) {
  const int64_t tiles = (rows + kEncRows - 1) / kEncRows;
  const int64_t grid = tiles < 8192 ? tiles : 8192;
  hipLaunchKernelGGL(encode_scalar_kernel<T>, dim3((unsigned)grid), dim3(kEncThreads), 0, st,
                     (const T*)k, map, rows, D, Mt, cs, bounds, nb, bits, (uint8_t*)codes,
                     (T*)norms, ties);
  return launch_status("smaq_encode_scalar");
}

template <typename TN, typename TO>
static int launch_dequant_s(const void* codes, const void* norms, int64_t rows, int D, int bits,
                            const float* c, const float* inv, const float* Mt, void* out,
                            hipStream_t st) {
  const int64_t n = rows * D;
  hipLaunchKernelGGL((dequant_scalar_kernel<TN, TO>), dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, st, (const uint8_t*)codes, (const TN*)norms, rows, D, bits, c, inv, Mt,
                     (TO*)out);
  return launch_status("smaq_dequant_scalar");
}

template <typename TN, typename TO>
static int launch_scores(const float* qrot, int64_t batch, int64_t nq, int64_t N, int D,
                         const void* codes, int bits, const void* norms, const float* c,
                         int has_scale, float scale, void* out, hipStream_t st) {
  dim3 grid((unsigned)((N + 255) / 256), (unsigned)nq, (unsigned)batch);
  hipLaunchKernelGGL((scores_scalar_kernel<TN, TO>), grid, dim3(256), 0, st, qrot, nq, N, D,
                     (const uint8_t*)codes, bits, (const TN*)norms, c, has_scale, scale, (TO*)out);
  return launch_status("smaq_scores_scalar");
}

// Dispatch helper over the three storage dtypes.
#define SMAQ_DISPATCH_DTYPE(code, T, ...)            \
  switch (code) {                                    \
    case SMAQ_F32: { using T = float; __VA_ARGS__ }  \
    case SMAQ_F16: { using T = _Float16; __VA_ARGS__ } \
    case SMAQ_BF16: { using T = bf16; __VA_ARGS__ }  \
    default: break;                                  \
  }

}  // namespace smaq

using namespace smaq;

extern "C" int smaq_encode_scalar(const void* k, int kdtype, long long n_outer, long long n_inner,
                                  long long s_outer, long long s_inner, long long out_outer, int D,
                                  const float* Mt,
                                  const float* coord_scales, const float* bounds, int n_bounds,
                                  int bits, void* codes_out, void* norms_out,
                                  unsigned long long* tie_count, void* stream) {
  SMAQ_REQUIRE(k && Mt && bounds && codes_out && norms_out, "smaq_encode_scalar: null pointer");
  SMAQ_REQUIRE(D > 0 && D <= kMaxDim, "smaq_encode_scalar: head_dim must be in [1, %d], got %d",
               kMaxDim, D);
  SMAQ_REQUIRE(bits >= 1 && bits <= 8, "smaq_encode_scalar: bits must be in [1, 8], got %d", bits);
  SMAQ_REQUIRE(n_bounds >= 0 && n_bounds <= kMaxBounds && n_bounds < 256,
               "smaq_encode_scalar: %d decision boundaries unsupported", n_bounds);
  SMAQ_REQUIRE(n_outer >= 0 && n_inner > 0, "smaq_encode_scalar: bad row shape");
  SMAQ_REQUIRE(out_outer == 0 || out_outer >= n_inner, "smaq_encode_scalar: output rows overlap "
               "(out_outer %lld < n_inner %lld)", out_outer, n_inner);
  const int64_t rows = (int64_t)n_outer * n_inner;
  if (rows == 0) return SMAQ_OK;
  RowMap map{n_inner, s_outer, s_inner, out_outer ? out_outer : n_inner};
  hipStream_t st = (hipStream_t)stream;
  if (encode_scalar_mfma_supported(D, bits, n_bounds, codes_out, k, kdtype, s_outer, s_inner))
    return launch_encode_scalar_mfma(kdtype, k, map, rows, Mt, coord_scales, bounds, n_bounds, bits,
                                     codes_out, norms_out, tie_count, st);
  SMAQ_DISPATCH_DTYPE(kdtype, T,
      return launch_encode<T>(k, map, rows, D, Mt, coord_scales, bounds, n_bounds, bits,
                              codes_out, norms_out, tie_count, st);)
  set_error("smaq_encode_scalar: unsupported dtype %d", kdtype);
  return SMAQ_EUNSUPPORTED;
}

extern "C" int smaq_rotate_rows(const void* x, int xdtype, long long rows, int D, const float* Mt,
                                const float* coord_scales, float* out, void* stream) {
  SMAQ_REQUIRE(x && Mt && out, "smaq_rotate_rows: null pointer");
  SMAQ_REQUIRE(D > 0, "smaq_rotate_rows: bad head_dim");
  if (rows <= 0) return SMAQ_OK;
  SMAQ_REQUIRE(D <= 1024, "smaq_rotate_rows: head_dim above 1024");
  const int64_t blocks = ((int64_t)rows + kRotRows - 1) / kRotRows;
  SMAQ_REQUIRE(blocks < (1ll << 31), "smaq_rotate_rows: too many rows");
  hipStream_t st = (hipStream_t)stream;
  if (D == 128 && ((uintptr_t)Mt & 15) == 0) {  // (16-byte loads of Mt)
    const int rpb = rows > kRot128ManyRows ? 8 : 4;
    SMAQ_REQUIRE((rows + rpb - 1) / rpb < (1ll << 31), "smaq_rotate_rows: too many rows");
    const dim3 grid((unsigned)((rows + rpb - 1) / rpb));
    if (xdtype != SMAQ_F32 && xdtype != SMAQ_F16 && xdtype != SMAQ_BF16) {
      set_error("smaq_rotate_rows: unsupported dtype %d", xdtype);
      return SMAQ_EUNSUPPORTED;
    }
    if (rpb == 8)
      hipLaunchKernelGGL(rotate_rows128_kernel<8>, grid, dim3(256), 0, st, x, xdtype, (int64_t)rows, Mt,
                         coord_scales, out);
    else
      hipLaunchKernelGGL(rotate_rows128_kernel<4>, grid, dim3(256), 0, st, x, xdtype, (int64_t)rows, Mt,
                         coord_scales, out);
    return launch_status("smaq_rotate_rows");
  }
  SMAQ_DISPATCH_DTYPE(xdtype, T,
      hipLaunchKernelGGL(rotate_rows_kernel<T>, dim3((unsigned)blocks), dim3(D),
                         (size_t)kRotRows * D * sizeof(float), st, (const T*)x, (int64_t)rows, D, Mt,
                         coord_scales, out);
      return launch_status("smaq_rotate_rows");)
  set_error("smaq_rotate_rows: unsupported dtype %d", xdtype);
  return SMAQ_EUNSUPPORTED;
}

extern "C" int smaq_dequant_scalar(const void* codes, const void* norms, int ndtype,
                                   long long rows, int D, int bits, const float* centroids,
                                   const float* inv_scales, const float* Mt, void* out, int odtype,
                                   void* stream) {
  SMAQ_REQUIRE(codes && norms && centroids && Mt && out, "smaq_dequant_scalar: null pointer");
  SMAQ_REQUIRE(D > 0 && bits >= 1 && bits <= 8, "smaq_dequant_scalar: bad shape");
  if (rows <= 0) return SMAQ_OK;
  hipStream_t st = (hipStream_t)stream;
  SMAQ_DISPATCH_DTYPE(ndtype, TN,
      SMAQ_DISPATCH_DTYPE(odtype, TO,
          return launch_dequant_s<TN, TO>(codes, norms, rows, D, bits, centroids, inv_scales, Mt,
                                          out, st);))
  set_error("smaq_dequant_scalar: unsupported dtypes %d/%d", ndtype, odtype);
  return SMAQ_EUNSUPPORTED;
}

extern "C" int smaq_scores_scalar(const float* qrot, long long batch, long long nq, long long N,
                                  int D, const void* codes, int bits, const void* norms, int ndtype,
                                  const float* centroids, int has_scale, float scale, void* out,
                                  int odtype, void* stream) {
  SMAQ_REQUIRE(qrot && codes && norms && centroids && out, "smaq_scores_scalar: null pointer");
  SMAQ_REQUIRE(D > 0 && bits >= 1 && bits <= 8, "smaq_scores_scalar: bad shape");
  SMAQ_REQUIRE(nq < 65536 && batch < 65536, "smaq_scores_scalar: too many query rows");
  if (batch <= 0 || nq <= 0 || N <= 0) return SMAQ_OK;
  hipStream_t st = (hipStream_t)stream;
  SMAQ_DISPATCH_DTYPE(ndtype, TN,
      SMAQ_DISPATCH_DTYPE(odtype, TO,
          return launch_scores<TN, TO>(qrot, batch, nq, N, D, codes, bits, norms, centroids,
                                       has_scale, scale, out, st);))
  set_error("smaq_scores_scalar: unsupported dtypes %d/%d", ndtype, odtype);
  return SMAQ_EUNSUPPORTED;
}
