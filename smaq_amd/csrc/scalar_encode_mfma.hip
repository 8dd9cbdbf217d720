// Scalar key encoder on the gfx950 matrix cores (D = 128, 2/3/4-bit codes).
//
// Same results as encode_scalar_kernel (scalar_codec.hip), which reproduces
// the reference's torch-CPU arithmetic bit for bit: norm with 8 FMA partials
// (fp16: one sequential sum), u = rnd(k / rnd(n + 1e-10)), y_j = one
// sequential FMA chain over d, code = #boundaries below y.  Here the chain is
// replaced by v_mfma_f32_16x16x32_bf16 over exact bf16 splits of u and of the
// matrix (u: 1, 2 or 3 parts for bf16, fp16, fp32 keys; matrix: 3 parts), so
// every product is exact and only the accumulation differs.
//
// Decision margin.  Let S = sum_d |u_d m_dj| (from one more MFMA of |u| and
// the |M| hi parts; x 1.03 covers those truncated parts) and u = 2^-24.  The
// code must be the one the reference's chain y_c gives, and the matrix-core
// value y_m and y_c both differ from the exact sum y:
//   * y_c: 128 fmaf steps, each one rounding of a partial sum whose
//     magnitude is at most S, so |y_c - y| <= 128 u S;
//   * y_m: a chain of N MFMAs per output (N = 12, 20, 24 for bf16, fp16,
//     fp32 keys: 4 K-steps x the part products kept), each adding exact
//     products to its accumulator with at most two roundings of a value
//     bounded by S (the largest error measured on gfx950 over 12 chained
//     MFMAs was 10.4 u S, below the one-rounding-per-MFMA 12 u S), so the
//     accumulation adds at most 2 N u S;
//   * the part products not formed (u part i x matrix part j with i + j >= 3;
//     truncated bf16 parts satisfy |p1| < 2^-7 |x|, |p2| < 2^-14 |x|) sum to
//     less than 2 * 2^-21 S = 16 u S for fp32 keys (pairs 1x2, 2x1, 2x2) and
//     2^-21 S = 8 u S for fp16 keys (pair 1x2); bf16 keys form every pair.
// Hence |y_m - y_c| <= (2 N + 128 + dropped) u S =: err.  A code is final when every
// boundary is farther than err plus the tie tolerance from y_m; otherwise y
// is recomputed with the exact sequential chain and counted as the reference
// does (including the tie counter).
//
// Tile: 64 rows per workgroup iteration, 4 waves; wave w owns output columns
// 32w .. 32w+31 and keeps its matrix parts in registers for the whole grid
// stride loop.
#include <type_traits>

#include "encode_internal.h"

namespace smaq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTR = 64;        // rows per tile
constexpr int kD = 128;        // head_dim served
constexpr int kXS = 132;       // floats per row of the fp32 tile
constexpr int kAR = 272;       // bytes per row of one bf16 A part (256 + 16 pad)
template <typename T> struct UParts { static constexpr int n = 3; };       // fp32
template <> struct UParts<bf16> { static constexpr int n = 1; };
template <> struct UParts<_Float16> { static constexpr int n = 2; };

// MFMAs chained into one output: 4 K-steps x the (u part, matrix part) pairs
// with up + ep < 3 (the smaller products are not formed; see kDropped)
template <int UP>
constexpr int kChainedMfma = 4 * (UP == 1 ? 3 : (UP == 2 ? 5 : 6));

// bound on the part products not formed, in units of 2^-24 S
template <int UP>
constexpr float kDropped = UP == 1 ? 0.0f : (UP == 2 ? 8.0f : 16.01f);

// |y_m - y_c| / S bound: two roundings per chained MFMA, the products not
// formed, one rounding per step of the reference's 128-step chain; x 1.03 for
// the truncated parts in S
template <int UP>
constexpr float kErr = (2.0f * kChainedMfma<UP> + kDropped<UP> + 128.0f) * 1.03f / 16777216.0f;

__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bfloat(uint32_t b) { return __builtin_bit_cast(float, b); }

// x = p0 + p1 + p2 exactly (truncated bf16 parts; normal range)
__device__ __forceinline__ void split_bf16(float x, uint32_t* p) {
  const uint32_t b0 = fbits(x) & 0xffff0000u;
  const float r1 = x - bfloat(b0);
  const uint32_t b1 = fbits(r1) & 0xffff0000u;
  const float r2 = r1 - bfloat(b1);
  p[0] = b0 >> 16;
  p[1] = b1 >> 16;
  p[2] = fbits(r2) >> 16;
}

// Eight consecutive storage-dtype values -> fp32 (16 or 32 bytes).
template <typename T>
__device__ __forceinline__ void load8f(const T* p, float* out) {
  if constexpr (sizeof(T) == 2) {
    const uint4 v = *(const uint4*)p;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(w[i >> 1] >> (16 * (i & 1)))));
  } else {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

template <typename T, int BITS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void encode_scalar_mfma_kernel(
    const T* __restrict__ k, RowMap map, int64_t rows, const float* __restrict__ Mt,
    const float* __restrict__ coord_scales, const float* __restrict__ bounds_g,
    uint8_t* __restrict__ codes_out, T* __restrict__ norms_out, unsigned long long* tie_count) {
  constexpr int UP = UParts<T>::n;
  constexpr int nb = (1 << BITS) - 1;  // decision boundaries
  __shared__ __attribute__((aligned(16))) float xs[kTR * kXS];          // x, then u (fp32)
  __shared__ __attribute__((aligned(16))) uint8_t ua[UP][kTR * kAR];    // u bf16 parts, MFMA A layout
  __shared__ uint8_t cs[kTR][kD];                                       // codes
  __shared__ float part[kTR][8];
  __shared__ float nprime[kTR];
  __shared__ float bounds[16];
  // guard[c] = (b_{c-1} + 1e-6 |b_{c-1}|, b_c - 1e-6 |b_c|): the boundaries
  // next to code c widened by the tie tolerance (+-inf past the ends)
  __shared__ __attribute__((aligned(8))) float2 guard[17];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int n = lane & 15, kg = lane >> 4;
  constexpr bool kSequentialNorm = sizeof(T) == 2 && !std::is_same<T, bf16>::value;

  if (tid < nb) bounds[tid] = bounds_g[tid];
  float bnd[nb];  // wave-uniform copies for the unrolled counts
#pragma unroll
  for (int i = 0; i < nb; ++i) bnd[i] = bounds_g[i];
  if (tid <= nb) {
    const float lo = tid > 0 ? bounds_g[tid - 1] : 0.0f, hi = tid < nb ? bounds_g[tid] : 0.0f;
    guard[tid] = float2{tid > 0 ? lo + 1e-6f * fabsf(lo) : -__builtin_inff(),
                        tid < nb ? hi - 1e-6f * fabsf(hi) : __builtin_inff()};
  }

  // matrix parts as B operands: column 32w + 16cb + n, k = 32ks + 8kg + e;
  // bs = |hi part| for the error bound
  u32x4 bm[2][4][3], bs[2][4];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int col = 32 * w + 16 * cb + n;
      uint32_t pw[3][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t lo[3], hi[3];
        split_bf16(Mt[(32 * ks + 8 * kg + 2 * i) * kD + col], lo);
        split_bf16(Mt[(32 * ks + 8 * kg + 2 * i + 1) * kD + col], hi);
#pragma unroll
        for (int p = 0; p < 3; ++p) pw[p][i] = lo[p] | (hi[p] << 16);
      }
#pragma unroll
      for (int p = 0; p < 3; ++p) bm[cb][ks][p] = u32x4{pw[p][0], pw[p][1], pw[p][2], pw[p][3]};
      bs[cb][ks] = bm[cb][ks][0] & 0x7fff7fffu;
    }
  __syncthreads();

  constexpr int vpb = 8 / BITS;       // 2 or 4 codes per byte (bits 3/4 or 2)
  constexpr int P = kD / vpb;         // bytes per row
  unsigned ties = 0;
  const int lr = tid >> 2, lq = tid & 3;  // loader / packer: row, quarter of the row

  for (int64_t tile = blockIdx.x; tile * kTR < rows; tile += gridDim.x) {
    const int64_t r0 = tile * kTR;
    const int nr = (int)min((int64_t)kTR, rows - r0);
    // -- x tile (fp32 in LDS); rows past the end read as zeros
    {
      float* xr = &xs[lr * kXS + 32 * lq];
      if (lr < nr) {
        const T* src = k + map.offset(r0 + lr) + 32 * lq;
#pragma unroll
        for (int i = 0; i < 32; i += 8) {
          float f[8];
          load8f<T>(src + i, f);
          *(float4*)(xr + i) = float4{f[0], f[1], f[2], f[3]};
          *(float4*)(xr + i + 4) = float4{f[4], f[5], f[6], f[7]};
        }
      } else {
#pragma unroll
        for (int i = 0; i < 32; i += 4) *(float4*)(xr + i) = float4{0.f, 0.f, 0.f, 0.f};
      }
    }
    __syncthreads();
    // -- ||x|| partials: torch-CPU order
    if (kSequentialNorm) {
      if (lq == 0) {
        float a = 0.0f;
        for (int d = 0; d < kD; ++d) a = fmaf(xs[lr * kXS + d], xs[lr * kXS + d], a);
        part[lr][0] = a;
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int l = 2 * lq + h;
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < kD / 8; ++i) a = fmaf(xs[lr * kXS + l + 8 * i], xs[lr * kXS + l + 8 * i], a);
        part[lr][l] = a;
      }
    }
    __syncthreads();
    if (tid < kTR) {
      float b = part[tid][0];
      if (!kSequentialNorm)
        for (int l = 1; l < 8; ++l) b = b + part[tid][l];
      const float nn = Num<T>::round(sqrtf(b));
      if (tid < nr) norms_out[map.out_row(r0 + tid)] = Num<T>::from_f(nn);
      nprime[tid] = Num<T>::round(nn + 1e-10f);
    }
    __syncthreads();
    // -- u = rnd(x / n') (fp32 copy for the exact recount) and its bf16 parts
    {
      // thread (lr, lq) takes the pairs d = 2lq + 8i, +1 (bank-spread LDS access)
      const float np = nprime[lr];
#pragma unroll 4
      for (int i = 0; i < 16; ++i) {
        const int d = 2 * lq + 8 * i;
        float2* xp = (float2*)&xs[lr * kXS + d];
        const float2 xv = *xp;
        const float u0 = Num<T>::round(xv.x / np), u1 = Num<T>::round(xv.y / np);
        *xp = float2{u0, u1};
        uint32_t p0[3], p1[3];
        split_bf16(u0, p0);
        split_bf16(u1, p1);
#pragma unroll
        for (int p = 0; p < UP; ++p) *(uint32_t*)&ua[p][lr * kAR + 2 * d] = p0[p] | (p1[p] << 16);
      }
    }
    __syncthreads();
    // -- y = u M^T and S = |u| |M| on the matrix cores (rows 16rb + 4kg + v,
    // columns 32w + 16cb + n), then codes.  Element e = 16cb + 4rb + v is
    // marked in `redo` when a boundary is within its error band.
    uint32_t redo = 0;
#pragma unroll 1
    for (int rb = 0; rb < 4; ++rb) {
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      f32x4 sac[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        u32x4 a[UP];
#pragma unroll
        for (int p = 0; p < UP; ++p) a[p] = *(const u32x4*)&ua[p][(16 * rb + n) * kAR + 2 * (32 * ks + 8 * kg)];
        const u32x4 aabs = a[0] & 0x7fff7fffu;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
          for (int up = 0; up < UP; ++up)
#pragma unroll
            for (int ep = 0; ep + up < 3; ++ep)
              acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  __builtin_bit_cast(bf16x8, a[up]), __builtin_bit_cast(bf16x8, bm[cb][ks][ep]), acc[cb], 0, 0, 0);
          sac[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, aabs), __builtin_bit_cast(bf16x8, bs[cb][ks]), sac[cb], 0, 0, 0);
        }
      }
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const int col = 32 * w + 16 * cb + n;
        const float cscale = coord_scales ? coord_scales[col] : 1.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = 16 * rb + 4 * kg + v;
          const float y = coord_scales ? acc[cb][v] * cscale : acc[cb][v];
          const float err = (coord_scales ? sac[cb][v] * fabsf(cscale) : sac[cb][v]) * kErr<UP>;
          // band: err + 1e-6 * (|y| + err) + 1e-12 (with the +-1e-6 |b| in guard[])
          const float wband = fmaf(1e-6f, fabsf(y), fmaf(err, 1.000001f, 1e-12f));
          int c = 0;
#pragma unroll
          for (int i = 0; i < nb; ++i) c += (bnd[i] < y) ? 1 : 0;
          const float2 gd = guard[c];
          const bool safe = (y - wband > gd.x) && (y + wband < gd.y);
          if (y != y) c = nb;  // NaN -> searchsorted returns len
          else if (!safe && row < nr) redo |= 1u << (16 * cb + 4 * rb + v);
          cs[row][col] = (uint8_t)c;
        }
      }
    }
    // -- exact recount: y_j as the reference's sequential FMA chain
    while (__any(redo != 0)) {
      if (redo != 0) {
        const int e = __builtin_ctz(redo);
        redo &= redo - 1u;
        const int cb = e >> 4, rb = (e >> 2) & 3, v = e & 3;
        const int row = 16 * rb + 4 * kg + v, col = 32 * w + 16 * cb + n;
        float y = 0.0f;
        for (int d0 = 0; d0 < kD; d0 += 16) {
          float m[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) m[i] = Mt[(d0 + i) * kD + col];
#pragma unroll
          for (int i = 0; i < 16; ++i) y = fmaf(xs[row * kXS + d0 + i], m[i], y);
        }
        if (coord_scales) y = y * coord_scales[col];
        cs[row][col] = (uint8_t)count_below(bounds, nb, y, &ties);
      }
    }
    __syncthreads();
    // -- pack: row lr, bytes lq * P/4 .. (P/4 per thread: 16 or 8)
    if (lr < nr) {
      // 32 codes (one per byte of cs) -> 32 / vpb packed bytes; each code
      // dword [c0 c1 c2 c3] folds into packed bytes with one dot product
      constexpr int nbytes = P / 4;
      const uint32_t* src = (const uint32_t*)&cs[lr][32 * lq];
      uint8_t* dst = codes_out + map.out_row(r0 + lr) * P + lq * nbytes;
      uint32_t wds[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t cw = src[q];
        if constexpr (vpb == 4) {  // one byte: c0 | c1 << 2 | c2 << 4 | c3 << 6
          wds[q >> 2] |= __builtin_amdgcn_udot4(cw, 0x40100401u, 0u, false) << (8 * (q & 3));
        } else {                   // two bytes: c0 | c1 << B, c2 | c3 << B
          const uint32_t b0 = __builtin_amdgcn_udot4(cw, (1u << BITS) << 8 | 1u, 0u, false);
          const uint32_t b1 = __builtin_amdgcn_udot4(cw, ((1u << BITS) << 24) | (1u << 16), 0u, false);
          wds[q >> 1] |= (b0 | (b1 << 8)) << (16 * (q & 1));
        }
      }
      if constexpr (nbytes == 16) *(uint4*)dst = uint4{wds[0], wds[1], wds[2], wds[3]};
      else *(uint2*)dst = uint2{wds[0], wds[1]};
    }
    __syncthreads();
  }
  add_count(tie_count, ties);
}

}  // namespace

bool encode_scalar_mfma_supported(int D, int bits, int nb, const void* codes_out, const void* k,
                                  int kdtype, long long s_outer, long long s_inner) {
  // rows are read in 16-byte pieces: row element offsets must keep that alignment
  const long long esz = kdtype == SMAQ_F32 ? 4 : 2;
  const bool aligned = ((uintptr_t)k % 16) == 0 && ((s_outer * esz) % 16) == 0 && ((s_inner * esz) % 16) == 0;
  return D == kD && (bits == 2 || bits == 3 || bits == 4) && nb == (1 << bits) - 1 &&
         ((uintptr_t)codes_out & 15) == 0 && aligned;
}

template <typename T>
static int launch_t(const void* k, RowMap map, int64_t rows, const float* Mt, const float* cs,
                    const float* bounds, int nb, int bits, void* codes, void* norms,
                    unsigned long long* ties, hipStream_t st) {
  const int64_t tiles = (rows + kTR - 1) / kTR;
  const int64_t grid = tiles < 1024 ? tiles : 1024;
  switch (bits) {
    case 2: hipLaunchKernelGGL((encode_scalar_mfma_kernel<T, 2>), dim3((unsigned)grid), dim3(256), 0, st,
                               (const T*)k, map, rows, Mt, cs, bounds, (uint8_t*)codes, (T*)norms, ties); break;
    case 3: hipLaunchKernelGGL((encode_scalar_mfma_kernel<T, 3>), dim3((unsigned)grid), dim3(256), 0, st,
                               (const T*)k, map, rows, Mt, cs, bounds, (uint8_t*)codes, (T*)norms, ties); break;
    default: hipLaunchKernelGGL((encode_scalar_mfma_kernel<T, 4>), dim3((unsigned)grid), dim3(256), 0, st,
                                (const T*)k, map, rows, Mt, cs, bounds, (uint8_t*)codes, (T*)norms, ties); break;
  }
  return launch_status("smaq_encode_scalar(mfma)");
}

int launch_encode_scalar_mfma(int kdtype, const void* k, RowMap map, int64_t rows, const float* Mt,
                              const float* cs, const float* bounds, int nb, int bits, void* codes,
                              void* norms, unsigned long long* ties, hipStream_t st) {
  switch (kdtype) {
    case SMAQ_F32: return launch_t<float>(k, map, rows, Mt, cs, bounds, nb, bits, codes, norms, ties, st);
    case SMAQ_F16: return launch_t<_Float16>(k, map, rows, Mt, cs, bounds, nb, bits, codes, norms, ties, st);
    case SMAQ_BF16: return launch_t<bf16>(k, map, rows, Mt, cs, bounds, nb, bits, codes, norms, ties, st);
    default: break;
  }
  set_error("smaq_encode_scalar: unsupported dtype %d", kdtype);
  return SMAQ_EUNSUPPORTED;
}

}  // namespace smaq
