// Value codec: groupwise asymmetric min/max quantisation (the value bit-packer)
// and its dequantiser.
//
// Bit-exactness: every elementwise op is rounded to the value dtype, as
// torch-CPU does for bf16/fp16 tensors (compute in fp32, round once, RNE):
//   range = rnd(max - min); scale = rnd(range / levels)  (true division)
//   scale = max(scale, rnd(1e-10))  -- clamp bound converted to the dtype
//   min / max propagate NaN (torch's reductions)
//   code  = clamp(rint(rnd(rnd(v - min) / scale)), 0, levels), NaN -> 0
#include <algorithm>
#include <type_traits>

#include "smaq_common.h"

namespace smaq {

// Group minimum / maximum as torch's min / max reductions: a NaN anywhere in
// the group is the result (v_minimum3_f32 / v_maximum3_f32 on gfx950).
__device__ __forceinline__ float nan_min(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float nan_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Codes stored per byte: 2-bit -> 4, 4-bit -> 2, other widths unpacked.
__host__ __device__ __forceinline__ int value_codes_per_byte(int bits) {
  return bits == 2 ? 4 : (bits == 4 ? 2 : 1);
}

template <typename T>
__global__ __launch_bounds__(256) void pack_values_kernel(
    const T* __restrict__ v, RowMap map, int64_t rows, int D, int bits, int group,
    int groups_per_thread, uint8_t* __restrict__ data, T* __restrict__ scales,
    T* __restrict__ zeros) {
  const int n_groups = D / group;
  const int units_per_row = n_groups / groups_per_thread;
  const int64_t unit = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (unit >= rows * units_per_row) return;
  const int64_t row = unit / units_per_row;
  const int g0 = (int)(unit - row * units_per_row) * groups_per_thread;
  const T* src = v + map.offset(row);
  const int64_t orow = map.out_row(row);
  const int vpb = value_codes_per_byte(bits);
  const int row_bytes = D / vpb;
  const float levels = (float)((1 << bits) - 1);
  const float min_scale = dtype_const<T>(1e-10f);

  uint32_t acc = 0;  // byte under construction
  int filled = 0;
  for (int g = g0; g < g0 + groups_per_thread; ++g) {
    const T* gp = src + (int64_t)g * group;
    float lo = Num<T>::to_f(gp[0]);
    float hi = lo;
    for (int e = 1; e < group; ++e) {
      const float x = Num<T>::to_f(gp[e]);
      lo = nan_min(lo, x);
      hi = nan_max(hi, x);
    }
    float sc = Num<T>::round(Num<T>::round(hi - lo) / levels);
    if (sc < min_scale) sc = min_scale;  // clamp(min=1e-10), NaN passes
    scales[orow * n_groups + g] = Num<T>::from_f(sc);
    zeros[orow * n_groups + g] = Num<T>::from_f(lo);
    for (int e = 0; e < group; ++e) {
      const float x = Num<T>::to_f(gp[e]);
      float q = round_half_even(Num<T>::round(Num<T>::round(x - lo) / sc));
      q = fminf(fmaxf(q, 0.0f), levels);
      const uint32_t code = (q == q) ? (uint32_t)q : 0u;  // NaN -> 0
      acc |= code << (filled * bits);
      if (++filled == vpb) {
        const int d = g * group + e;
        data[orow * row_bytes + d / vpb] = (uint8_t)acc;
        acc = 0;
        filled = 0;
      }
    }
  }
}

// Group size 32, 2- or 4-bit codes: one thread per (row, group) with 16-byte
// loads and one 8- / 16-byte store of the packed codes (same arithmetic as
// pack_values_kernel).
template <typename T, int BITS>
__global__ __launch_bounds__(256) void pack_values_g32_kernel(
    const T* __restrict__ v, RowMap map, int64_t rows, int n_groups, uint8_t* __restrict__ data,
    T* __restrict__ scales, T* __restrict__ zeros) {
  constexpr int kG = 32;
  constexpr int vpb = 8 / BITS;
  constexpr float levels = (float)((1 << BITS) - 1);
  const int64_t unit = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (unit >= rows * n_groups) return;
  const int64_t row = n_groups == 4 ? unit >> 2 : unit / n_groups;
  const int g = (int)(unit - row * n_groups);
  const T* gp = v + map.offset(row) + g * kG;
  const int64_t orow = map.out_row(row);
  const float min_scale = dtype_const<T>(1e-10f);

  float x[kG];
  constexpr int per16 = 16 / (int)sizeof(T);
#pragma unroll
  for (int i = 0; i < kG; i += per16) {
    const uint4 w = *(const uint4*)(gp + i);
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < per16; ++e) {
      if constexpr (sizeof(T) == 2)
        x[i + e] = Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(wd[e >> 1] >> (16 * (e & 1)))));
      else
        x[i + e] = __builtin_bit_cast(float, wd[e]);
    }
  }
  float lo = x[0], hi = x[0];
#pragma unroll
  for (int e = 1; e < kG; ++e) {
    lo = nan_min(lo, x[e]);
    hi = nan_max(hi, x[e]);
  }
  float sc = Num<T>::round(Num<T>::round(hi - lo) / levels);
  if (sc < min_scale) sc = min_scale;  // clamp(min=1e-10), NaN passes
  scales[orow * n_groups + g] = Num<T>::from_f(sc);
  zeros[orow * n_groups + g] = Num<T>::from_f(lo);
  uint32_t out[4] = {0u, 0u, 0u, 0u};
  if constexpr (std::is_same<T, bf16>::value) {
    // bf16: a / sc as a * RN(1 / sc), with the roundings to bf16 done by the
    // hardware conversion (RNE).  Same codes as the division: a and sc carry
    // 8-bit significands, so a / sc is never a bf16 rounding midpoint (that
    // needs a 9-bit numerator) and lies at least 2^-17 (relative) from every
    // midpoint, while a * RN(1 / sc) is within 2^-23 of it; both round to
    // the same bf16 value, hence the same code.  NaN and infinities give the
    // same NaN / 0 quotients as the division (inf * 0, x * 0).
    const float rs = 1.0f / sc;
#pragma unroll
    for (int e = 0; e < kG; ++e) {
      const float a = (float)(__bf16)(x[e] - lo);
      float q = round_half_even((float)(__bf16)(a * rs));
      q = fminf(fmaxf(q, 0.0f), levels);
      const uint32_t code = (q == q) ? (uint32_t)q : 0u;  // NaN -> 0
      out[e / (4 * vpb)] |= code << (BITS * (e % (4 * vpb)));
    }
  } else {
#pragma unroll
    for (int e = 0; e < kG; ++e) {
      float q = round_half_even(Num<T>::round(Num<T>::round(x[e] - lo) / sc));
      q = fminf(fmaxf(q, 0.0f), levels);
      const uint32_t code = (q == q) ? (uint32_t)q : 0u;  // NaN -> 0
      out[e / (4 * vpb)] |= code << (BITS * (e % (4 * vpb)));
    }
  }
  uint8_t* dst = data + orow * (n_groups * kG / vpb) + g * (kG / vpb);
  if constexpr (BITS == 2) *(uint2*)dst = uint2{out[0], out[1]};
  else *(uint4*)dst = uint4{out[0], out[1], out[2], out[3]};
}

template <typename T>
__global__ __launch_bounds__(256) void dequant_values_kernel(
    const uint8_t* __restrict__ data, const T* __restrict__ scales, const T* __restrict__ zeros,
    int64_t rows, int D, int bits, int group, float* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * D) return;
  const int64_t row = idx / D;
  const int d = (int)(idx - row * D);
  const int vpb = value_codes_per_byte(bits);
  const int row_bytes = D / vpb;
  const uint32_t byte = data[row * row_bytes + d / vpb];
  const uint32_t code = (vpb == 1) ? byte : (byte >> ((d % vpb) * bits)) & ((1u << bits) - 1u);
  const int n_groups = D / group;
  const float s = Num<T>::to_f(scales[row * n_groups + d / group]);
  const float z = Num<T>::to_f(zeros[row * n_groups + d / group]);
  out[idx] = (float)code * s + z;  // two roundings (fp-contract off), as torch
}

template <typename T>
static int launch_pack(const void* v, RowMap map, int64_t rows, int D, int bits, int group,
                       void* data, void* scales, void* zeros, hipStream_t stream) {
  const int64_t esz = sizeof(T);
  const bool aligned16 = ((uintptr_t)v % 16) == 0 && (map.s_outer * esz) % 16 == 0 &&
                         (map.s_inner * esz) % 16 == 0 && ((uintptr_t)data % 16) == 0;
  if (group == 32 && (bits == 2 || bits == 4) && aligned16) {
    const int n_groups = D / 32;
    const int64_t units = rows * n_groups;
    const unsigned blocks = (unsigned)((units + 255) / 256);
    if (bits == 2)
      hipLaunchKernelGGL((pack_values_g32_kernel<T, 2>), dim3(blocks), dim3(256), 0, stream, (const T*)v, map,
                         rows, n_groups, (uint8_t*)data, (T*)scales, (T*)zeros);
    else
      hipLaunchKernelGGL((pack_values_g32_kernel<T, 4>), dim3(blocks), dim3(256), 0, stream, (const T*)v, map,
                         rows, n_groups, (uint8_t*)data, (T*)scales, (T*)zeros);
    return launch_status("smaq_pack_values");
  }
  const int vpb = value_codes_per_byte(bits);
  const int gpt = (group % vpb == 0) ? 1 : D / group;  // bytes straddle groups
  const int64_t units = rows * ((D / group) / gpt);
  const int threads = 256;
  const int64_t blocks = (units + threads - 1) / threads;
  hipLaunchKernelGGL(pack_values_kernel<T>, dim3((unsigned)blocks), dim3(threads), 0, stream,
                     (const T*)v, map, rows, D, bits, group, gpt, (uint8_t*)data, (T*)scales,
                     (T*)zeros);
  return launch_status("smaq_pack_values");
}

template <typename T>
static int launch_dequant(const void* data, const void* scales, const void* zeros, int64_t rows,
                          int D, int bits, int group, float* out, hipStream_t stream) {
  const int64_t n = rows * D;
  const int threads = 256;
  hipLaunchKernelGGL(dequant_values_kernel<T>, dim3((unsigned)((n + threads - 1) / threads)),
                     dim3(threads), 0, stream, (const uint8_t*)data, (const T*)scales,
                     (const T*)zeros, rows, D, bits, group, out);
  return launch_status("smaq_dequant_values");
}


// ------------------------------------------------- weighted packed values --
// out[b][q][d] = sum_n w[b][q][n] * (code[b][n][d] * scale + zero): the
// compressed term of SMAQKVCache.attend, the dequantised values never
// written out.  A lane holds one 4-byte word of a value row (4 * VPB
// codes, all of one group); L = D / (4 VPB) lanes cover a row and a wave
// load covers 64 / L rows.  Workgroup (split s, batch b) sums its token range
// per lane, across the lanes of a column by exchanges and across its four
// waves through LDS, in a fixed order; the splits are summed in split order
// by a second launch.
constexpr int kAvThreads = 256;
constexpr int kAvQ = 4;         // query rows per pass over the tokens
constexpr int kAvMaxD = 512;

template <int VPB, typename T>
__global__ __launch_bounds__(kAvThreads) void apply_values_kernel(
    const float* __restrict__ w, int64_t w_bstride, int64_t w_qstride, int nq, int64_t N, int D,
    const uint8_t* __restrict__ data, int64_t d_bstride, const T* __restrict__ scales,
    const T* __restrict__ zeros, int64_t s_bstride, int group, int64_t split_len, float* __restrict__ part,
    int64_t part_split) {
  constexpr int DPL = 4 * VPB;  // codes per lane
  constexpr int BITS = VPB == 4 ? 2 : (VPB == 2 ? 4 : 8);
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  __shared__ float red[4][kAvQ][kAvMaxD];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int s = blockIdx.x, b = blockIdx.y;
  const int L = D / DPL, tpw = 64 / L;
  const int dl = lane & (L - 1), tl = lane / L;
  const int d0 = dl * DPL;
  const int row_bytes = D / VPB, ng = D / group;
  const int64_t t0 = (int64_t)s * split_len;
  const int64_t t1 = min(N, t0 + split_len);
  const uint8_t* dcol = data + (int64_t)b * d_bstride + 4 * dl;
  const T* scol = scales + (int64_t)b * s_bstride + d0 / group;
  const T* zcol = zeros + (int64_t)b * s_bstride + d0 / group;
  const float* wb = w + (int64_t)b * w_bstride;
  float* pout = part + (int64_t)s * part_split + (int64_t)b * nq * D;
  for (int q0 = 0; q0 < nq; q0 += kAvQ) {
    const int nqq = min(kAvQ, nq - q0);
    float acc[kAvQ][DPL];
#pragma unroll
    for (int q = 0; q < kAvQ; ++q)
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[q][e] = 0.0f;
#pragma unroll 2
    for (int64_t t = t0 + (int64_t)wv * tpw + tl; t < t1; t += 4 * tpw) {
      const uint32_t word = *(const uint32_t*)(dcol + t * row_bytes);
      const float sc = Num<T>::to_f(scol[t * ng]);
      const float z = Num<T>::to_f(zcol[t * ng]);
      float v[DPL];
#pragma unroll
      for (int e = 0; e < DPL; ++e) v[e] = (float)((word >> (BITS * e)) & MASK) * sc + z;  // fp-contract off
#pragma unroll
      for (int q = 0; q < kAvQ; ++q) {
        if (q < nqq) {
          const float wq = wb[(int64_t)(q0 + q) * w_qstride + t];
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[q][e] = __builtin_fmaf(wq, v[e], acc[q][e]);
        }
      }
    }
    // the rows of a wave load share no column: sum the lanes of a column
    for (int off = L; off < 64; off <<= 1)
#pragma unroll
      for (int q = 0; q < kAvQ; ++q)
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[q][e] += __shfl_xor(acc[q][e], off, 64);
    if (tl == 0)
#pragma unroll
      for (int q = 0; q < kAvQ; ++q)
#pragma unroll
        for (int e = 0; e < DPL; ++e) red[wv][q][d0 + e] = acc[q][e];
    __syncthreads();
    for (int i = tid; i < nqq * D; i += kAvThreads) {
      const int q = i / D, d = i - q * D;
      pout[(int64_t)(q0 + q) * D + d] = (red[0][q][d] + red[1][q][d]) + (red[2][q][d] + red[3][q][d]);
    }
    __syncthreads();
  }
}

// out[i] = sum over splits, in split order
__global__ __launch_bounds__(256) void apply_values_reduce_kernel(const float* __restrict__ part, int n_splits,
                                                                  int64_t total, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  float acc = part[i];
  for (int k = 1; k < n_splits; ++k) acc += part[(int64_t)k * total + i];
  out[i] = acc;
}

// token splits of a launch: at least 512 tokens each, about 2048 workgroups
static int64_t apply_values_splits(long long batch, long long N) {
  const int64_t by_len = std::max<int64_t>(1, (N + 511) / 512);
  const int64_t by_grid = std::max<int64_t>(1, (2048 + batch - 1) / std::max<long long>(1, batch));
  return std::min<int64_t>(std::min(by_len, by_grid), 65535);
}

}  // namespace smaq

using namespace smaq;

extern "C" int smaq_pack_values(const void* v, int vdtype, long long n_outer, long long n_inner,
                                long long s_outer, long long s_inner, long long out_outer, int D,
                                int bits, int group, void* data_out, void* scales_out, void* zeros_out,
                                void* stream) {
  SMAQ_REQUIRE(v && data_out && scales_out && zeros_out, "smaq_pack_values: null pointer");
  SMAQ_REQUIRE(D > 0 && group > 0 && D % group == 0,
               "head_dim %d must be divisible by group_size %d", D, group);
  SMAQ_REQUIRE(bits >= 1 && bits <= 8, "smaq_pack_values: bits must be in [1, 8], got %d", bits);
  SMAQ_REQUIRE(D % value_codes_per_byte(bits) == 0,
               "head_dim %d must be divisible by %d for %d-bit packing", D,
               value_codes_per_byte(bits), bits);
  SMAQ_REQUIRE(n_outer >= 0 && n_inner > 0, "smaq_pack_values: bad row shape");
  const int64_t rows = (int64_t)n_outer * n_inner;
  if (rows == 0) return SMAQ_OK;
  SMAQ_REQUIRE(rows * (D / group) < (1ll << 40), "smaq_pack_values: too many rows");
  SMAQ_REQUIRE(out_outer == 0 || out_outer >= n_inner, "smaq_pack_values: output rows overlap "
               "(out_outer %lld < n_inner %lld)", out_outer, n_inner);
  RowMap map{n_inner, s_outer, s_inner, out_outer ? out_outer : n_inner};
  hipStream_t st = (hipStream_t)stream;
  switch (vdtype) {
    case SMAQ_F32: return launch_pack<float>(v, map, rows, D, bits, group, data_out, scales_out, zeros_out, st);
    case SMAQ_F16: return launch_pack<_Float16>(v, map, rows, D, bits, group, data_out, scales_out, zeros_out, st);
    case SMAQ_BF16: return launch_pack<bf16>(v, map, rows, D, bits, group, data_out, scales_out, zeros_out, st);
  }
  set_error("smaq_pack_values: unsupported dtype %d", vdtype);
  return SMAQ_EUNSUPPORTED;
}

extern "C" int smaq_dequant_values(const void* data, const void* scales, const void* zeros,
                                   int sdtype, long long rows, int D, int bits, int group,
                                   float* out, void* stream) {
  SMAQ_REQUIRE(data && scales && zeros && out, "smaq_dequant_values: null pointer");
  SMAQ_REQUIRE(D > 0 && group > 0 && D % group == 0,
               "head_dim %d must be divisible by group_size %d", D, group);
  SMAQ_REQUIRE(bits >= 1 && bits <= 8, "smaq_dequant_values: bits must be in [1, 8]");
  SMAQ_REQUIRE(D % value_codes_per_byte(bits) == 0, "smaq_dequant_values: bad packing");
  if (rows <= 0) return SMAQ_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (sdtype) {
    case SMAQ_F32: return launch_dequant<float>(data, scales, zeros, rows, D, bits, group, out, st);
    case SMAQ_F16: return launch_dequant<_Float16>(data, scales, zeros, rows, D, bits, group, out, st);
    case SMAQ_BF16: return launch_dequant<bf16>(data, scales, zeros, rows, D, bits, group, out, st);
  }
  set_error("smaq_dequant_values: unsupported dtype %d", sdtype);
  return SMAQ_EUNSUPPORTED;
}

extern "C" long long smaq_apply_values_workspace_bytes(long long batch, long long nq, long long N, int D) {
  if (batch <= 0 || nq <= 0 || D <= 0) return 0;
  const int64_t n_splits = apply_values_splits(batch, N);
  return n_splits > 1 ? (long long)(n_splits * batch * nq * D * (int64_t)sizeof(float)) : 0;
}

extern "C" int smaq_apply_values(const float* w, long long w_bstride, long long w_qstride, long long batch,
                                 long long nq, long long N, int D, const void* data, long long d_bstride, int bits,
                                 int group, const void* scales, const void* zeros, long long s_bstride, int sdtype,
                                 float* out, void* workspace, long long workspace_bytes, void* stream) {
  SMAQ_REQUIRE(batch >= 0 && nq >= 0 && N >= 0, "smaq_apply_values: negative shape");
  if (batch == 0 || nq == 0) return SMAQ_OK;
  SMAQ_REQUIRE(out && (N == 0 || (w && data && scales && zeros)), "smaq_apply_values: null pointer");
  SMAQ_REQUIRE(batch <= 65535, "smaq_apply_values: batch %lld above 65535", batch);
  SMAQ_REQUIRE(bits >= 1 && bits <= 8, "smaq_apply_values: bits must be in [1, 8], got %d", bits);
  SMAQ_REQUIRE(D > 0 && D <= kAvMaxD && group > 0 && D % group == 0,
               "smaq_apply_values: head_dim %d (at most %d) must be divisible by group_size %d", D, kAvMaxD, group);
  const int vpb = value_codes_per_byte(bits), dpl = 4 * vpb;
  const int lanes = D / dpl;
  if (!(D % dpl == 0 && lanes <= 64 && (lanes & (lanes - 1)) == 0 && group % dpl == 0)) {
    set_error("smaq_apply_values: unsupported layout (head_dim %d, %d-bit codes, group %d): a value row must be "
              "a power-of-two number (<= 64) of 4-byte words each inside one group",
              D, bits, group);
    return SMAQ_EUNSUPPORTED;
  }
  SMAQ_REQUIRE(((uintptr_t)data % 4) == 0 && d_bstride % 4 == 0, "smaq_apply_values: value rows must be 4-byte aligned");
  const int64_t n_splits = apply_values_splits(batch, N);
  const int64_t split_len = std::max<int64_t>(1, (N + n_splits - 1) / n_splits);
  const int64_t total = batch * nq * (int64_t)D;
  float* part = out;
  if (n_splits > 1) {
    SMAQ_REQUIRE(workspace && workspace_bytes >= n_splits * total * (int64_t)sizeof(float),
                 "smaq_apply_values: workspace of %lld bytes below %lld", workspace_bytes,
                 (long long)(n_splits * total * (int64_t)sizeof(float)));
    part = (float*)workspace;
  }
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)n_splits, (unsigned)batch);
#define SMAQ_AV(VPB, T)                                                                                           \
  hipLaunchKernelGGL((apply_values_kernel<VPB, T>), grid, dim3(kAvThreads), 0, st, w, (int64_t)w_bstride,          \
                     (int64_t)w_qstride, (int)nq, (int64_t)N, D, (const uint8_t*)data, (int64_t)d_bstride,           \
                     (const T*)scales, (const T*)zeros, (int64_t)s_bstride, group, split_len, part, total)
#define SMAQ_AV_T(VPB)                                      \
  switch (sdtype) {                                         \
    case SMAQ_F32: SMAQ_AV(VPB, float); break;              \
    case SMAQ_F16: SMAQ_AV(VPB, _Float16); break;           \
    case SMAQ_BF16: SMAQ_AV(VPB, bf16); break;              \
    default: set_error("smaq_apply_values: unsupported dtype %d", sdtype); return SMAQ_EUNSUPPORTED; \
  }
  if (vpb == 4) {
    SMAQ_AV_T(4)
  } else if (vpb == 2) {
    SMAQ_AV_T(2)
  } else {
    SMAQ_AV_T(1)
  }
#undef SMAQ_AV_T
#undef SMAQ_AV
  int rc = launch_status("smaq_apply_values");
  if (rc != SMAQ_OK || n_splits == 1) return rc;
  hipLaunchKernelGGL(apply_values_reduce_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, part,
                     (int)n_splits, total, out);
  return launch_status("smaq_apply_values(reduce)");
}
