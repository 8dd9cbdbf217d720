// Chunked-prefill attention on the gfx950 matrix cores (head_dim 128).
//
// Prefill is compute-bound (every key tile serves many query rows), so the
// packed cache is first decoded once per part into f16 tile images in the
// workspace (the dequantisation the generic kernels do per query tile):
//   keys   K~[t][d]  = lut[code] * norm (scalar) or decoded centroid (block-VQ);
//                      the recent window's exact keys; hi = f16(x) and
//                      lo = f16(x - hi), ~22 significant bits
//   values V^[d][t]  = code * scale + zero (fp32, as the reference's
//                      dequantize_values), or the recent window's values,
//                      stored dimension-major as x = v * 2^-8 split the same
//                      way: the hi plane in the image, the lo plane in a
//                      second array
// The 2^-8 keeps values up to 1.6e7 inside f16's range (bf16 inputs reach
// far beyond f16's 65504); the kernel multiplies its sums by 2^8 back.
//
// Precision.  The weights p always enter PV as ph = f16(p) and
// pl = f16(p - ph).  A key range whose tiles all hold values the hi plane
// alone represents to within kRepBudget runs the cheap form vh.(ph + pl);
// an output o = sum w v (w = p / l) then moves by at most
// sum w |v - 2^8 vh| <= kRepBudget from the fp32 path, whatever the weights
// (2^-11 |v| per value: every |v| < 8 passes).  The pre-pass records each
// tile's largest such error; a workgroup whose key range holds a tile above
// the budget (or a value that is not finite) runs the precise form
// vh.(ph + pl) + vl.ph instead, ~22 significant bits at any value scale.
// The budget is the 2e-3 absolute tolerance of the attention outputs less
// what the ~22-bit scores and fp32 sums add (~1e-5 at the c4 shape).
//
// Tile image (64 tokens of one (sequence, KV head), 48 KB, exactly what the
// kernel holds in LDS):
//   [K hi | K lo]  64 key rows x 256 B; 16-byte unit u (dims 8u..8u+7) of
//                  row r sits at unit u ^ (r & 15)
//   [V hi]         128 dim rows x 128 B; unit u = 4 st + kg holds keys
//                  32 st + 4 kg + {0..3} and 32 st + 16 + 4 kg + {0..3} (the
//                  eight k-elements one lane feeds the PV matrix op), at unit
//                  u ^ ((d >> 1) & 7) of row d
//   (V lo, 16 KB, in the same layout as V hi, in the value-lo array)
// The XOR placements make the kernel's 16-byte operand reads of 16
// consecutive lanes hit 16 distinct bank quads (64 banks), and the kernel
// copies a tile with plain contiguous direct-to-LDS loads.
//
// The attention kernel then works in the transposed orientation, which fits
// the MFMA register layouts without any transpose:
//   S^T[key][query] = K~ . Q^T   v_mfma_f32_16x16x32_f16, A = key rows (LDS),
//                                B = query columns (registers, hi/lo split)
//   softmax per query column (keys = C rows: 4 per lane, 4 lane groups)
//   O^T[dim][query] += V^T . P^T  A = value rows (dimension-major tile),
//                                B = P^T straight from the S^T accumulators
// with qh.kh + qh.kl + ql.kh (ql.kh skipped where every query lo part is
// zero).  Each workgroup (8 waves x 32 query rows) streams the 64-key tiles
// of one (sequence, query head, key split), copied straight into LDS
// (global_load_lds_dwordx4) one tile ahead.  The cheap form keeps a ring of
// three 48 KB images and the second wave of every SIMD runs its PV one tile
// late, so that the two waves' matrix and vector phases interleave; the
// precise form double-buffers 64 KB images (the value-lo plane appended)
// with every wave in step.  The kernel writes the same (m, l, o) partials as
// the other attention kernels; attn_combine_kernel merges splits and the
// history / recent parts.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "attention_internal.h"

namespace smaq {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kKT = 64;           // keys per tile
constexpr int kQW = 32;           // query rows per wave
constexpr int kPW = 8;            // waves per workgroup
constexpr int kPT = 64 * kPW;     // threads per workgroup
constexpr int kQB = kPW * kQW;    // query rows per workgroup
constexpr int kImg = 8192 * kPrefillPlanes;  // halves per tile image (48 KB)
constexpr int kImgKL = 8192, kImgV = 16384;   // part offsets (halves)
constexpr int kImgP = kImg + kPrefillLoHalves; // halves per LDS buffer of the precise form (64 KB)
constexpr float kLog2e = 1.4426950408889634f;
// 16-byte direct-to-LDS loads per thread and tile: the image, the value-lo plane
constexpr int kCopyLoads = kImg * 2 / 16 / kPT;
constexpr int kCopyLoadsLo = kPrefillLoHalves * 2 / 16 / kPT;
static_assert(kCopyLoads == 6 && kImg * 2 == kCopyLoads * 16 * kPT, "tile copy: whole 16-byte loads per thread");
static_assert(kCopyLoadsLo == 2 && kPrefillLoHalves * 2 == kCopyLoadsLo * 16 * kPT, "lo-plane copy: whole loads");
static_assert(2 * kImgP <= 3 * kImg, "the precise form's two buffers fit the cheap form's ring");
constexpr float kLazy = 8.0f;     // softmax reference max raised by > 2^8 only
// values enter the tile images as v * 2^-8 (top of this file)
constexpr float kValIn = 0x1p-8f, kValOut = 0x1p8f;
// largest representation error a key range may leave to the cheap form
constexpr float kRepBudget = 1.96e-3f;

// halves offset of 16-byte unit u of key row r / value row d in a tile image part
__device__ __forceinline__ int kimg_off(int r, int u) { return r * 128 + 8 * (u ^ (r & 15)); }
__device__ __forceinline__ int vimg_off(int d, int u) { return d * 64 + 8 * (u ^ ((d >> 1) & 7)); }
// key (0..63) held by element e (0..7) of value unit u (0..7)
__device__ __forceinline__ int vunit_key(int u, int e) { return 32 * (u >> 2) + 4 * (u & 3) + (e & 3) + 16 * (e >> 2); }

__device__ __forceinline__ uint32_t h16(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }

__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// split_f16 of two numbers, packed: hi = RN(x) of both in one packed
// convert; x - hi (exact in fp32) by two mixed-precision FMAs x * one - hi
// reading hi as f16, and the lo pair in one more packed convert.  `one` is
// 1.0 kept opaque to the compiler, so that the FMA is not folded into an
// add (which has no mixed-precision form).
__device__ __forceinline__ void split2_f16(float x0, float x1, float one, uint32_t& hi, uint32_t& lo) {
  const f16x2 h = __builtin_convertvector((f32x2){x0, x1}, f16x2);
  const f32x2 r = {__builtin_fmaf(one, x0, -(float)h[0]), __builtin_fmaf(one, x1, -(float)h[1])};
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, f16x2));
}

// two numbers rounded to f16 in one packed convert
__device__ __forceinline__ uint32_t pack2_f16(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x0, x1}, f16x2));
}

__device__ __forceinline__ int exponent_of(float x) {
  if (!(x > 0.0f)) return 0;
  int e;
  frexpf(x, &e);
  return e - 1;
}

// ------------------------------------------------------------ pre-pass ----
// One block = one 64-token tile of one (sequence, KV head): thread (token
// tid/4, dims 32*(tid%4)..) decodes its keys and values; values go
// dimension-major through LDS.  Every store is one 16-byte unit.
__device__ __forceinline__ uint4 pack8(const _Float16* h) {
  uint4 r;
  r.x = h16(h[0]) | (h16(h[1]) << 16);
  r.y = h16(h[2]) | (h16(h[3]) << 16);
  r.z = h16(h[4]) | (h16(h[5]) << 16);
  r.w = h16(h[6]) | (h16(h[7]) << 16);
  return r;
}

// keys of token tt (dims dq..dq+31) into the K parts; vs[d][tt] = values
__device__ __forceinline__ void store_keys(_Float16* img, int tt, int dq, const float* kv) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) split_f16(kv[8 * i + e], hi[e], lo[e]);
    const int off = kimg_off(tt, dq / 8 + i);
    *(uint4*)(img + off) = pack8(hi);
    *(uint4*)(img + kImgKL + off) = pack8(lo);
  }
}

// value rows: thread (dim tid/2, key half tid%2) writes units 4*(tid%2)..+3
// of the hi plane (image) and the lo plane; returns this thread's largest
// hi-only error |v - 2^8 hi| (NaN when a value is not finite or leaves the
// f16 range)
__device__ __forceinline__ float store_values(_Float16* img, _Float16* lo_img, const float (*vs)[kKT + 1],
                                              int tid) {
  const int d = tid >> 1, st = tid & 1;
  float err = 0.0f;
#pragma unroll
  for (int kg = 0; kg < 4; ++kg) {
    const int u = 4 * st + kg;
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = vs[d][vunit_key(u, e)];
      split_f16(v * kValIn, hi[e], lo[e]);
      // exact: v and 2^8 hi agree to within f16's rounding
      const float r = fabsf(v - (float)hi[e] * kValOut);
      err = (r > err || r != r) ? r : err;
    }
    *(uint4*)(img + kImgV + vimg_off(d, u)) = pack8(hi);
    *(uint4*)(lo_img + vimg_off(d, u)) = pack8(lo);
  }
  return err;
}

// The tile's largest hi-only value error over every thread's (NaN-
// propagating maxima); one thread writes it.
__device__ __forceinline__ void store_tile_err(float* dst, float err, int tid) {
  __shared__ float red[4];
  auto nmax = [](float a, float b) { return (a > b || a != a) ? a : b; };
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) err = nmax(err, __shfl_xor(err, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = err;
  __syncthreads();
  if (tid == 0) *dst = nmax(nmax(red[0], red[1]), nmax(red[2], red[3]));
}

// WIDE: the thread's 32 dims are 16 key bytes (two codes or two 2-dim block
// indices per byte, 64-byte key rows) and 8 value bytes (2-bit codes, groups
// of 32, 32-byte value rows) with one scale / zero, read as one 16-byte and
// one 8-byte load; the decoded numbers are the same as the byte-wise path's.
template <int KEY, typename TN, typename TV, bool WIDE>
__global__ __launch_bounds__(256) void decode_hist_planes_kernel(smaq_attn_params p, HistAddr addr,
                                                                 PrefillPlanes pl) {
  __shared__ float vs[kD][kKT + 1];
  const int tid = threadIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * kKT;
  const int tt = tid >> 2, dq = 32 * (tid & 3);
  const int64_t t = t0 + tt;
  const int64_t len = p.hist_len ? min((int64_t)p.hist_len[b], (int64_t)p.max_hist_len) : p.max_hist_len;
  const int64_t tile = ((int64_t)b * p.n_kv_heads + h) * (pl.Lp / kKT) + blockIdx.x;
  _Float16* img = pl.img + tile * kImg;
  float kv[32];
  if (WIDE && t < len) {
    const int64_t ra = addr.row(b, h, t);
    const uint4 kb = *(const uint4*)((const uint8_t*)p.key_bytes + ra * 64 + dq / 2);
    const uint32_t kw[4] = {kb.x, kb.y, kb.z, kb.w};
    if constexpr (KEY == SMAQ_KEY_SCALAR) {
      const float nrm = Num<TN>::to_f(((const TN*)p.key_norms)[ra]);
      const int kbits = p.key_bits;
      const uint32_t kmask = (1u << kbits) - 1u;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t byte = (kw[j >> 2] >> (8 * (j & 3))) & 0xffu;
        kv[2 * j] = p.key_lut[byte & kmask] * nrm;
        kv[2 * j + 1] = p.key_lut[(byte >> kbits) & kmask] * nrm;
      }
    } else {
      const int nc = p.vq_centroids;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int ci = min((int)((kw[j >> 2] >> (8 * (j & 3))) & 0xffu), nc - 1);
        const float2 c = *(const float2*)(p.key_lut + ((int64_t)(dq / 2 + j) * nc + ci) * 2);
        kv[2 * j] = c.x;
        kv[2 * j + 1] = c.y;
      }
    }
    const uint2 vb = *(const uint2*)((const uint8_t*)p.val_bytes + ra * 32 + dq / 4);
    const float sc = Num<TV>::to_f(((const TV*)p.val_scales)[ra * 4 + (tid & 3)]);
    const float z = Num<TV>::to_f(((const TV*)p.val_zeros)[ra * 4 + (tid & 3)]);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const uint32_t code = ((i < 16 ? vb.x : vb.y) >> (2 * (i & 15))) & 3u;
      vs[dq + i][tt] = (float)code * sc + z;
    }
  } else if (t < len) {
    const int64_t ra = addr.row(b, h, t);
    const uint8_t* kr = (const uint8_t*)p.key_bytes + ra * p.key_row_bytes;
    float nrm = 1.0f;
    if (KEY == SMAQ_KEY_SCALAR) nrm = Num<TN>::to_f(((const TN*)p.key_norms)[ra]);
    const int kbits = p.key_bits, kvpb = (8 / kbits) > 1 ? 8 / kbits : 1;
    const uint32_t kmask = (1u << kbits) - 1u;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int d = dq + i;
      if (KEY == SMAQ_KEY_SCALAR) {
        const uint32_t byte = kr[d / kvpb];
        kv[i] = p.key_lut[(byte >> ((d % kvpb) * kbits)) & kmask] * nrm;
      } else {
        const int bd = p.vq_block_dim, nc = p.vq_centroids, blk = d / bd;
        const int ci = min((int)kr[blk], nc - 1);
        kv[i] = p.key_lut[((int64_t)blk * nc + ci) * bd + (d - blk * bd)];
      }
    }
    const uint8_t* vr = (const uint8_t*)p.val_bytes + ra * p.val_row_bytes;
    const int vbits = p.val_bits, vvpb = vbits == 2 ? 4 : (vbits == 4 ? 2 : 1);
    const uint32_t vmask = (1u << vbits) - 1u;
    const int ng = kD / p.val_group;
    const TV* vsc = (const TV*)p.val_scales + ra * ng;
    const TV* vz = (const TV*)p.val_zeros + ra * ng;
    for (int i = 0; i < 32; ++i) {
      const int d = dq + i;
      const uint32_t byte = vr[d / vvpb];
      const uint32_t code = (vvpb == 1) ? byte : (byte >> ((d % vvpb) * vbits)) & vmask;
      const int gi = d / p.val_group;
      vs[d][tt] = (float)code * Num<TV>::to_f(vsc[gi]) + Num<TV>::to_f(vz[gi]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      kv[i] = 0.0f;
      vs[dq + i][tt] = 0.0f;
    }
  }
  store_keys(img, tt, dq, kv);
  __syncthreads();
  store_tile_err(pl.err + tile, store_values(img, pl.img_lo + tile * kPrefillLoHalves, vs, tid), tid);
}

// Recent window: recent_k/v [batch][R][Hkv][D] -> tile images.
template <typename TR>
__global__ __launch_bounds__(256) void decode_recent_planes_kernel(smaq_attn_params p, PrefillPlanes pl) {
  __shared__ float vs[kD][kKT + 1];
  const int tid = threadIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * kKT;
  const int tt = tid >> 2, dq = 32 * (tid & 3);
  const int64_t t = t0 + tt;
  const int64_t len = p.recent_len ? min((int64_t)p.recent_len[b], (int64_t)p.max_recent_len) : p.max_recent_len;
  const int64_t tile = ((int64_t)b * p.n_kv_heads + h) * (pl.Lp / kKT) + blockIdx.x;
  _Float16* img = pl.img + tile * kImg;
  const int64_t src = (int64_t)b * p.recent_batch_stride + (t * p.n_kv_heads + h) * kD + dq;
  float kv[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    float vv = 0.0f;
    kv[i] = 0.0f;
    if (t < len) {
      kv[i] = Num<TR>::to_f(((const TR*)p.recent_k)[src + i]);
      vv = Num<TR>::to_f(((const TR*)p.recent_v)[src + i]);
    }
    vs[dq + i][tt] = vv;
  }
  store_keys(img, tt, dq, kv);
  __syncthreads();
  store_tile_err(pl.err + tile, store_values(img, pl.img_lo + tile * kPrefillLoHalves, vs, tid), tid);
}

// --------------------------------------------------------------- kernel ----
// grid: x = key split, y = query head, z = sequence * query blocks
template <bool CAUSAL>
__global__ __launch_bounds__(kPT) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_mfma_kernel(
    smaq_attn_params p, PrefillPart pp, Partials part) {
  // cheap form: a ring of three tile images; precise form: two 64 KB buffers
  __shared__ __attribute__((aligned(16))) _Float16 lds[3 * kImg];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int n = lane & 15, kg = lane >> 4;
  const int g = p.n_q_heads / p.n_kv_heads;
  const int nqb = (p.q_len + kQB - 1) / kQB;
  const int s = blockIdx.x, hq = blockIdx.y;
  const int b = blockIdx.z / nqb, qblk = blockIdx.z - b * nqb;
  const int h = hq / g, j = hq - h * g;
  const int rows = p.q_len * g;

  // ---- this lane's query columns: token qt0 + 16 qb + n (qb = 0, 1)
  const int qt0 = qblk * kQB + w * kQW;
  int qtok[2];
  bool qvalid[2];
  long long qpos[2];
  float qfac[2];
  u32x4 bqh[2][4], bql[2][4];  // B operands: [qb][dim step] hi / lo
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int t = qt0 + 16 * qb + n;
    qtok[qb] = t;
    qvalid[qb] = t < p.q_len;
    const int tc = qvalid[qb] ? t : 0;
    const float* qr = pp.q + (((int64_t)b * p.q_len + tc) * p.n_q_heads + hq) * kD;
    float qv[32];
    float qmax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qv[8 * ks + e] = qvalid[qb] ? qr[32 * ks + 8 * kg + e] : 0.0f;
        qmax = fmaxf(qmax, fabsf(qv[8 * ks + e]));
      }
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16, 64));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
    const int eq = exponent_of(qmax);
    const float qsc = ldexpf(1.0f, -eq);
    qfac[qb] = p.scale * kLog2e * ldexpf(1.0f, eq);
    qpos[qb] = (CAUSAL && qvalid[qb]) ? p.q_positions[(int64_t)b * p.q_len + t] : 0;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        _Float16 h0, l0, h1, l1;
        split_f16(qv[8 * ks + 2 * i] * qsc, h0, l0);
        split_f16(qv[8 * ks + 2 * i + 1] * qsc, h1, l1);
        hw[i] = h16(h0) | (h16(h1) << 16);
        lw[i] = h16(l0) | (h16(l1) << 16);
      }
      bqh[qb][ks] = u32x4{hw[0], hw[1], hw[2], hw[3]};
      bql[qb][ks] = u32x4{lw[0], lw[1], lw[2], lw[3]};
    }
  }

  // Queries that are exact in f16 after the power-of-two scaling (fp16 and,
  // within f16's exponent range, bf16 queries) have all-zero lo parts; their
  // ql.kh product adds exact zeros, so the QK below skips it for the whole
  // wave -- bit-identical scores, a third fewer QK matrix ops.
  uint32_t q_lo_bits = 0;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) q_lo_bits |= bql[qb][ks][0] | bql[qb][ks][1] | bql[qb][ks][2] | bql[qb][ks][3];
  const bool q_lo_zero = __all(q_lo_bits == 0);

  // ---- key range of this split, cut at the last key any query here can see
  const int64_t len = pp.len ? min((int64_t)pp.len[b], pp.max_len) : pp.max_len;
  const int64_t k0 = (int64_t)s * pp.split_len;
  int64_t k1 = min(len, k0 + pp.split_len);
  if (CAUSAL) {
    long long pmax = -1;
    const int tl = min(p.q_len, qblk * kQB + kQB) - 1;
    for (int t = qblk * kQB; t <= tl; ++t) pmax = max(pmax, (long long)p.q_positions[(int64_t)b * p.q_len + t]);
    k1 = min(k1, (int64_t)(pmax - pp.pos_offset + 1));
  }

  int64_t vis[2];  // keys [.., vis) are visible to the query column
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) vis[qb] = CAUSAL ? min(k1, (int64_t)(qpos[qb] - pp.pos_offset + 1)) : k1;

  float m_run[2] = {-__builtin_inff(), -__builtin_inff()};
  float m_thr[2] = {-__builtin_inff(), -__builtin_inff()};
  float l_run[2] = {0.0f, 0.0f};
  f32x4 acc_o[2][8];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 8; ++db) acc_o[qb][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- tile images of this (sequence, KV head).  Tile kt / 64 is copied
  // into an LDS buffer by direct-to-LDS loads: load j of wave w covers the
  // 16-byte units 512 j + 64 w .. + 63, contiguous in LDS (loads 0-5 the
  // image; in the precise form 6-7 the value-lo plane, placed after it)
  const int64_t tile0 = ((int64_t)b * p.n_kv_heads + h) * (pp.Lp / kKT);
  const _Float16* img0 = pp.img + tile0 * kImg;
  const _Float16* lo0 = pp.img_lo + tile0 * kPrefillLoHalves;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  // (unit 512 j + tid sits 16 (512 j + tid) bytes into the image: a
  // wave-uniform base plus one 32-bit lane offset, the loads' SGPR-base form)
  const uint32_t lane_off = 16u * (uint32_t)tid;
  auto copy_tile = [&](int64_t kt, _Float16* dst, auto prec_tag) {
    const char* src = (const char*)(img0 + (kt / kKT) * kImg);
#pragma unroll
    for (int jl = 0; jl < kCopyLoads; ++jl)
      __builtin_amdgcn_global_load_lds((const void*)(src + 16 * kPT * jl + lane_off),
                                       (__attribute__((address_space(3))) void*)(dst + 8 * (kPT * jl + 64 * wu)), 16, 0,
                                       0);
    if constexpr (decltype(prec_tag)::value) {
      const char* srl = (const char*)(lo0 + (kt / kKT) * kPrefillLoHalves);
#pragma unroll
      for (int jl = 0; jl < kCopyLoadsLo; ++jl)
        __builtin_amdgcn_global_load_lds((const void*)(srl + 16 * kPT * jl + lane_off),
                                         (__attribute__((address_space(3))) void*)(dst + kImg + 8 * (kPT * jl + 64 * wu)),
                                         16, 0, 0);
    }
  };
  // The precise form when a tile of the key range leaves more than the
  // budget to the value hi plane, or holds a value that is not finite (each
  // lane reads every 64th tile error the pre-pass wrote).  The form is
  // chosen once for the whole loop, the same in every wave.
  bool over = false;
  for (int64_t t = k0 / kKT + lane; t * kKT < k1; t += 64) over |= !(pp.err[tile0 + t] <= kRepBudget);
  const bool precise = __any(over);
  float one = 1.0f;  // opaque to the compiler (see split2_f16)
  asm volatile("" : "+v"(one));
  u32x4 ph[2][2], pl[2][2];  // [qb][32-key step]: P^T as B operands
  // ---- O^T += V^T P^T over one value plane: dims 16db + 4kg + v (rows),
  // query column n; with the weights' hi and lo parts or the hi parts only
  auto pv_plane = [&](const _Float16* vimg, auto with_pl) {
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        // A: dim 16db + n, keys 32st + 4kg + 0..3 and 32st + 16 + 4kg + 0..3
        // (one unit of the value plane)
        const u32x4 av = *(const u32x4*)&vimg[vimg_off(16 * db + n, 4 * st + kg)];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          acc_o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av),
                                                                 __builtin_bit_cast(f16x8, ph[qb][st]), acc_o[qb][db], 0, 0, 0);
          if constexpr (decltype(with_pl)::value)
            acc_o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av),
                                                                   __builtin_bit_cast(f16x8, pl[qb][st]), acc_o[qb][db], 0, 0, 0);
        }
      }
  };
  // vimg: the value hi plane of a buffer; the precise form's lo plane
  // follows the image in its buffer
  auto pv = [&](const _Float16* vimg, auto prec_tag) {
    __builtin_amdgcn_s_setprio(1);
    pv_plane(vimg, std::true_type{});
    if constexpr (decltype(prec_tag)::value) pv_plane(vimg + (kImg - kImgV), std::false_type{});
    __builtin_amdgcn_s_setprio(0);
  };
  // In the cheap form waves w and w + 4 of the workgroup share a SIMD.
  // Waves 0-3 run tile i as QK(i), softmax(i), PV(i); waves 4-7 as
  // PV(i - 1), QK(i), softmax(i), so that on every SIMD one wave's softmax
  // runs beside the other's matrix work rather than in step with it.  The
  // ring then holds tiles i - 1, i and (arriving) i + 1 while tile i is
  // computed: tile i + 1 is copied into the buffer of tile i - 2 once every
  // wave has passed tile i's barrier.  The precise form runs every wave in
  // step over two buffers (tile i + 1 into the buffer of tile i - 1).
  auto run = [&](auto prec_tag) {
    constexpr bool PREC = decltype(prec_tag)::value;
    constexpr int NBUF = PREC ? 2 : 3;
    constexpr int SLOT = PREC ? kImgP : kImg;
    const bool late = !PREC && wu >= 4;
    if (k0 < k1) copy_tile(k0, lds, prec_tag);
    int buf = 0;  // buffer of tile i (tile i - 1 sits in buf - 1 mod NBUF)
    for (int64_t kt0 = k0; kt0 < k1; kt0 += kKT) {
      // this thread's copies of tile i have landed, then every thread's
      // have, and every wave is done with the buffer tile i + 1 takes.  The
      // barrier carries no memory fence; the empty asm statements keep the
      // compiler from moving LDS accesses across the wait or the barrier.
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      const int nbuf = buf == NBUF - 1 ? 0 : buf + 1;
      if (kt0 + kKT < k1) copy_tile(kt0 + kKT, lds + nbuf * SLOT, prec_tag);
      const _Float16* kimg = lds + buf * SLOT;
      const _Float16* vimg = kimg + kImgV;
      if (late && kt0 > k0) pv(lds + (buf == 0 ? NBUF - 1 : buf - 1) * SLOT + kImgV, prec_tag);
      buf = nbuf;
      // ---- S^T = K Q^T: keys 16kb + 4kg + v (rows), query 16qb + n (column)
      f32x4 sacc[2][4];
  #pragma unroll
      for (int qb = 0; qb < 2; ++qb)
  #pragma unroll
        for (int kb = 0; kb < 4; ++kb) sacc[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      // matrix sections at raised wave priority (the two waves of a SIMD then
      // overlap one's softmax with the other's matrix work: 4.66 -> 4.49 ms at
      // c4; a fixed priority difference between the two was slower)
      __builtin_amdgcn_s_setprio(1);
      // two straight-line versions (with / without the query-lo products),
      // chosen once per tile, so that no branch splits the matrix section
      auto qk = [&](auto with_lo) {
  #pragma unroll
        for (int kb = 0; kb < 4; ++kb)
  #pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            // key row 16 kb + n, dims 32 ks + 8 kg .. + 7 (unit 4 ks + kg)
            const int off = kimg_off(16 * kb + n, 4 * ks + kg);
            const u32x4 ah = *(const u32x4*)&kimg[off];
            const u32x4 al = *(const u32x4*)&kimg[kImgKL + off];
  #pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
              sacc[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ah),
                                                                    __builtin_bit_cast(f16x8, bqh[qb][ks]), sacc[qb][kb], 0, 0, 0);
              sacc[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, al),
                                                                    __builtin_bit_cast(f16x8, bqh[qb][ks]), sacc[qb][kb], 0, 0, 0);
              if constexpr (decltype(with_lo)::value)
                sacc[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ah),
                                                                      __builtin_bit_cast(f16x8, bql[qb][ks]), sacc[qb][kb], 0, 0, 0);
            }
          }
      };
      if (q_lo_zero)
        qk(std::false_type{});
      else
        qk(std::true_type{});
      __builtin_amdgcn_s_setprio(0);
      // ---- softmax per query column (base 2, lazily raised reference max).
      // When every column of the wave sees all 64 keys of the tile (no causal
      // or length cut), the maximum is taken on the raw scores (qfac > 0
      // commutes with it) and a weight is exp2(s qfac - m), one fused
      // multiply-add; boundary tiles and columns with no visible key yet take
      // the masked form.
      const bool plain = __all(kt0 + kKT <= vis[0] && kt0 + kKT <= vis[1]);
      // Keys kt0 + i are visible to column qb for i < lim_of(qb).  The masked
      // branches below take opaque copies of the scale and of vis: the
      // compiler otherwise computes their products, compares and limits on the
      // unmasked tiles as well, to share them between the masked maximum and
      // the masked weights.
      auto lim_of = [&](int qb) -> int {
        int64_t vv = vis[qb];
        asm volatile("" : "+v"(vv));
        return (int)max((int64_t)-1, min((int64_t)kKT, vv - kt0));
      };
  #pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        float mt = -__builtin_inff();
        if (plain) {
  #pragma unroll
          for (int kb = 0; kb < 4; ++kb)
  #pragma unroll
            for (int v = 0; v < 4; ++v) mt = fmaxf(mt, sacc[qb][kb][v]);
          mt *= qfac[qb];
        } else {
          float qf = qfac[qb];
          asm volatile("" : "+v"(qf));
          const int lm = lim_of(qb);
  #pragma unroll
          for (int kb = 0; kb < 4; ++kb)
  #pragma unroll
            for (int v = 0; v < 4; ++v) {
              const float x = sacc[qb][kb][v] * qf;
              mt = fmaxf(mt, 16 * kb + 4 * kg + v >= lm ? -__builtin_inff() : x);
            }
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        if (__any(mt > m_thr[qb])) {
          const float m_new = fmaxf(m_run[qb], mt);
          const float alpha = (m_run[qb] == -__builtin_inff()) ? 0.0f : exp2f(m_run[qb] - m_new);
  #pragma unroll
          for (int db = 0; db < 8; ++db) acc_o[qb][db] *= alpha;
          l_run[qb] *= alpha;
          m_run[qb] = m_new;
          m_thr[qb] = m_new + kLazy;
        }
        const bool dead = m_run[qb] == -__builtin_inff();
        float ls = 0.0f;
        uint32_t hw[2][4], lw[2][4];
        // step kb >> 1; elements 0..3 from the even key block, 4..7 the odd one
        if (plain && !__any(dead)) {
          const float mneg = -m_run[qb];
  #pragma unroll
          for (int kb = 0; kb < 4; ++kb)
  #pragma unroll
            for (int v = 0; v < 4; v += 2) {
              const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][kb][v], qfac[qb], mneg));
              const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][kb][v + 1], qfac[qb], mneg));
              ls += p0 + p1;
              const int dw = 2 * (kb & 1) + (v >> 1);
              split2_f16(p0, p1, one, hw[kb >> 1][dw], lw[kb >> 1][dw]);
            }
        } else {
          float qf = qfac[qb];
          asm volatile("" : "+v"(qf));
          const int lm = lim_of(qb);
  #pragma unroll
          for (int kb = 0; kb < 4; ++kb)
  #pragma unroll
            for (int v = 0; v < 4; v += 2) {
              float x0 = sacc[qb][kb][v] * qf, x1 = sacc[qb][kb][v + 1] * qf;
              if (16 * kb + 4 * kg + v >= lm) x0 = -__builtin_inff();
              if (16 * kb + 4 * kg + v + 1 >= lm) x1 = -__builtin_inff();
              const float p0 = dead ? 0.0f : __builtin_amdgcn_exp2f(x0 - m_run[qb]);
              const float p1 = dead ? 0.0f : __builtin_amdgcn_exp2f(x1 - m_run[qb]);
              ls += p0 + p1;
              const int dw = 2 * (kb & 1) + (v >> 1);
              split2_f16(p0, p1, one, hw[kb >> 1][dw], lw[kb >> 1][dw]);
            }
        }
        l_run[qb] += ls;
  #pragma unroll
        for (int st = 0; st < 2; ++st) {
          ph[qb][st] = u32x4{hw[st][0], hw[st][1], hw[st][2], hw[st][3]};
          pl[qb][st] = u32x4{lw[st][0], lw[st][1], lw[st][2], lw[st][3]};
        }
      }
      if (!late) pv(vimg, prec_tag);
    }
    // the late waves' PV of the last tile (its buffer is not copied over again)
    if (late && k0 < k1) pv(lds + (buf == 0 ? NBUF - 1 : buf - 1) * SLOT + kImgV, prec_tag);
  };
  if (precise)
    run(std::true_type{});
  else
    run(std::false_type{});

  // ---- partials (natural-log max), one row per valid query column; the
  // sums return from the value planes' 2^-8 to the values' scale
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float l = l_run[qb];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (!qvalid[qb]) continue;
    const int row = qtok[qb] * g + j;
    const int64_t pi = part.idx(b, h, p.n_kv_heads, rows, row, pp.s_base + s);
    float* o = part.o + pi * kD + 4 * kg;  // 4-byte aligned only
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int v = 0; v < 4; ++v) o[16 * db + v] = acc_o[qb][db][v] * kValOut;
    if (kg == 0) {
      part.m[pi] = m_run[qb] == -__builtin_inff() ? m_run[qb] : m_run[qb] * 0.6931471805599453f;
      part.l[pi] = l;
    }
  }
}

}  // namespace

static bool known_dtype(int t) { return t == SMAQ_F32 || t == SMAQ_F16 || t == SMAQ_BF16; }

bool prefill_mfma_supported(const smaq_attn_params& p) {
  const int64_t nqb = (p.q_len + kQB - 1) / kQB;
  if (p.head_dim != kD || p.q_len < 16 || (int64_t)p.batch * nqb >= 65536) return false;
  if (p.has_history && (!known_dtype(p.val_dtype) || (p.key_format == SMAQ_KEY_SCALAR && !known_dtype(p.norm_dtype))))
    return false;
  return !p.has_recent || known_dtype(p.recent_dtype);
}

int64_t prefill_padded_len(int64_t L) { return ((L + kKT - 1) / kKT) * kKT; }

static int64_t align256_(int64_t x) { return (x + 255) & ~(int64_t)255; }

int64_t prefill_planes_bytes(int64_t batch, int64_t n_kv_heads, int64_t Lp) {
  const int64_t tiles = batch * n_kv_heads * (Lp / kKT);
  return align256_(tiles * kImg * 2) + align256_(tiles * kPrefillLoHalves * 2) + align256_(tiles * 4);
}

PrefillPlanes prefill_planes_at(char* ws, int64_t batch, int64_t n_kv_heads, int64_t Lp) {
  const int64_t tiles = batch * n_kv_heads * (Lp / kKT);
  PrefillPlanes P;
  P.img = (_Float16*)ws;
  ws += align256_(tiles * kImg * 2);
  P.img_lo = (_Float16*)ws;
  ws += align256_(tiles * kPrefillLoHalves * 2);
  P.err = (float*)ws;
  P.Lp = Lp;
  return P;
}

int device_cu_count() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
    return cus;
  return 256;
}

// Workgroups hold 144 KB of LDS, one per CU.  Split the keys so that the
// grid covers at least three rounds of the device's CUs and, among up to
// twice that many splits, the one whose last round is fullest (splits of at
// least four tiles).
int64_t prefill_split_len(const smaq_attn_params& p, int64_t L) {
  const int n_cu = device_cu_count();
  const int64_t wgs = (int64_t)p.batch * p.n_q_heads * ((p.q_len + kQB - 1) / kQB);
  const int64_t max_s = (L + 4 * kKT - 1) / (4 * kKT);
  const int64_t s_min = std::min(max_s, std::max<int64_t>(1, (3 * n_cu + wgs - 1) / wgs));
  int64_t best = s_min;
  double best_fill = -1.0;
  for (int64_t s = s_min; s <= std::min(max_s, 2 * s_min); ++s) {
    const int64_t n = wgs * s, rounds = (n + n_cu - 1) / n_cu;
    const double fill = (double)n / ((double)n_cu * (double)rounds);
    if (fill > best_fill + 1e-9) {
      best_fill = fill;
      best = s;
    }
  }
  int64_t split = (L + best - 1) / best;
  split = ((split + kKT - 1) / kKT) * kKT;
  return split < 4 * kKT ? 4 * kKT : split;
}

int launch_prefill_planes_hist(const smaq_attn_params& p, const HistAddr& a, const PrefillPlanes& pl,
                               hipStream_t st) {
  dim3 grid((unsigned)(pl.Lp / kKT), p.n_kv_heads, p.batch);
  const bool wide_keys = p.key_row_bytes == 64 && ((uintptr_t)p.key_bytes & 15) == 0 &&
                         (p.key_format == SMAQ_KEY_SCALAR ? (p.key_bits == 3 || p.key_bits == 4)
                                                          : (p.vq_block_dim == 2 && p.vq_centroids <= 256 &&
                                                             ((uintptr_t)p.key_lut & 7) == 0));
  const bool wide = wide_keys && p.val_bits == 2 && p.val_group == 32 && p.val_row_bytes == 32 &&
                    ((uintptr_t)p.val_bytes & 7) == 0;
#define SMAQ_PLANES_W(KEY, TN, TV)                                                                          \
  if (wide) hipLaunchKernelGGL((decode_hist_planes_kernel<KEY, TN, TV, true>), grid, dim3(256), 0, st, p, a, pl); \
  else hipLaunchKernelGGL((decode_hist_planes_kernel<KEY, TN, TV, false>), grid, dim3(256), 0, st, p, a, pl);
#define SMAQ_PLANES_V(KEY, TN)                             \
  switch (p.val_dtype) {                                   \
    case SMAQ_F32: SMAQ_PLANES_W(KEY, TN, float); break;    \
    case SMAQ_F16: SMAQ_PLANES_W(KEY, TN, _Float16); break; \
    default: SMAQ_PLANES_W(KEY, TN, bf16); break;           \
  }
  if (p.key_format == SMAQ_KEY_SCALAR) {
    switch (p.norm_dtype) {
      case SMAQ_F32: SMAQ_PLANES_V(SMAQ_KEY_SCALAR, float); break;
      case SMAQ_F16: SMAQ_PLANES_V(SMAQ_KEY_SCALAR, _Float16); break;
      default: SMAQ_PLANES_V(SMAQ_KEY_SCALAR, bf16); break;
    }
  } else {
    SMAQ_PLANES_V(SMAQ_KEY_BLOCKVQ, float);
  }
#undef SMAQ_PLANES_V
#undef SMAQ_PLANES_W
  return launch_status("smaq_attn_hybrid(prefill planes)");
}

int launch_prefill_planes_recent(const smaq_attn_params& p, const PrefillPlanes& pl, hipStream_t st) {
  dim3 grid((unsigned)(pl.Lp / kKT), p.n_kv_heads, p.batch);
  switch (p.recent_dtype) {
    case SMAQ_F32: hipLaunchKernelGGL(decode_recent_planes_kernel<float>, grid, dim3(256), 0, st, p, pl); break;
    case SMAQ_F16: hipLaunchKernelGGL(decode_recent_planes_kernel<_Float16>, grid, dim3(256), 0, st, p, pl); break;
    default: hipLaunchKernelGGL(decode_recent_planes_kernel<bf16>, grid, dim3(256), 0, st, p, pl); break;
  }
  return launch_status("smaq_attn_hybrid(prefill recent planes)");
}

int launch_prefill_mfma(const smaq_attn_params& p, const PrefillPart& pp, int n_splits, const Partials& part,
                        hipStream_t st) {
  const int nqb = (p.q_len + kQB - 1) / kQB;
  dim3 grid((unsigned)n_splits, p.n_q_heads, (unsigned)(p.batch * nqb));
  if (p.q_positions)
    hipLaunchKernelGGL((prefill_mfma_kernel<true>), grid, dim3(kPT), 0, st, p, pp, part);
  else
    hipLaunchKernelGGL((prefill_mfma_kernel<false>), grid, dim3(kPT), 0, st, p, pp, part);
  return launch_status("smaq_attn_hybrid(prefill)");
}

}  // namespace smaq
