// Chunked-prefill attention on the gfx950 matrix cores (head_dim 128).
//
// Prefill is compute-bound (every key tile serves many query rows), so the
// packed cache is first decoded once per part into f16 hi/lo planes in the
// workspace (the dequantisation the generic kernels do per query tile):
//   keys   K~[t][d]  = lut[code] * norm (scalar) or decoded centroid (block-VQ);
//                      the recent window's exact keys
//   values V^[d][t]  = code * scale + zero (fp32, as the reference's
//                      dequantize_values), stored dimension-major
// each as hi = f16(x), lo = f16(x - hi), ~22 significant bits.
//
// The attention kernel then works in the transposed orientation, which fits
// the MFMA register layouts without any transpose:
//   S^T[key][query] = K~ . Q^T   v_mfma_f32_16x16x32_f16, A = key rows (LDS),
//                                B = query columns (registers, hi/lo split)
//   softmax per query column (keys = C rows: 4 per lane, 4 lane groups)
//   O^T[dim][query] += V^T . P^T  A = value rows (dimension-major tile),
//                                B = P^T straight from the S^T accumulators
// with qh.kh + qh.kl + ql.kh and vh.ph + vh.pl + vl.ph.  Each workgroup (4
// waves x 32 query rows) streams 64-key tiles of one (sequence, query head,
// key split) and writes the same (m, l, o) partials as the other attention
// kernels; attn_combine_kernel merges splits and the history / recent parts.
#include <math.h>

#include "attention_internal.h"

namespace smaq {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kKT = 64;           // keys per tile
constexpr int kQW = 32;           // query rows per wave
constexpr int kQB = 4 * kQW;      // query rows per workgroup
constexpr int kKS = 136;          // halves per key row of the K tile (128 + 8 pad)
constexpr int kVS = 72;           // halves per dim row of the V tile (64 + 8 pad)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;     // softmax reference max raised by > 2^8 only

__device__ __forceinline__ uint32_t h16(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }

__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

__device__ __forceinline__ int exponent_of(float x) {
  if (!(x > 0.0f)) return 0;
  int e;
  frexpf(x, &e);
  return e - 1;
}

// ------------------------------------------------------------ pre-pass ----
// One block = 64 tokens of one (sequence, KV head): thread (token tid/4,
// dims 32*(tid%4)..) decodes its keys and values; values go dimension-major
// through LDS.
template <int KEY, typename TN, typename TV>
__global__ __launch_bounds__(256) void decode_hist_planes_kernel(smaq_attn_params p, HistAddr addr,
                                                                 PrefillPlanes pl) {
  __shared__ float vs[kD][kKT + 1];
  const int tid = threadIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * kKT;
  const int tt = tid >> 2, dq = 32 * (tid & 3);
  const int64_t t = t0 + tt;
  const int64_t len = p.hist_len ? min((int64_t)p.hist_len[b], (int64_t)p.max_hist_len) : p.max_hist_len;
  const int64_t plane = ((int64_t)b * p.n_kv_heads + h) * pl.Lp;
  _Float16* kh = pl.kh + (plane + t) * kD + dq;
  _Float16* kl = pl.kl + (plane + t) * kD + dq;
  if (t < len) {
    const int64_t ra = addr.row(b, h, t);
    const uint8_t* kr = (const uint8_t*)p.key_bytes + ra * p.key_row_bytes;
    float nrm = 1.0f;
    if (KEY == SMAQ_KEY_SCALAR) nrm = Num<TN>::to_f(((const TN*)p.key_norms)[ra]);
    const int kbits = p.key_bits, kvpb = (8 / kbits) > 1 ? 8 / kbits : 1;
    const uint32_t kmask = (1u << kbits) - 1u;
    for (int i = 0; i < 32; ++i) {
      const int d = dq + i;
      float kv;
      if (KEY == SMAQ_KEY_SCALAR) {
        const uint32_t byte = kr[d / kvpb];
        kv = p.key_lut[(byte >> ((d % kvpb) * kbits)) & kmask] * nrm;
      } else {
        const int bd = p.vq_block_dim, nc = p.vq_centroids, blk = d / bd;
        const int ci = min((int)kr[blk], nc - 1);
        kv = p.key_lut[((int64_t)blk * nc + ci) * bd + (d - blk * bd)];
      }
      _Float16 hi, lo;
      split_f16(kv, hi, lo);
      kh[i] = hi;
      kl[i] = lo;
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
    for (int i = 0; i < 32; ++i) {
      kh[i] = (_Float16)0.0f;
      kl[i] = (_Float16)0.0f;
      vs[dq + i][tt] = 0.0f;
    }
  }
  __syncthreads();
  // values: thread (dim tid/2, tokens 32*(tid%2)..)
  const int d = tid >> 1, tq = 32 * (tid & 1);
  _Float16* vh = pl.vh + (((int64_t)b * p.n_kv_heads + h) * kD + d) * pl.Lp + t0 + tq;
  _Float16* vl = pl.vl + (((int64_t)b * p.n_kv_heads + h) * kD + d) * pl.Lp + t0 + tq;
  for (int i = 0; i < 32; ++i) {
    _Float16 hi, lo;
    split_f16(vs[d][tq + i], hi, lo);
    vh[i] = hi;
    vl[i] = lo;
  }
}

// Recent window: recent_k/v [batch][R][Hkv][D] -> planes.
template <typename TR>
__global__ __launch_bounds__(256) void decode_recent_planes_kernel(smaq_attn_params p, PrefillPlanes pl) {
  __shared__ float vs[kD][kKT + 1];
  const int tid = threadIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t t0 = (int64_t)blockIdx.x * kKT;
  const int tt = tid >> 2, dq = 32 * (tid & 3);
  const int64_t t = t0 + tt;
  const int64_t len = p.recent_len ? min((int64_t)p.recent_len[b], (int64_t)p.max_recent_len) : p.max_recent_len;
  const int64_t plane = ((int64_t)b * p.n_kv_heads + h) * pl.Lp;
  _Float16* kh = pl.kh + (plane + t) * kD + dq;
  _Float16* kl = pl.kl + (plane + t) * kD + dq;
  const int64_t src = (int64_t)b * p.recent_batch_stride + (t * p.n_kv_heads + h) * kD + dq;
  for (int i = 0; i < 32; ++i) {
    float kv = 0.0f, vv = 0.0f;
    if (t < len) {
      kv = Num<TR>::to_f(((const TR*)p.recent_k)[src + i]);
      vv = Num<TR>::to_f(((const TR*)p.recent_v)[src + i]);
    }
    _Float16 hi, lo;
    split_f16(kv, hi, lo);
    kh[i] = hi;
    kl[i] = lo;
    vs[dq + i][tt] = vv;
  }
  __syncthreads();
  const int d = tid >> 1, tq = 32 * (tid & 1);
  _Float16* vh = pl.vh + (((int64_t)b * p.n_kv_heads + h) * kD + d) * pl.Lp + t0 + tq;
  _Float16* vl = pl.vl + (((int64_t)b * p.n_kv_heads + h) * kD + d) * pl.Lp + t0 + tq;
  for (int i = 0; i < 32; ++i) {
    _Float16 hi, lo;
    split_f16(vs[d][tq + i], hi, lo);
    vh[i] = hi;
    vl[i] = lo;
  }
}

// --------------------------------------------------------------- kernel ----
// grid: x = key split, y = query head, z = sequence * query blocks
template <bool CAUSAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_mfma_kernel(
    smaq_attn_params p, PrefillPart pp, Partials part) {
  __shared__ __attribute__((aligned(16))) _Float16 ktile[2][kKT * kKS];   // [hi/lo][key][dim]
  __shared__ __attribute__((aligned(16))) _Float16 vtile[2][kD * kVS];    // [hi/lo][dim][key]

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

  const int64_t plane = ((int64_t)b * p.n_kv_heads + h) * pp.Lp;
  for (int64_t kt0 = k0; kt0 < k1; kt0 += kKT) {
    // ---- stage the 64-key tile: K rows [key][dim], V rows [dim][key]
    __syncthreads();
    {
      // K: 64 keys x 256 B per part = 1024 x 16 B pieces per part
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int piece = tid + 256 * i;          // 0..1023
        const int key = piece >> 4, c = piece & 15;
        const int64_t gi = (plane + kt0 + key) * kD + 8 * c;
        *(uint4*)&ktile[0][key * kKS + 8 * c] = *(const uint4*)(pp.kh + gi);
        *(uint4*)&ktile[1][key * kKS + 8 * c] = *(const uint4*)(pp.kl + gi);
      }
      // V: 128 dims x 128 B per part = 1024 x 16 B pieces per part
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int piece = tid + 256 * i;
        const int d = piece >> 3, c = piece & 7;
        const int64_t gi = (((int64_t)b * p.n_kv_heads + h) * kD + d) * pp.Lp + kt0 + 8 * c;
        *(uint4*)&vtile[0][d * kVS + 8 * c] = *(const uint4*)(pp.vh + gi);
        *(uint4*)&vtile[1][d * kVS + 8 * c] = *(const uint4*)(pp.vl + gi);
      }
    }
    __syncthreads();
    // ---- S^T = K Q^T: keys 16kb + 4kg + v (rows), query 16qb + n (column)
    f32x4 sacc[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) sacc[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int off = (16 * kb + n) * kKS + 32 * ks + 8 * kg;
        const u32x4 ah = *(const u32x4*)&ktile[0][off];
        const u32x4 al = *(const u32x4*)&ktile[1][off];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          sacc[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ah),
                                                                __builtin_bit_cast(f16x8, bqh[qb][ks]), sacc[qb][kb], 0, 0, 0);
          sacc[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, al),
                                                                __builtin_bit_cast(f16x8, bqh[qb][ks]), sacc[qb][kb], 0, 0, 0);
          sacc[qb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ah),
                                                                __builtin_bit_cast(f16x8, bql[qb][ks]), sacc[qb][kb], 0, 0, 0);
        }
      }
    // ---- softmax per query column (base 2, lazily raised reference max)
    u32x4 ph[2][2], pl[2][2];  // [qb][32-key step]: P^T as B operands
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      // keys kt0 + i are visible to this column for i < lim
      const int lim = (int)max((int64_t)-1, min((int64_t)kKT, vis[qb] - kt0));
      float sv[16];
      float mt = -__builtin_inff();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float x = sacc[qb][kb][v] * qfac[qb];
          if (16 * kb + 4 * kg + v >= lim) x = -__builtin_inff();
          sv[4 * kb + v] = x;
          mt = fmaxf(mt, x);
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
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int v = 0; v < 4; v += 2) {
          const float p0 = dead ? 0.0f : __builtin_amdgcn_exp2f(sv[4 * kb + v] - m_run[qb]);
          const float p1 = dead ? 0.0f : __builtin_amdgcn_exp2f(sv[4 * kb + v + 1] - m_run[qb]);
          ls += p0 + p1;
          _Float16 h0, l0, h1, l1;
          split_f16(p0, h0, l0);
          split_f16(p1, h1, l1);
          // step kb >> 1; elements 0..3 from the even key block, 4..7 the odd one
          const int dw = 2 * (kb & 1) + (v >> 1);
          hw[kb >> 1][dw] = h16(h0) | (h16(h1) << 16);
          lw[kb >> 1][dw] = h16(l0) | (h16(l1) << 16);
        }
      l_run[qb] += ls;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        ph[qb][st] = u32x4{hw[st][0], hw[st][1], hw[st][2], hw[st][3]};
        pl[qb][st] = u32x4{lw[st][0], lw[st][1], lw[st][2], lw[st][3]};
      }
    }
    // ---- O^T += V^T P^T: dims 16db + 4kg + v (rows), query column n
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        // A: dim 16db + n, keys 32st + 4kg + 0..3 and 32st + 16 + 4kg + 0..3
        const int base = (16 * db + n) * kVS + 32 * st + 4 * kg;
        const uint2 h0 = *(const uint2*)&vtile[0][base], h1 = *(const uint2*)&vtile[0][base + 16];
        const uint2 l0 = *(const uint2*)&vtile[1][base], l1 = *(const uint2*)&vtile[1][base + 16];
        const u32x4 avh = u32x4{h0.x, h0.y, h1.x, h1.y};
        const u32x4 avl = u32x4{l0.x, l0.y, l1.x, l1.y};
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          acc_o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, avh),
                                                                 __builtin_bit_cast(f16x8, ph[qb][st]), acc_o[qb][db], 0, 0, 0);
          acc_o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, avh),
                                                                 __builtin_bit_cast(f16x8, pl[qb][st]), acc_o[qb][db], 0, 0, 0);
          acc_o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, avl),
                                                                 __builtin_bit_cast(f16x8, ph[qb][st]), acc_o[qb][db], 0, 0, 0);
        }
      }
  }

  // ---- partials (natural-log max), one row per valid query column
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
      for (int v = 0; v < 4; ++v) o[16 * db + v] = acc_o[qb][db][v];
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

int64_t prefill_split_len(const smaq_attn_params& p, int64_t L) {
  const int64_t wgs = (int64_t)p.batch * p.n_q_heads * ((p.q_len + kQB - 1) / kQB);
  const int64_t want = wgs >= 512 ? 1 : (512 + wgs - 1) / wgs;
  int64_t split = (L + want - 1) / want;
  split = ((split + kKT - 1) / kKT) * kKT;
  return split < 4 * kKT ? 4 * kKT : split;
}

int launch_prefill_planes_hist(const smaq_attn_params& p, const HistAddr& a, const PrefillPlanes& pl,
                               hipStream_t st) {
  dim3 grid((unsigned)(pl.Lp / kKT), p.n_kv_heads, p.batch);
#define SMAQ_PLANES_V(KEY, TN)                                                                        \
  switch (p.val_dtype) {                                                                              \
    case SMAQ_F32: hipLaunchKernelGGL((decode_hist_planes_kernel<KEY, TN, float>), grid, dim3(256), 0, st, p, a, pl); break; \
    case SMAQ_F16: hipLaunchKernelGGL((decode_hist_planes_kernel<KEY, TN, _Float16>), grid, dim3(256), 0, st, p, a, pl); break; \
    default: hipLaunchKernelGGL((decode_hist_planes_kernel<KEY, TN, bf16>), grid, dim3(256), 0, st, p, a, pl); break; \
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
    hipLaunchKernelGGL(prefill_mfma_kernel<true>, grid, dim3(256), 0, st, p, pp, part);
  else
    hipLaunchKernelGGL(prefill_mfma_kernel<false>, grid, dim3(256), 0, st, p, pp, part);
  return launch_status("smaq_attn_hybrid(prefill)");
}

}  // namespace smaq
