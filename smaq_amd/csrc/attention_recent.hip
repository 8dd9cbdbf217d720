// Exact recent window of a decode step (one query token per sequence,
// head_dim 128, 1, 2 or 4 query heads per KV head): the partials of the
// window's tokens for one (split, KV head, sequence), as the generic recent
// kernel in attention.hip writes them, from wide coalesced loads.
//
// Reference: the recent segment of compute_hybrid_attention
// (smaq/score.py:61-72): scores q . k * scale in fp32 against the exact keys,
// one softmax shared with the history, the weights applied to the exact
// values.  Here: per 64-token chunk, wave w takes tokens 16w..16w+15; a lane
// holds a quarter of one token's key (32 dims, 16-byte loads: 4 lanes read a
// 256-byte key row, kept packed) and reads the same quarter of the G query
// rows from LDS, and the quarters are summed with two lane exchanges.  At
// <= 128 VGPRs (16-bit windows) four workgroups share a CU, so the windows
// of a decode batch are cut into one-chunk splits that all run in one round
// (recent_decode_split_len).  The online softmax
// runs over the chunk (natural-log units, as the other partial writers); for
// the weighted values lane l holds dims 2l, 2l+1 of its wave's 16 tokens (one
// 256-byte value row per wave load).  The chunk's key and value loads are all
// issued before any is used, and the first chunk's together with the
// window length and the query rows, so a one-chunk split costs one memory
// round trip.
#include <math.h>

#include "attention_internal.h"
#include "rotate128.h"

namespace smaq {

namespace {

constexpr int kRD = 128;     // head_dim
constexpr int kRChunk = 64;  // tokens per online-softmax step (16 per wave)

// 32 consecutive recent-window elements (64 or 128 bytes), kept as loaded
// and widened on use.
template <typename T>
struct Row32 {
  static constexpr int kWords = sizeof(T) == 2 ? 16 : 32;
  uint32_t w[kWords];
  __device__ __forceinline__ void load(const T* src) {
#pragma unroll
    for (int i = 0; i < kWords; i += 4) {
      const uint4 v = *(const uint4*)((const uint32_t*)src + i);
      w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (sizeof(T) == 2)
      return Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(w[i >> 1] >> (16 * (i & 1)))));
    else
      return __builtin_bit_cast(float, w[i]);
  }
};

// Two consecutive elements, kept as loaded (one or two dwords).
template <typename T>
struct Pair {
  uint32_t w[sizeof(T) == 2 ? 1 : 2];
  __device__ __forceinline__ void load(const T* src) {
    if constexpr (sizeof(T) == 2) {
      w[0] = *(const uint32_t*)src;
    } else {
      const uint2 v = *(const uint2*)src;
      w[0] = v.x; w[1] = v.y;
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (sizeof(T) == 2)
      return Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(w[0] >> (16 * i))));
    else
      return __builtin_bit_cast(float, w[i]);
  }
};

// Waves per SIMD: 4 (<= 128 VGPRs) for 16-bit windows; fp32 windows hold
// twice the loaded words, 2.
template <typename TR>
constexpr int kRecentWaves = sizeof(TR) == 2 ? 4 : 2;

template <int G>
struct RecentLds {
  __attribute__((aligned(16))) float qs[G][kRD];  // the query rows
  float sc[G][kRChunk];                            // the chunk's scores, then weights
  float m_s[G], l_s[G], a_s[G];
  float red[4][G][kRD];                            // per-wave outputs, summed at the end
};

// Split s of the window of (KV head h, sequence b); tid = thread index.
template <typename TR, int G>
__device__ __forceinline__ void recent_block(RecentLds<G>& L, const smaq_attn_params& p, const Partials& part,
                                             int s_base, int64_t split_len, int s, int h, int b, int tid) {
  auto& qs = L.qs;
  auto& sc = L.sc;
  auto& m_s = L.m_s;
  auto& l_s = L.l_s;
  auto& a_s = L.a_s;
  auto& red = L.red;
  const int lane = tid & 63, w = tid >> 6;
  const int64_t t0 = (int64_t)s * split_len;
  const int64_t tstride = (int64_t)p.n_kv_heads * kRD;
  const TR* rk = (const TR*)p.recent_k + (int64_t)b * p.recent_batch_stride + (int64_t)h * kRD;
  const TR* rv = (const TR*)p.recent_v + (int64_t)b * p.recent_batch_stride + (int64_t)h * kRD;
  const int tq = lane & 15, dq = lane >> 4;
  const int kt = 16 * w + tq;
  // A chunk's loads: this lane's key quarter (token 16w + tq) and its wave's
  // 16 value pairs.  Rows are clamped to the buffer's last row
  // (max_recent_len - 1), not to the sequence's length, so the first chunk's
  // loads go out before the length, the query and the barrier; rows past
  // the window are dropped below.
  const int64_t last_row = p.max_recent_len - 1;
  Row32<TR> k;
  Pair<TR> v[16];
  auto load_chunk = [&](int64_t c0) {
    k.load(rk + min(c0 + kt, last_row) * tstride + 32 * dq);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i].load(rv + min(c0 + 16 * w + i, last_row) * tstride + 2 * lane);
  };
  load_chunk(t0);
  const int64_t len = p.recent_len ? min((int64_t)p.recent_len[b], (int64_t)p.max_recent_len) : p.max_recent_len;
  const int64_t t1 = min(len, t0 + split_len);
  const long long qpos = p.q_positions ? p.q_positions[b] : 0;

  // the G query rows of this KV head, staged in LDS (lane (tq, dq) reads
  // dims 32 dq .. of each)
  for (int i = tid; i < G * kRD; i += 256)
    qs[i / kRD][i % kRD] = exact_query(p, ((int64_t)b * p.n_q_heads + h * G) * kRD + i);
  if (tid < G) {
    m_s[tid] = -__builtin_inff();
    l_s[tid] = 0.0f;
  }
  float o[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) o[g][0] = o[g][1] = 0.0f;
  __syncthreads();

  for (int64_t c0 = t0; c0 < t1; c0 += kRChunk) {
    const int nt = (int)min((int64_t)kRChunk, t1 - c0);
    if (c0 > t0) load_chunk(c0);
    // scores: quarter dot products, summed over the 4 lanes of a token
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
      const float k0 = k.get(i), k1 = k.get(i + 1), k2 = k.get(i + 2), k3 = k.get(i + 3);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float4 qv = *(const float4*)&qs[g][32 * dq + i];
        acc[g] = fmaf(qv.x, k0, acc[g]);
        acc[g] = fmaf(qv.y, k1, acc[g]);
        acc[g] = fmaf(qv.z, k2, acc[g]);
        acc[g] = fmaf(qv.w, k3, acc[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      acc[g] += __shfl_xor(acc[g], 16, 64);
      acc[g] += __shfl_xor(acc[g], 32, 64);
    }
    if (dq == 0) {
      const bool live = kt < nt && !(p.q_positions && p.recent_pos_offset + c0 + kt > qpos);
#pragma unroll
      for (int g = 0; g < G; ++g) sc[g][kt] = live ? acc[g] * p.scale : -__builtin_inff();
    }
    __syncthreads();
    // online softmax of row g by wave g
    if (w < G) {
      const float x = sc[w][lane];
      const float m_old = m_s[w];
      const float m_new = fmaxf(m_old, warp_max(x));
      const float pw = m_new == -__builtin_inff() ? 0.0f : __expf(x - m_new);
      const float alpha = m_old == -__builtin_inff() ? 0.0f : __expf(m_old - m_new);
      const float ls = warp_sum(pw);
      sc[w][lane] = pw;
      if (lane == 0) {
        l_s[w] = l_s[w] * alpha + ls;
        m_s[w] = m_new;
        a_s[w] = alpha;
      }
    }
    __syncthreads();
    // weighted values of this wave's tokens
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float alpha = a_s[g];
      o[g][0] *= alpha;
      o[g][1] *= alpha;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (16 * w + i >= nt) break;  // uniform over the wave
      const float v0 = v[i].get(0), v1 = v[i].get(1);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pw = sc[g][16 * w + i];
        o[g][0] = fmaf(pw, v0, o[g][0]);
        o[g][1] = fmaf(pw, v1, o[g][1]);
      }
    }
    __syncthreads();  // sc is rewritten by the next chunk
  }

  // the 4 waves' sums, then the partial of each query row
#pragma unroll
  for (int g = 0; g < G; ++g) {
    red[w][g][2 * lane] = o[g][0];
    red[w][g][2 * lane + 1] = o[g][1];
  }
  __syncthreads();
  for (int i = tid; i < G * kRD; i += 256) {
    const int g = i / kRD, d = i - g * kRD;
    const float sum = (red[0][g][d] + red[1][g][d]) + (red[2][g][d] + red[3][g][d]);
    const int64_t pi = part.idx(b, h, p.n_kv_heads, G, g, s_base + s);
    part.o[pi * kRD + d] = sum;
    if (d == 0) {
      part.m[pi] = m_s[g];
      part.l[pi] = l_s[g];
    }
  }
}

template <typename TR, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kRecentWaves<TR>, kRecentWaves<TR>))) void recent_decode_kernel(
    smaq_attn_params p, Partials part, int s_base, int64_t split_len) {
  __shared__ RecentLds<G> lds;
  recent_block<TR, G>(lds, p, part, s_base, split_len, blockIdx.x, blockIdx.y, blockIdx.z, threadIdx.x);
}

// The query rotation (into q_hist) and the recent window in one launch: they
// are independent (the window reads the raw query), so the shorter one runs
// beside the longer instead of after it.  Blocks [0, n_rot) rotate 4 rows
// each (rotate128.h); block n_rot + ((b * Hkv + h) * n_splits + s) takes split
// s of (KV head h, sequence b).
template <typename TR, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kRecentWaves<TR>, kRecentWaves<TR>))) void rotate_recent_kernel(
    smaq_attn_params p, Partials part, int s_base, int n_splits, int64_t split_len, int n_rot) {
  __shared__ union {
    RecentLds<G> r;
    Rot128Lds<4> q;
  } lds;
  const int bx = blockIdx.x, tid = threadIdx.x;
  if (bx < n_rot) {
    rotate128_block<4>(lds.q, p.q_raw, p.q_raw_dtype, (int64_t)p.batch * p.q_len * p.n_q_heads, p.rot_mt,
                       p.rot_scale, (float*)p.q_hist, bx, tid);
    return;
  }
  const int r = bx - n_rot;
  const int s = r % n_splits, hb = r / n_splits;
  recent_block<TR, G>(lds.r, p, part, s_base, split_len, s, hb % p.n_kv_heads, hb / p.n_kv_heads, tid);
}

template <typename TR>
void launch_g(const smaq_attn_params& p, const Partials& part, int s_base, int n_splits, int64_t split_len,
              hipStream_t st) {
  const dim3 grid((unsigned)n_splits, (unsigned)p.n_kv_heads, (unsigned)p.batch);
  switch (p.n_q_heads / p.n_kv_heads) {
    case 1: hipLaunchKernelGGL((recent_decode_kernel<TR, 1>), grid, dim3(256), 0, st, p, part, s_base, split_len); break;
    case 2: hipLaunchKernelGGL((recent_decode_kernel<TR, 2>), grid, dim3(256), 0, st, p, part, s_base, split_len); break;
    default: hipLaunchKernelGGL((recent_decode_kernel<TR, 4>), grid, dim3(256), 0, st, p, part, s_base, split_len); break;
  }
}

}  // namespace

int64_t recent_decode_split_len() { return kRChunk; }

bool recent_decode_supported(const smaq_attn_params& p) {
  const int g = p.n_q_heads / p.n_kv_heads;
  return p.impl != 1 && p.has_recent && p.q_len == 1 && p.head_dim == kRD && (g == 1 || g == 2 || g == 4) &&
         (p.recent_dtype == SMAQ_F32 || p.recent_dtype == SMAQ_F16 || p.recent_dtype == SMAQ_BF16) &&
         // 16-byte key loads and 4- or 8-byte value loads at element offsets
         // that are multiples of 8 and 2
         (((uintptr_t)p.recent_k | (uintptr_t)p.recent_v) & 15) == 0;
}

template <typename TR>
void launch_rg(const smaq_attn_params& p, const Partials& part, int s_base, int n_splits, int64_t split_len,
               hipStream_t st) {
  const int64_t rows = (int64_t)p.batch * p.q_len * p.n_q_heads;
  const int n_rot = (int)((rows + 3) / 4);
  const dim3 grid((unsigned)(n_rot + (int64_t)n_splits * p.n_kv_heads * p.batch));
  switch (p.n_q_heads / p.n_kv_heads) {
    case 1: hipLaunchKernelGGL((rotate_recent_kernel<TR, 1>), grid, dim3(256), 0, st, p, part, s_base, n_splits, split_len, n_rot); break;
    case 2: hipLaunchKernelGGL((rotate_recent_kernel<TR, 2>), grid, dim3(256), 0, st, p, part, s_base, n_splits, split_len, n_rot); break;
    default: hipLaunchKernelGGL((rotate_recent_kernel<TR, 4>), grid, dim3(256), 0, st, p, part, s_base, n_splits, split_len, n_rot); break;
  }
}

bool rotate_recent_supported(const smaq_attn_params& p) {
  const int64_t rows = (int64_t)p.batch * p.q_len * p.n_q_heads;
  return recent_decode_supported(p) && p.rot_mt && p.q_raw && p.q_hist && ((uintptr_t)p.rot_mt & 15) == 0 &&
         (p.q_raw_dtype == SMAQ_F32 || p.q_raw_dtype == SMAQ_F16 || p.q_raw_dtype == SMAQ_BF16) &&
         (rows + 3) / 4 + (int64_t)p.n_kv_heads * p.batch * 64 < (1ll << 31);
}

int launch_rotate_recent(const smaq_attn_params& p, const Partials& part, int s_base, int n_splits,
                         int64_t split_len, hipStream_t st) {
  switch (p.recent_dtype) {
    case SMAQ_F32: launch_rg<float>(p, part, s_base, n_splits, split_len, st); break;
    case SMAQ_F16: launch_rg<_Float16>(p, part, s_base, n_splits, split_len, st); break;
    default: launch_rg<bf16>(p, part, s_base, n_splits, split_len, st); break;
  }
  return launch_status("smaq_attn_hybrid(rotation + recent)");
}

int launch_recent_decode(const smaq_attn_params& p, const Partials& part, int s_base, int n_splits,
                         int64_t split_len, hipStream_t st) {
  switch (p.recent_dtype) {
    case SMAQ_F32: launch_g<float>(p, part, s_base, n_splits, split_len, st); break;
    case SMAQ_F16: launch_g<_Float16>(p, part, s_base, n_splits, split_len, st); break;
    default: launch_g<bf16>(p, part, s_base, n_splits, split_len, st); break;
  }
  return launch_status("smaq_attn_hybrid(recent decode)");
}

}  // namespace smaq
