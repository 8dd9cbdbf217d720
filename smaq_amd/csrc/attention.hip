// Fused quantized-KV attention (decode and prefill), flash-decoding style.
//
//   partial kernels : one workgroup per (context split, KV head x row tile,
//                     sequence).  Scores against the compressed history are
//                     computed straight from the packed bytes (scalar codes
//                     through the centroid LUT, or block-VQ indices through the
//                     pre-decoded centroids), an online softmax runs over each
//                     64-token chunk, and packed values are dequantised in
//                     registers for the weighted sum.  The exact recent window
//                     is one more segment with its own splits.
//   combine kernel  : merges the (m, l, o) partials of every split; history and
//                     recent outputs are normalised by the one shared softmax
//                     denominator, each cast to the output dtype and then
//                     added, as compute_hybrid_attention does.
//
// Score arithmetic follows the reference per segment: scalar history
// ((q_rot . c[code]) * norm) * scale, block-VQ (q . k_hat) * scale, recent
// (q . k) * scale, all fp32.
#include <math.h>

#include "attention_internal.h"

namespace smaq {

constexpr int kAttnThreads = 256;
constexpr int kChunk = 64;       // tokens per online-softmax step
constexpr int kRowTile = 16;     // query rows per workgroup
constexpr int kMaxHeadDim = 256;

// Online softmax over one chunk of scores already in sc[r][0..kChunk).
__device__ __forceinline__ void softmax_chunk(float (*sc)[kChunk], float* m_s, float* l_s,
                                              float* alpha_s, int nr) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int r = w; r < nr; r += kAttnThreads / 64) {
    const float s = sc[r][lane];
    const float cm = warp_max(s);
    const float m_old = m_s[r];
    const float m_new = fmaxf(m_old, cm);
    const float p = (m_new == -__builtin_inff()) ? 0.0f : __expf(s - m_new);
    const float alpha = (m_old == -__builtin_inff()) ? 0.0f : __expf(m_old - m_new);
    const float ls = warp_sum(p);
    sc[r][lane] = p;
    if (lane == 0) {
      l_s[r] = l_s[r] * alpha + ls;
      m_s[r] = m_new;
      alpha_s[r] = alpha;
    }
  }
}

// ------------------------------------------------------------ history ------
template <int KEY, typename TN, typename TV>
__global__ __launch_bounds__(kAttnThreads) void attn_hist_kernel(smaq_attn_params p, HistAddr addr,
                                                                 Partials part, int64_t split_len,
                                                                 int row_tiles) {
  __shared__ float qs[kRowTile][kMaxHeadDim];
  __shared__ float sc[kRowTile][kChunk];
  __shared__ float m_s[kRowTile], l_s[kRowTile], alpha_s[kRowTile];
  __shared__ long long qpos[kRowTile];
  __shared__ int64_t rowaddr[kChunk];
  __shared__ float lut[256];

  const int D = p.head_dim;
  const int g = p.n_q_heads / p.n_kv_heads;
  const int rows = p.q_len * g;
  const int s = blockIdx.x;
  const int h = blockIdx.y / row_tiles;
  const int rt = blockIdx.y - h * row_tiles;
  const int b = blockIdx.z;
  const int r0 = rt * kRowTile;
  const int nr = min(kRowTile, rows - r0);
  const int tid = threadIdx.x;
  const int64_t len = p.hist_len ? min((int64_t)p.hist_len[b], (int64_t)p.max_hist_len) : p.max_hist_len;
  const int64_t t0 = (int64_t)s * split_len;
  const int64_t t1 = min(len, t0 + split_len);

  for (int i = tid; i < nr * D; i += kAttnThreads) {
    const int r = i / D, d = i - r * D;
    const int row = r0 + r, t = row / g, j = row - t * g;
    qs[r][d] = p.q_hist[(((int64_t)b * p.q_len + t) * p.n_q_heads + h * g + j) * D + d];
  }
  if (tid < nr) {
    m_s[tid] = -__builtin_inff();
    l_s[tid] = 0.0f;
    const int t = (r0 + tid) / g;
    qpos[tid] = p.q_positions ? p.q_positions[(int64_t)b * p.q_len + t] : 0;
  }
  if (KEY == SMAQ_KEY_SCALAR) {
    for (int i = tid; i < (1 << p.key_bits); i += kAttnThreads) lut[i] = p.key_lut[i];
  }

  // PV mapping: thread owns dim pd and rows pr0, pr0 + prs, ...
  const int prs = kAttnThreads / D;
  const int pd = tid % D, pr0 = tid / D;
  float o[kRowTile];
#pragma unroll
  for (int i = 0; i < kRowTile; ++i) o[i] = 0.0f;

  // score mapping: thread owns token st and rows sr0, sr0 + 4, ...
  const int st = tid % kChunk, sr0 = tid / kChunk;
  const int kbits = p.key_bits;
  const int kvpb = (8 / kbits) > 1 ? 8 / kbits : 1;
  const uint32_t kmask = (1u << kbits) - 1u;
  const int vbits = p.val_bits;
  const int vvpb = vbits == 2 ? 4 : (vbits == 4 ? 2 : 1);
  const uint32_t vmask = (1u << vbits) - 1u;
  const int ng = D / p.val_group;
  const uint8_t* kbytes = (const uint8_t*)p.key_bytes;
  const uint8_t* vbytes = (const uint8_t*)p.val_bytes;
  const TV* vsc = (const TV*)p.val_scales;
  const TV* vz = (const TV*)p.val_zeros;
  __syncthreads();

  for (int64_t c0 = t0; c0 < t1; c0 += kChunk) {
    // ---- scores
    const int64_t t = c0 + st;
    const bool valid = t < t1;
    int64_t ra = 0;
    if (valid) ra = addr.row(b, h, t);
    if (sr0 == 0) rowaddr[st] = ra;
    float acc[kRowTile / 4];
#pragma unroll
    for (int i = 0; i < kRowTile / 4; ++i) acc[i] = 0.0f;
    if (valid) {
      const uint8_t* kr = kbytes + ra * p.key_row_bytes;
      if (KEY == SMAQ_KEY_SCALAR) {
        for (int d = 0; d < D; ++d) {
          const uint32_t byte = kr[d / kvpb];
          const float kv = lut[(byte >> ((d % kvpb) * kbits)) & kmask];
#pragma unroll
          for (int i = 0; i < kRowTile / 4; ++i) {
            const int r = sr0 + 4 * i;
            if (r < nr) acc[i] = fmaf(qs[r][d], kv, acc[i]);
          }
        }
      } else {
        const int bd = p.vq_block_dim, nc = p.vq_centroids;
        for (int blk = 0; blk < p.vq_blocks; ++blk) {
          const int ci = min((int)kr[blk], nc - 1);
          const float* cent = p.key_lut + ((int64_t)blk * nc + ci) * bd;
          for (int e = 0; e < bd; ++e) {
            const float kv = cent[e];
            const int d = blk * bd + e;
#pragma unroll
            for (int i = 0; i < kRowTile / 4; ++i) {
              const int r = sr0 + 4 * i;
              if (r < nr) acc[i] = fmaf(qs[r][d], kv, acc[i]);
            }
          }
        }
      }
    }
    const float nrm = (KEY == SMAQ_KEY_SCALAR && valid) ? Num<TN>::to_f(((const TN*)p.key_norms)[ra]) : 1.0f;
#pragma unroll
    for (int i = 0; i < kRowTile / 4; ++i) {
      const int r = sr0 + 4 * i;
      if (r < nr) {
        float sv = (KEY == SMAQ_KEY_SCALAR) ? (acc[i] * nrm) * p.scale : acc[i] * p.scale;
        if (!valid) sv = -__builtin_inff();
        if (p.q_positions && valid && p.hist_pos_offset + t > qpos[r]) sv = -__builtin_inff();
        sc[r][st] = sv;
      }
    }
    __syncthreads();
    softmax_chunk(sc, m_s, l_s, alpha_s, nr);
    __syncthreads();
    // ---- weighted values
    const int nt = (int)min((int64_t)kChunk, t1 - c0);
#pragma unroll
    for (int i = 0; i < kRowTile; ++i) {
      const int r = pr0 + i * prs;
      if (i * prs < kRowTile && r < nr && pr0 < prs) o[i] *= alpha_s[r];
    }
    if (pr0 < prs) {
      for (int k = 0; k < nt; ++k) {
        const int64_t va = rowaddr[k];
        const uint32_t byte = vbytes[va * p.val_row_bytes + pd / vvpb];
        const uint32_t code = (vvpb == 1) ? byte : (byte >> ((pd % vvpb) * vbits)) & vmask;
        const int gi = pd / p.val_group;
        const float vhat = (float)code * Num<TV>::to_f(vsc[va * ng + gi]) + Num<TV>::to_f(vz[va * ng + gi]);
#pragma unroll
        for (int i = 0; i < kRowTile; ++i) {
          const int r = pr0 + i * prs;
          if (i * prs < kRowTile && r < nr) o[i] = fmaf(sc[r][k], vhat, o[i]);
        }
      }
    }
    __syncthreads();
  }
  // ---- write partials
  if (pr0 < prs) {
#pragma unroll
    for (int i = 0; i < kRowTile; ++i) {
      const int r = pr0 + i * prs;
      if (i * prs < kRowTile && r < nr) {
        const int64_t pi = part.idx(b, h, p.n_kv_heads, rows, r0 + r, s);
        part.o[pi * D + pd] = o[i];
      }
    }
  }
  if (tid < nr) {
    const int64_t pi = part.idx(b, h, p.n_kv_heads, rows, r0 + tid, s);
    part.m[pi] = m_s[tid];
    part.l[pi] = l_s[tid];
  }
}

// ------------------------------------------------------------- recent ------
template <typename TR>
__global__ __launch_bounds__(kAttnThreads) void attn_recent_kernel(smaq_attn_params p, Partials part,
                                                                   int s_base, int64_t split_len,
                                                                   int row_tiles) {
  __shared__ float qs[kRowTile][kMaxHeadDim];
  __shared__ float sc[kRowTile][kChunk];
  __shared__ float m_s[kRowTile], l_s[kRowTile], alpha_s[kRowTile];
  __shared__ long long qpos[kRowTile];
  // keys of one chunk, transposed ([dim][token], row pitch kChunk + 1 so
  // that both the staging writes and the score reads are free of bank
  // conflicts), for head_dim <= kStagedDim: the score loop then reads LDS
  // instead of one 2- or 4-byte global load per dim from a different row
  // in every lane
  constexpr int kStagedDim = 128;
  constexpr int kKT = kChunk + 1;
  __shared__ float kT[kStagedDim * kKT];

  const int D = p.head_dim;
  const bool staged = D <= kStagedDim;
  const int g = p.n_q_heads / p.n_kv_heads;
  const int rows = p.q_len * g;
  const int s = blockIdx.x;
  const int h = blockIdx.y / row_tiles;
  const int rt = blockIdx.y - h * row_tiles;
  const int b = blockIdx.z;
  const int r0 = rt * kRowTile;
  const int nr = min(kRowTile, rows - r0);
  const int tid = threadIdx.x;
  const int64_t len = p.recent_len ? min((int64_t)p.recent_len[b], (int64_t)p.max_recent_len) : p.max_recent_len;
  const int64_t t0 = (int64_t)s * split_len;
  const int64_t t1 = min(len, t0 + split_len);
  const TR* rk = (const TR*)p.recent_k + (int64_t)b * p.recent_batch_stride;
  const TR* rv = (const TR*)p.recent_v + (int64_t)b * p.recent_batch_stride;
  const int64_t tstride = (int64_t)p.n_kv_heads * D;

  for (int i = tid; i < nr * D; i += kAttnThreads) {
    const int r = i / D, d = i - r * D;
    const int row = r0 + r, t = row / g, j = row - t * g;
    qs[r][d] = exact_query(p, (((int64_t)b * p.q_len + t) * p.n_q_heads + h * g + j) * D + d);
  }
  if (tid < nr) {
    m_s[tid] = -__builtin_inff();
    l_s[tid] = 0.0f;
    const int t = (r0 + tid) / g;
    qpos[tid] = p.q_positions ? p.q_positions[(int64_t)b * p.q_len + t] : 0;
  }
  const int prs = kAttnThreads / D;
  const int pd = tid % D, pr0 = tid / D;
  float o[kRowTile];
#pragma unroll
  for (int i = 0; i < kRowTile; ++i) o[i] = 0.0f;
  const int st = tid % kChunk, sr0 = tid / kChunk;
  __syncthreads();

  for (int64_t c0 = t0; c0 < t1; c0 += kChunk) {
    const int64_t t = c0 + st;
    const bool valid = t < t1;
    if (staged) {
      // coalesced row reads (consecutive dims in consecutive lanes); the
      // previous chunk's readers passed the barrier at the loop end
      const int nt = (int)min((int64_t)kChunk, t1 - c0);
      const int per = kAttnThreads / D, d = tid % D;  // D divides kAttnThreads
      const TR* kc = rk + c0 * tstride + (int64_t)h * D + d;
#pragma unroll 8
      for (int tk = tid / D; tk < nt; tk += per) kT[d * kKT + tk] = Num<TR>::to_f(kc[tk * tstride]);
      __syncthreads();
    }
    float acc[kRowTile / 4];
#pragma unroll
    for (int i = 0; i < kRowTile / 4; ++i) acc[i] = 0.0f;
    if (valid && staged) {
      for (int d = 0; d < D; ++d) {
        const float kv = kT[d * kKT + st];
#pragma unroll
        for (int i = 0; i < kRowTile / 4; ++i) {
          const int r = sr0 + 4 * i;
          if (r < nr) acc[i] = fmaf(qs[r][d], kv, acc[i]);
        }
      }
    } else if (valid) {
      const TR* kr = rk + t * tstride + (int64_t)h * D;
      for (int d = 0; d < D; ++d) {
        const float kv = Num<TR>::to_f(kr[d]);
#pragma unroll
        for (int i = 0; i < kRowTile / 4; ++i) {
          const int r = sr0 + 4 * i;
          if (r < nr) acc[i] = fmaf(qs[r][d], kv, acc[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kRowTile / 4; ++i) {
      const int r = sr0 + 4 * i;
      if (r < nr) {
        float sv = valid ? acc[i] * p.scale : -__builtin_inff();
        if (p.q_positions && valid && p.recent_pos_offset + t > qpos[r]) sv = -__builtin_inff();
        sc[r][st] = sv;
      }
    }
    __syncthreads();
    softmax_chunk(sc, m_s, l_s, alpha_s, nr);
    __syncthreads();
    const int nt = (int)min((int64_t)kChunk, t1 - c0);
#pragma unroll
    for (int i = 0; i < kRowTile; ++i) {
      const int r = pr0 + i * prs;
      if (i * prs < kRowTile && r < nr && pr0 < prs) o[i] *= alpha_s[r];
    }
    if (staged) {
      // the chunk's values, laid over the keys' stage ([token][dim]): all of
      // a thread's loads are issued before the first use (one memory round
      // trip, not one per token)
      const int per = kAttnThreads / D, d = tid % D;
      const TR* vc = rv + c0 * tstride + (int64_t)h * D + d;
#pragma unroll 8
      for (int tk = tid / D; tk < nt; tk += per) kT[tk * D + d] = Num<TR>::to_f(vc[tk * tstride]);
      __syncthreads();
      if (pr0 < prs) {
        for (int k = 0; k < nt; ++k) {
          const float vv = kT[k * D + pd];
#pragma unroll
          for (int i = 0; i < kRowTile; ++i) {
            const int r = pr0 + i * prs;
            if (i * prs < kRowTile && r < nr) o[i] = fmaf(sc[r][k], vv, o[i]);
          }
        }
      }
    } else if (pr0 < prs) {
      for (int k = 0; k < nt; ++k) {
        const float vv = Num<TR>::to_f(rv[(c0 + k) * tstride + (int64_t)h * D + pd]);
#pragma unroll
        for (int i = 0; i < kRowTile; ++i) {
          const int r = pr0 + i * prs;
          if (i * prs < kRowTile && r < nr) o[i] = fmaf(sc[r][k], vv, o[i]);
        }
      }
    }
    __syncthreads();
  }
  if (pr0 < prs) {
#pragma unroll
    for (int i = 0; i < kRowTile; ++i) {
      const int r = pr0 + i * prs;
      if (i * prs < kRowTile && r < nr) {
        const int64_t pi = part.idx(b, h, p.n_kv_heads, rows, r0 + r, s_base + s);
        part.o[pi * D + pd] = o[i];
      }
    }
  }
  if (tid < nr) {
    const int64_t pi = part.idx(b, h, p.n_kv_heads, rows, r0 + tid, s_base + s);
    part.m[pi] = m_s[tid];
    part.l[pi] = l_s[tid];
  }
}

// ----------------------------------------------------------- widen ---------
// x (storage dtype) -> fp32, elementwise.
template <typename T>
__global__ __launch_bounds__(256) void widen_kernel(const T* __restrict__ x, int64_t n, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = Num<T>::to_f(x[i]);
}

// ------------------------------------------------------------ combine ------
// kCombineRows query rows per workgroup (threadIdx.y), one thread per
// output dim (threadIdx.x): fewer, larger workgroups than one per row
constexpr int kCombineRows = 4;

template <typename TO>
__global__ __launch_bounds__(kMaxHeadDim * kCombineRows) void attn_combine_kernel(smaq_attn_params p,
                                                                                  Partials part, int s_hist) {
  const int D = p.head_dim;
  const int g = p.n_q_heads / p.n_kv_heads;
  const int rows = p.q_len * g;
  const int r = blockIdx.x * kCombineRows + threadIdx.y;  // row within the KV head group
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int d = threadIdx.x;
  if (d >= D || r >= rows) return;
  const int64_t base = part.idx(b, h, p.n_kv_heads, rows, r, 0);
  // splits in chunks of 8 whose loads are all issued before any is used (one
  // memory round trip per chunk); a later chunk with a larger maximum rescales
  // the sums.  With up to 8 splits this is the plain two-pass merge.
  float M = -__builtin_inff();
  float L = 0.0f, oh = 0.0f, orc = 0.0f;
  // a partial whose sum is NaN holds a NaN score: the reference's softmax
  // row is then NaN, so the output row is too (the merge below would
  // otherwise drop that partial)
  bool poisoned = false;
  for (int s0 = 0; s0 < part.S; s0 += 8) {
    float mv[8], lv[8], ov[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lv[i] = 0.0f;
      mv[i] = -__builtin_inff();
      ov[i] = 0.0f;
      if (s0 + i < part.S) {  // uniform: loads of splits that exist only
        lv[i] = part.l[base + s0 + i];
        mv[i] = part.m[base + s0 + i];
        ov[i] = part.o[(base + s0 + i) * D + d];
      }
    }
    float Mc = M;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (lv[i] > 0.0f) Mc = fmaxf(Mc, mv[i]);
      poisoned |= lv[i] != lv[i];
    }
    if (Mc > M) {
      const float c = __expf(M - Mc);
      L *= c;
      oh *= c;
      orc *= c;
      M = Mc;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (!(lv[i] > 0.0f)) continue;
      const float w = __expf(mv[i] - M);
      L = fmaf(lv[i], w, L);
      const float v = ov[i] * w;
      if (s0 + i < s_hist) oh += v; else orc += v;
    }
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  oh *= inv;
  orc *= inv;
  float res;
  if (p.has_history && p.has_recent) res = Num<TO>::round(Num<TO>::round(oh) + Num<TO>::round(orc));
  else res = p.has_history ? oh : orc;
  if (poisoned) res = __builtin_nanf("");
  const int t = r / g, j = r - t * g;
  ((TO*)p.out)[(((int64_t)b * p.q_len + t) * p.n_q_heads + h * g + j) * D + d] = Num<TO>::from_f(res);
}

struct Plan {
  int row_tiles;
  int64_t hist_split, recent_split;
  int s_hist, s_recent;
  bool mfma, prefill;
  // matrix-core decode with one workgroup per (sequence, KV head) and
  // per-sequence lengths: dispatch the longest sequences first
  bool longest_first;
  // ... as work items (n_items > 0): the sequences past the first round of
  // workgroup slots run in up to s_hist pieces of about piece_len tokens
  int n_items, first_round;
  int64_t piece_len;
  int64_t hist_lp, recent_lp;  // prefill plane lengths
};

// Longest-first pieces (matrix-core decode, ragged lengths, more sequences
// than one round of workgroup slots holds): the sequences that start after
// the first round run in pieces of about kDecodePiece tokens (at most
// kDecodeMaxPieces, so longer histories take longer pieces), merged by the
// kernel's arrival counters.  In one split per sequence, the long units
// dispatched into the slots that free up last form the end of the launch,
// when most slots are already idle.
#ifndef SMAQ_DECODE_PIECE
#define SMAQ_DECODE_PIECE 4096
#endif
constexpr int64_t kDecodePiece = SMAQ_DECODE_PIECE;
constexpr int kDecodeMaxPieces = 8;

static int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

static Plan make_plan(const smaq_attn_params* p) {
  Plan pl;
  const int g = p->n_q_heads / p->n_kv_heads;
  const int rows = p->q_len * g;
  pl.row_tiles = (rows + kRowTile - 1) / kRowTile;
  pl.mfma = (p->impl == 0 || p->impl == 2) && p->has_history && mfma_decode_supported(*p);
  pl.prefill = (p->impl == 0 || p->impl == 3) && !pl.mfma && prefill_mfma_supported(*p);
  const int64_t units = (int64_t)p->batch * p->n_kv_heads * pl.row_tiles;
  // aim for >= 2048 workgroups over the history
  int64_t want = units >= 2048 ? 1 : (2048 + units - 1) / units;
  int64_t hl = p->has_history ? p->max_hist_len : 0;
  int64_t split = hl > 0 ? (hl + want - 1) / want : kChunk;
  split = ((split + kChunk - 1) / kChunk) * kChunk;
  if (split < 4 * kChunk) split = 4 * kChunk;
  if (pl.mfma) split = mfma_decode_split_len(*p);
  pl.hist_split = split;
  int64_t rl = p->has_recent ? p->max_recent_len : 0;
  pl.recent_split = (!pl.prefill && recent_decode_supported(*p)) ? recent_decode_split_len() : 4 * kChunk;
  pl.hist_lp = pl.recent_lp = 0;
  if (pl.prefill) {
    if (hl > 0) pl.hist_split = prefill_split_len(*p, hl);
    if (rl > 0) pl.recent_split = prefill_split_len(*p, rl);
    pl.hist_lp = prefill_padded_len(hl);
    pl.recent_lp = prefill_padded_len(rl);
  }
  pl.s_hist = hl > 0 ? (int)((hl + pl.hist_split - 1) / pl.hist_split) : 0;
  pl.s_recent = rl > 0 ? (int)((rl + pl.recent_split - 1) / pl.recent_split) : 0;
  // With ragged lengths and a single split per sequence the workgroups differ
  // in length by up to max / min; dispatched in batch order, the long ones
  // that start late leave the GPU mostly idle at the end (measured: 256
  // sequences U[1024, 16384] take 0.46 ms in batch order, 0.40 ms longest
  // first).  More splits instead cost more than they balance: each
  // workgroup's start is a chain of dependent memory round trips.
  pl.longest_first = pl.mfma && p->hist_len != nullptr && pl.s_hist == 1 && p->batch > 1;
  pl.n_items = pl.first_round = 0;
  pl.piece_len = 0;
  const int phases = p->phases ? p->phases : 15;
  if (pl.longest_first && kDecodePiece > 0 && p->arrivals && (pl.s_recent == 0 || (phases & 3) == 3)) {
    const bool wide = p->norm_dtype == SMAQ_F32 || p->val_dtype == SMAQ_F32;
    const int first_round = device_cu_count() * (wide ? 3 : 4) / p->n_kv_heads;
    constexpr int64_t step = kMfmaDecodeStep;
    int64_t piece = (hl + kDecodeMaxPieces - 1) / kDecodeMaxPieces;
    piece = piece < kDecodePiece ? kDecodePiece : piece;
    piece = (piece + step - 1) / step * step;
    const int max_pieces = (int)((hl + piece - 1) / piece);
    // (the items are the decode grid's y dimension, at most 65535)
    const int64_t items = first_round + (int64_t)(p->batch - first_round) * max_pieces;
    if (p->batch > first_round && max_pieces >= 2 && items <= 65535) {
      pl.first_round = first_round;
      pl.piece_len = piece;
      pl.s_hist = max_pieces;
      pl.n_items = (int)items;
    }
  }
  return pl;
}

// Bytes of the longest-first order (int per sequence) or its work items
// (16 bytes each).
static int64_t order_bytes(const smaq_attn_params* p, const Plan& pl) {
  return pl.n_items > 0 ? (int64_t)pl.n_items * 16 : (int64_t)p->batch * (int64_t)sizeof(int);
}

// Bytes of the partials (m, l, o) and the offset of the longest-first order.
static int64_t partial_bytes(const smaq_attn_params* p, const Plan& pl) {
  const int64_t S = pl.s_hist + pl.s_recent;
  const int64_t rows = (int64_t)p->q_len * (p->n_q_heads / p->n_kv_heads);
  const int64_t n = (int64_t)p->batch * p->n_kv_heads * rows * (S > 0 ? S : 1);
  return n * (p->head_dim + 2) * (int64_t)sizeof(float);
}

}  // namespace smaq

using namespace smaq;

extern "C" long long smaq_attn_workspace_bytes(const smaq_attn_params* p) {
  if (!p || p->n_kv_heads <= 0 || p->n_q_heads % p->n_kv_heads) return -1;
  const Plan pl = make_plan(p);
  int64_t bytes = partial_bytes(p, pl);
  if (pl.longest_first) bytes = align256(bytes) + order_bytes(p, pl);
  if (pl.prefill) {
    // tile images, value-lo planes and tile errors of each part
    bytes = align256(bytes) + prefill_planes_bytes(p->batch, p->n_kv_heads, pl.hist_lp) +
            prefill_planes_bytes(p->batch, p->n_kv_heads, pl.recent_lp);
  }
  return bytes;
}

template <int KEY, typename TN, typename TV>
static void launch_hist(const smaq_attn_params& p, const HistAddr& a, const Partials& part,
                        const Plan& pl, hipStream_t st) {
  dim3 grid(pl.s_hist, p.n_kv_heads * pl.row_tiles, p.batch);
  hipLaunchKernelGGL((attn_hist_kernel<KEY, TN, TV>), grid, dim3(kAttnThreads), 0, st, p, a, part,
                     pl.hist_split, pl.row_tiles);
}

template <int KEY, typename TN>
static int dispatch_hist_v(const smaq_attn_params& p, const HistAddr& a, const Partials& part,
                           const Plan& pl, hipStream_t st) {
  switch (p.val_dtype) {
    case SMAQ_F32: launch_hist<KEY, TN, float>(p, a, part, pl, st); return SMAQ_OK;
    case SMAQ_F16: launch_hist<KEY, TN, _Float16>(p, a, part, pl, st); return SMAQ_OK;
    case SMAQ_BF16: launch_hist<KEY, TN, bf16>(p, a, part, pl, st); return SMAQ_OK;
  }
  set_error("smaq_attn_hybrid: unsupported value dtype %d", p.val_dtype);
  return SMAQ_EUNSUPPORTED;
}

extern "C" int smaq_attn_hybrid(const smaq_attn_params* pp, void* stream) {
  SMAQ_REQUIRE(pp, "smaq_attn_hybrid: null params");
  const smaq_attn_params& p = *pp;
  hipStream_t st = (hipStream_t)stream;
  SMAQ_REQUIRE(p.batch > 0 && p.q_len > 0 && p.n_kv_heads > 0 && p.n_q_heads > 0,
               "smaq_attn_hybrid: empty shape");
  SMAQ_REQUIRE(p.n_q_heads % p.n_kv_heads == 0, "smaq_attn_hybrid: Hq %% Hkv != 0");
  SMAQ_REQUIRE(p.head_dim > 0 && p.head_dim <= kMaxHeadDim && kAttnThreads % p.head_dim == 0,
               "smaq_attn_hybrid: head_dim %d unsupported (must divide 256)", p.head_dim);
  SMAQ_REQUIRE(p.batch < 65536 && (int64_t)p.n_kv_heads * ((p.q_len * (p.n_q_heads / p.n_kv_heads) + kRowTile - 1) / kRowTile) < 65536,
               "smaq_attn_hybrid: grid too large");
  SMAQ_REQUIRE(p.out && p.workspace, "smaq_attn_hybrid: null output/workspace");
  SMAQ_REQUIRE(p.has_history || p.has_recent, "smaq_attn_hybrid: nothing to attend");
  if (p.has_history) {
    SMAQ_REQUIRE(p.q_hist && p.key_bytes && p.key_lut && p.val_bytes && p.val_scales && p.val_zeros,
                 "smaq_attn_hybrid: null history pointer");
    if (p.rot_mt) SMAQ_REQUIRE(p.q_raw, "smaq_attn_hybrid: rot_mt without q_raw");
    SMAQ_REQUIRE(p.val_group > 0 && p.head_dim % p.val_group == 0, "smaq_attn_hybrid: bad value group");
    SMAQ_REQUIRE(p.val_bits >= 1 && p.val_bits <= 8, "smaq_attn_hybrid: bad value bits");
    if (p.block_table) SMAQ_REQUIRE(p.block_size > 0 && p.max_blocks > 0, "smaq_attn_hybrid: bad paging");
    if (p.key_format == SMAQ_KEY_SCALAR) {
      SMAQ_REQUIRE(p.key_bits >= 1 && p.key_bits <= 8 && p.key_norms, "smaq_attn_hybrid: bad scalar keys");
    } else {
      SMAQ_REQUIRE(p.key_format == SMAQ_KEY_BLOCKVQ && p.vq_blocks * p.vq_block_dim == p.head_dim &&
                       p.vq_centroids >= 1 && p.vq_centroids <= 256,
                   "smaq_attn_hybrid: bad block-VQ keys");
    }
    SMAQ_REQUIRE(p.max_hist_len > 0, "smaq_attn_hybrid: history without tokens");
  }
  if (p.has_recent) {
    SMAQ_REQUIRE((p.q_exact || p.q_raw) && p.recent_k && p.recent_v && p.max_recent_len > 0,
                 "smaq_attn_hybrid: null recent pointer");
  }
  const Plan pl = make_plan(&p);
  if (p.impl == 2 && !pl.mfma) {
    set_error("smaq_attn_hybrid: the matrix-core decode kernel does not serve this shape");
    return SMAQ_EUNSUPPORTED;
  }
  if (p.impl == 3 && !pl.prefill) {
    set_error("smaq_attn_hybrid: the matrix-core prefill kernel does not serve this shape");
    return SMAQ_EUNSUPPORTED;
  }
  SMAQ_REQUIRE(p.impl >= 0 && p.impl <= 3, "smaq_attn_hybrid: unknown impl %d", p.impl);
  const long long need = smaq_attn_workspace_bytes(&p);
  SMAQ_REQUIRE(p.workspace_bytes >= need, "smaq_attn_hybrid: workspace %lld < %lld bytes",
               p.workspace_bytes, need);
  const int S = pl.s_hist + pl.s_recent;
  const int g = p.n_q_heads / p.n_kv_heads;
  const int64_t rows = (int64_t)p.q_len * g;
  const int64_t n_part = (int64_t)p.batch * p.n_kv_heads * rows * S;
  Partials part;
  part.S = S;
  part.m = (float*)p.workspace;
  part.l = part.m + n_part;
  part.o = part.l + n_part;

  const int phases = p.phases ? p.phases : 15;
  // The matrix-core decode kernel writes the output itself when the history
  // is one split and there is no recent part, or, given arrival counters,
  // merges its several splits itself (its last workgroup per sequence and KV
  // head): no combine launch.
  // (In item mode: the sequences of one piece.)
  const bool direct = pl.mfma && pl.s_recent == 0 && (pl.s_hist == 1 || pl.n_items > 0);
  // With a recent part the decode kernel merges the recent window's partials
  // too; the recent phase then runs first, in the same call.
  const bool merge = pl.mfma && (!direct || pl.n_items > 0) && p.arrivals != nullptr &&
                     (pl.s_recent == 0 || (phases & 3) == 3);
  auto launch_recent = [&]() -> int {
    if (recent_decode_supported(p)) return launch_recent_decode(p, part, pl.s_hist, pl.s_recent, pl.recent_split, st);
    dim3 grid(pl.s_recent, p.n_kv_heads * pl.row_tiles, p.batch);
    switch (p.recent_dtype) {
      case SMAQ_F32: hipLaunchKernelGGL(attn_recent_kernel<float>, grid, dim3(kAttnThreads), 0, st, p, part, pl.s_hist, pl.recent_split, pl.row_tiles); break;
      case SMAQ_F16: hipLaunchKernelGGL(attn_recent_kernel<_Float16>, grid, dim3(kAttnThreads), 0, st, p, part, pl.s_hist, pl.recent_split, pl.row_tiles); break;
      case SMAQ_BF16: hipLaunchKernelGGL(attn_recent_kernel<bf16>, grid, dim3(kAttnThreads), 0, st, p, part, pl.s_hist, pl.recent_split, pl.row_tiles); break;
      default: set_error("smaq_attn_hybrid: unsupported recent dtype %d", p.recent_dtype); return SMAQ_EUNSUPPORTED;
    }
    return launch_status("smaq_attn_hybrid(recent)");
  };
  const bool recent_first = merge && pl.s_recent > 0;
  // The query rotation (given rot_mt) is one launch into q_hist ahead of
  // the history phase (phase 8); when the recent window goes first as well
  // (and has the decode kernel), one launch runs both side by side.
  const bool rotation = p.has_history && p.rot_mt && (phases & 8);
  const bool paired = recent_first && rotation && !pl.prefill && rotate_recent_supported(p);
  if (paired) {
    const int rc = launch_rotate_recent(p, part, pl.s_hist, pl.s_recent, pl.recent_split, st);
    if (rc != SMAQ_OK) return rc;
  } else if (recent_first) {
    const int rc = launch_recent();
    if (rc != SMAQ_OK) return rc;
  }
  // The longest-first schedule (order or work items) of the matrix-core
  // decode kernel, unless phase 16 keeps the one an earlier call built;
  // built in the rotation's launch when the call has one.
  void* sched = pl.longest_first ? (char*)p.workspace + align256(partial_bytes(&p, pl)) : nullptr;
  const bool sched_now = pl.mfma && pl.longest_first && pl.s_hist > 0 && (phases & 1) && !(phases & 16);
  // (c5: the launch takes the rotation's 9.6 us, the step 3.2 us less)
  const bool sched_fused = sched_now && rotation && !paired && rotate_schedule_supported(p);
  if (sched_fused) {
    const int rc = launch_rotate_schedule(p, pl.first_round, pl.s_hist, pl.piece_len, pl.n_items, sched, st);
    if (rc != SMAQ_OK) return rc;
  } else if (rotation && !paired) {
    const int rc = smaq_rotate_rows(p.q_raw, p.q_raw_dtype, (long long)p.batch * p.q_len * p.n_q_heads, p.head_dim,
                                    p.rot_mt, p.rot_scale, (float*)p.q_hist, stream);
    if (rc != SMAQ_OK) return rc;
  }
  if (pl.prefill) {
    char* ws = (char*)p.workspace + align256(n_part * (p.head_dim + 2) * (int64_t)sizeof(float));
    auto planes = [&](int64_t lp) {
      const PrefillPlanes P = prefill_planes_at(ws, p.batch, p.n_kv_heads, lp);
      ws += prefill_planes_bytes(p.batch, p.n_kv_heads, lp);
      return P;
    };
    const PrefillPlanes hp = planes(pl.hist_lp);
    const PrefillPlanes rp = planes(pl.recent_lp);
    if (pl.s_hist > 0 && (phases & 1)) {
      HistAddr a{p.hist_seq_start, p.max_hist_len, p.hist_head_stride, p.block_table, p.max_blocks,
                 p.block_size, p.n_kv_heads};
      int rc = launch_prefill_planes_hist(p, a, hp, st);
      if (rc != SMAQ_OK) return rc;
      const PrefillPart pp{p.q_hist, hp.img, hp.img_lo, hp.err, p.hist_len, p.max_hist_len, hp.Lp, pl.hist_split,
                           p.hist_pos_offset, 0};
      if ((rc = launch_prefill_mfma(p, pp, pl.s_hist, part, st)) != SMAQ_OK) return rc;
    }
    if (pl.s_recent > 0 && (phases & 2)) {
      // the prefill kernel reads the plain query as fp32 rows: with a raw
      // query handed in, the library writes them into q_exact first
      if (p.q_raw) {
        SMAQ_REQUIRE(p.q_exact, "smaq_attn_hybrid: the prefill recent part needs a q_exact buffer");
        const int64_t n = (int64_t)p.batch * p.q_len * p.n_q_heads * p.head_dim;
        const unsigned blocks = (unsigned)((n + 255) / 256);
        switch (p.q_raw_dtype) {
          case SMAQ_F32: hipLaunchKernelGGL(widen_kernel<float>, dim3(blocks), dim3(256), 0, st, (const float*)p.q_raw, n, (float*)p.q_exact); break;
          case SMAQ_F16: hipLaunchKernelGGL(widen_kernel<_Float16>, dim3(blocks), dim3(256), 0, st, (const _Float16*)p.q_raw, n, (float*)p.q_exact); break;
          default: hipLaunchKernelGGL(widen_kernel<bf16>, dim3(blocks), dim3(256), 0, st, (const bf16*)p.q_raw, n, (float*)p.q_exact); break;
        }
        int rc = launch_status("smaq_attn_hybrid(query widen)");
        if (rc != SMAQ_OK) return rc;
      }
      int rc = launch_prefill_planes_recent(p, rp, st);
      if (rc != SMAQ_OK) return rc;
      const PrefillPart pp{p.q_exact, rp.img, rp.img_lo, rp.err, p.recent_len, p.max_recent_len, rp.Lp, pl.recent_split,
                           p.recent_pos_offset, pl.s_hist};
      if ((rc = launch_prefill_mfma(p, pp, pl.s_recent, part, st)) != SMAQ_OK) return rc;
    }
  } else if (pl.s_hist > 0 && (phases & 1)) {
    HistAddr a{p.hist_seq_start, p.max_hist_len, p.hist_head_stride, p.block_table, p.max_blocks,
               p.block_size, p.n_kv_heads};
    a.rows = p.hist_rows > 0 ? p.hist_rows : 0;
    int rc = SMAQ_EUNSUPPORTED;
    if (pl.mfma) {
      int* order = (int*)sched;
      if (sched_now && !sched_fused) {
        rc = pl.n_items > 0
                 ? launch_decode_items(p, pl.first_round, pl.s_hist, pl.piece_len, pl.n_items, order, st)
                 : launch_decode_order(p, order, st);
        if (rc != SMAQ_OK) return rc;
      }
      rc = launch_mfma_decode(p, a, part, pl.s_hist, direct, merge, order, pl.n_items, st);
      if (rc != SMAQ_OK) return rc;
    } else if (p.key_format == SMAQ_KEY_SCALAR) {
      switch (p.norm_dtype) {
        case SMAQ_F32: rc = dispatch_hist_v<SMAQ_KEY_SCALAR, float>(p, a, part, pl, st); break;
        case SMAQ_F16: rc = dispatch_hist_v<SMAQ_KEY_SCALAR, _Float16>(p, a, part, pl, st); break;
        case SMAQ_BF16: rc = dispatch_hist_v<SMAQ_KEY_SCALAR, bf16>(p, a, part, pl, st); break;
        default: set_error("smaq_attn_hybrid: unsupported norm dtype %d", p.norm_dtype);
      }
    } else {
      rc = dispatch_hist_v<SMAQ_KEY_BLOCKVQ, float>(p, a, part, pl, st);
    }
    if (rc != SMAQ_OK) return rc;
    if (!pl.mfma && (rc = launch_status("smaq_attn_hybrid(history)")) != SMAQ_OK) return rc;
  }
  if (!pl.prefill && !recent_first && pl.s_recent > 0 && (phases & 2)) {
    const int rc = launch_recent();
    if (rc != SMAQ_OK) return rc;
  }
  if (!(phases & 4) || direct || merge) return SMAQ_OK;
  dim3 cgrid((unsigned)((rows + kCombineRows - 1) / kCombineRows), p.n_kv_heads, p.batch);
  const dim3 cblock((unsigned)((p.head_dim + 63) / 64 * 64), kCombineRows);  // one thread per output dim
  switch (p.out_dtype) {
    case SMAQ_F32: hipLaunchKernelGGL(attn_combine_kernel<float>, cgrid, cblock, 0, st, p, part, pl.s_hist); break;
    case SMAQ_F16: hipLaunchKernelGGL(attn_combine_kernel<_Float16>, cgrid, cblock, 0, st, p, part, pl.s_hist); break;
    case SMAQ_BF16: hipLaunchKernelGGL(attn_combine_kernel<bf16>, cgrid, cblock, 0, st, p, part, pl.s_hist); break;
    default: set_error("smaq_attn_hybrid: unsupported output dtype %d", p.out_dtype); return SMAQ_EUNSUPPORTED;
  }
  return launch_status("smaq_attn_hybrid(combine)");
}

// ------------------------------------------------ allocation-free variant --
// smaq_attn_hybrid_noalloc runs smaq_attn_hybrid with the workspace taken from
// a file-scope device array instead of the caller's buffer, for callers that
// cannot allocate (code under HIP graph capture, serving loops that forbid
// hipMalloc).  Each GPU holds its own copy of the array for the life of the
// process; the host reaches it only through the address hipGetSymbolAddress
// returns on that device (the array's name in host code is not a device
// address).
#include <mutex>

namespace smaq {

constexpr long long kNoAllocScratchBytes = SMAQ_NOALLOC_SCRATCH_BYTES;
constexpr int kNoAllocMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kNoAllocMaxDevices];

// Device address of `scratch` on the stream's device, looked up once per
// device with that device current.
static int scratch_for_stream(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipStreamGetDevice(st, &dev);
  if (e != hipSuccess) {
    set_error("smaq_attn_hybrid_noalloc: hipStreamGetDevice failed: %s", hipGetErrorString(e));
    return SMAQ_ELAUNCH;
  }
  SMAQ_REQUIRE(dev >= 0 && dev < kNoAllocMaxDevices, "smaq_attn_hybrid_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) != hipSuccess) {
      set_error("smaq_attn_hybrid_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
      return SMAQ_ELAUNCH;
    }
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) {
      set_error("smaq_attn_hybrid_noalloc: hipSetDevice(%d) failed: %s", dev, hipGetErrorString(e));
      return SMAQ_ELAUNCH;
    }
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || ptr == nullptr) {
      set_error("smaq_attn_hybrid_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
      return SMAQ_ELAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SMAQ_OK;
}

}  // namespace smaq

extern "C" int smaq_attn_hybrid_noalloc(const smaq_attn_params* pp, void* stream) {
  SMAQ_REQUIRE(pp, "smaq_attn_hybrid_noalloc: null params");
  const long long need = smaq_attn_workspace_bytes(pp);
  SMAQ_REQUIRE(need >= 0, "smaq_attn_hybrid_noalloc: invalid parameters");
  SMAQ_REQUIRE(need <= smaq::kNoAllocScratchBytes,
               "smaq_attn_hybrid_noalloc: these shapes need %lld bytes of workspace, more than the %lld-byte "
               "built-in scratch; use smaq_attn_hybrid with a caller workspace",
               need, smaq::kNoAllocScratchBytes);
  void* ws = nullptr;
  const int rc = smaq::scratch_for_stream((hipStream_t)stream, &ws);
  if (rc != SMAQ_OK) return rc;
  smaq_attn_params p = *pp;
  p.workspace = ws;
  p.workspace_bytes = smaq::kNoAllocScratchBytes;
  return smaq_attn_hybrid(&p, stream);
}
