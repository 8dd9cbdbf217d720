// Block-VQ key encoder on the gfx950 matrix cores (8-dim blocks, 256
// centroids per block, up to 16 blocks).
//
// Same indices as encode_blockvq_kernel (blockvq_codec.hip), which follows
// the reference's torch-CPU arithmetic (smaq/block_vq.py:216-244):
//   x_e  = sequential fmaf chain over d of k_d * E_b[e][d]
//   d2_c = fmaf chain over e of (-2 x_e) * C_c[e], + |x|^2, + |C_c|^2,
//          clamp_min(0); index = first minimum of sqrt(d2)  (cdist's matmul form)
// Here x is computed the same way (bit for bit).  The 256 distances of a
// (token, block) come from one v_mfma_f32_16x16x32_f16 per 16 centroids, on
// a power-of-two rescaling of the block (sigma_b puts the largest centroid
// component in [2^11, 2^12), far above the f16 subnormal range):
//   y = -2 sigma x split as yh + yl (f16), sigma C split as ch + cl (f16),
//   K slots  [ch . yh | ch . yl | cl . yh | (q_hi, q_lo) . 2^14]
//   with q = |sigma C|^2 / 2^14 split hi/lo, and the accumulator starting at
//   sigma^2 (|x|^2 + delta).
// The dropped cl . yl term and the f16 splits cost at most ~1e-6 of
// S = |x|^2 + max |C|^2 (4.5e-7 on SMAQ-shaped keys against the reference's
// distances), the fp32 sums of 27 terms at most 27 ulps of S (1.6e-6), the
// reference's own rounding ~1.5e-6: each distance is within 4e-6 S of the
// reference's, so the argmin is the reference's whenever the runner-up is more
// than delta = 1.2e-5 S behind the best.  Otherwise (about 1e-3 of the
// (token, block) pairs on SMAQ-shaped keys; a key component beyond
// 2^13 / sigma; a non-finite key) the whole wave recomputes that pair's 256
// distances with the exact chain from the fp32 codebook in global memory and
// takes the reference's argmin and tie count.
//
// Layout: one persistent workgroup of 16 waves per CU holds the split
// codebook in LDS (16-byte rows, conflict-free ds_read_b128); each wave
// encodes 16 tokens at a time, block after block, with the next block's key
// bytes in flight.  The running minimum keeps the distance bits with the low
// 6 bits replaced by the centroid's position in the lane (tile, row), so one
// v_min3_u32 tracks value and index of two distances (distances are positive:
// delta is added to every one) and a v_med3_u32 / v_min_u32 pair the runner-up.
#include "encode_internal.h"

namespace smaq {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kVmWaves = 16;                  // waves per workgroup (4 per SIMD)
constexpr int kVmThreads = 64 * kVmWaves;
constexpr int kVmNc = 256;                    // centroids per block
constexpr int kVmBd = 8;                      // block dim
constexpr int kVmMaxBlocks = 16;
constexpr float kDeltaRel = 1.2e-5f;
constexpr float kYMax = 16384.0f;             // |y| bound (f16 operands, their hi parts rounded)
constexpr float kQScale = 16384.0f;           // 2^14: |sigma C|^2 is stored divided by this

// LDS map (bytes) for nb blocks
struct VmLds {
  int nb;
  __host__ __device__ int nq() const { return (nb + 3) / 4; }
  __host__ __device__ size_t ch() const { return 0; }                                  // [nb][256] x 16 B
  __host__ __device__ size_t cl() const { return (size_t)nb * kVmNc * 16; }            // [nb][256] x 16 B
  __host__ __device__ size_t cq() const { return 2 * (size_t)nb * kVmNc * 16; }        // [nq][256] x 16 B
  __host__ __device__ size_t bq() const { return cq() + (size_t)nq() * kVmNc * 16; }   // [4] x 16 B
  __host__ __device__ size_t ys() const { return bq() + 64; }                          // [16 waves][16] x 32 B
  __host__ __device__ size_t es() const { return ys() + (size_t)kVmWaves * 16 * 32; }  // [nb][64] f32
  __host__ __device__ size_t sig() const { return es() + (size_t)nb * 64 * 4; }        // [nb] f32
  __host__ __device__ size_t smax() const { return sig() + (size_t)nb * 4; }           // [nb] f32
  __host__ __device__ size_t bytes() const { return smax() + (size_t)nb * 4; }
};

__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bitsf(uint32_t b) { return __builtin_bit_cast(float, b); }
__device__ __forceinline__ uint32_t h16(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }

// Two keys k0, k1 at a time: with best <= second, the new minimum is
// min3(best, k0, k1) and the new runner-up min(second, med3(best, k0, k1))
// (the overall minimum lies in {best, k0, k1}, so the second smallest of the
// four is the smaller of `second` and the middle of those three).
__device__ __forceinline__ uint32_t med3_u32(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ uint32_t min3_u32(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_min3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// The lanes l ^ 16 (X16) and l ^ 32 (X32) as VALU permutes: with both
// operands x, v_permlane16_swap / v_permlane32_swap leave each lane the pair
// {x[l], x[l ^ 16]} / {x[l], x[l ^ 32]} (in some order), which is all a
// symmetric reduction (min, sum) needs -- no LDS round trip.
struct LanePair {
  uint32_t a, b;
};
__device__ __forceinline__ LanePair pair_x16(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  return {r[0], r[1]};
}
__device__ __forceinline__ LanePair pair_x32(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return {r[0], r[1]};
}
// (x[l] + x[l ^ 16]) + (x[l ^ 32] + x[l ^ 48]): the same value, bit for bit,
// in all four lanes of a token (fp32 addition commutes)
__device__ __forceinline__ float sum_kgroups(float x) {
  const LanePair p = pair_x16(fbits(x));
  const float s = bitsf(p.a) + bitsf(p.b);
  const LanePair q = pair_x32(fbits(s));
  return bitsf(q.a) + bitsf(q.b);
}

// Orders this wave's LDS writes before its later LDS reads of other lanes'
// data (a wave-local exchange).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One token's 8-value key block, kept as loaded (16 or 32 bytes).
template <typename T>
struct KeyBlock {
  static constexpr int kWords = sizeof(T) == 2 ? 4 : 8;
  u32x4 w[kWords / 4];
  __device__ __forceinline__ void load(const T* p) {
    w[0] = *(const u32x4*)p;
    if constexpr (sizeof(T) == 4) w[1] = *(const u32x4*)(p + 4);
  }
  __device__ __forceinline__ void unpack(float* out) const {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[2 * i] = Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)w[0][i]));
        out[2 * i + 1] = Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(w[0][i] >> 16)));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[i] = bitsf(w[0][i]);
        out[4 + i] = bitsf(w[1][i]);
      }
    }
  }
};

// Exact distances of one (token, block) by the whole wave (4 centroids per
// lane, read from the fp32 codebook Cb = C[b] in global memory) and the
// reference's choice: first index of the smallest sqrt(d2), with NaN winning
// at its first index; `tie` when another centroid is within 2e-6 relative of
// the smallest d2.
__device__ int exact_argmin(const float* x, float xsq, const float* __restrict__ Cb, int lane, bool* tie) {
  uint64_t key = ~0ull;
  float dmin = __builtin_inff();
  float d2v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    float ce[kVmBd];
#pragma unroll
    for (int e = 0; e < kVmBd; ++e) ce[e] = Cb[c * kVmBd + e];
    float a = 0.0f, csq = 0.0f;
#pragma unroll
    for (int e = 0; e < kVmBd; ++e) {
      a = fmaf(-2.0f * x[e], ce[e], a);
      csq = csq + ce[e] * ce[e];  // x.pow(2).sum(-1) order
    }
    a = a + xsq;
    a = a + csq;
    a = a < 0.0f ? 0.0f : a;  // clamp_min(0); NaN passes
    d2v[j] = a;
    const bool nan = a != a;
    const uint64_t s = nan ? 0ull : (uint64_t)fbits(sqrtf(a)) + 1ull;
    const uint64_t kk = (s << 32) | (uint64_t)c;
    key = kk < key ? kk : key;
    dmin = nan ? dmin : fminf(dmin, a);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(key >> 32), off, 64) << 32) |
                       (uint32_t)__shfl_xor((int)(uint32_t)key, off, 64);
    key = o < key ? o : key;
    dmin = fminf(dmin, __shfl_xor(dmin, off, 64));
  }
  int near = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) near += (d2v[j] <= dmin * (1.0f + 2e-6f)) ? 1 : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) near += __shfl_xor(near, off, 64);
  const bool any_nan = (key >> 32) == 0;
  *tie = !any_nan && near >= 2;
  return (int)(uint32_t)key;
}

template <typename T>
__global__ __launch_bounds__(kVmThreads) void encode_blockvq_mfma_kernel(
    const T* __restrict__ k, RowMap map, int64_t rows, int nb, const float* __restrict__ E_blocks,
    const float* __restrict__ C, uint8_t* __restrict__ idx_out, unsigned long long* tie_count) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const VmLds L{nb};
  float* const es_all = (float*)(lds + L.es());
  float* const sig_all = (float*)(lds + L.sig());
  float* const smax_all = (float*)(lds + L.smax());
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;

  // ---- per block: sigma_b (a power of two putting max |C| in [2^11, 2^12))
  // and max |C|^2; one wave per block
  for (int b = w; b < nb; b += kVmWaves) {
    float amax = 0.0f, smax = 0.0f;
    for (int c = lane; c < kVmNc; c += 64) {
      const float* cc = C + ((int64_t)b * kVmNc + c) * kVmBd;
      float s = 0.0f;
      for (int e = 0; e < kVmBd; ++e) {
        amax = __builtin_elementwise_maximum(amax, fabsf(cc[e]));  // a NaN is kept
        s = s + cc[e] * cc[e];
      }
      smax = fmaxf(smax, s);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      amax = __builtin_elementwise_maximum(amax, __shfl_xor(amax, off, 64));
      smax = fmaxf(smax, __shfl_xor(smax, off, 64));
    }
    if (lane == 0) {
      // a block with a non-finite centroid (the reference's argmin then
      // follows NaN distances) or outside a sane range sends every token to
      // the exact path: a NaN sigma makes every distance NaN
      const bool finite = amax < 3.0e38f;  // false for inf and NaN
      int e = 0;
      if (finite && amax > 0.0f) frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
      sig_all[b] = (finite && e > -100 && e < 100) ? ldexpf(1.0f, 12 - e) : __builtin_nanf("");
      smax_all[b] = smax;
    }
  }
  for (int i = tid; i < nb * 64; i += kVmThreads) es_all[i] = E_blocks[i];
  if (tid < 16) {  // |C|^2 slot operands: row r holds 2^14 in halves 2r, 2r+1
    const int r = tid >> 2, dw = tid & 3;
    ((uint32_t*)(lds + L.bq()))[tid] = dw == r ? 0x74007400u : 0u;
  }
  __syncthreads();
  // ---- split codebook: ch / cl rows of sigma C, q = |sigma C|^2 / 2^14 split
  for (int i = tid; i < L.nq() * 4 * kVmNc; i += kVmThreads) {
    const int c = i % kVmNc, b = i / kVmNc;  // q row b / 4, dword b % 4
    uint32_t qw = 0u;
    if (b < nb) {
      const float sg = sig_all[b];
      const float* cc = C + ((int64_t)b * kVmNc + c) * kVmBd;
      // dims in K-slot order [0, 4, 1, 5, 2, 6, 3, 7]: slots 2i, 2i + 1 hold
      // dims i, i + 4, the two shaped-key dims one k-group lane computes
      uint32_t hw[4], lw[4];
      float q = 0.0f;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float v0 = cc[d] * sg, v1 = cc[d + 4] * sg;
        const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
        const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
        hw[d] = h16(h0) | (h16(h1) << 16);
        lw[d] = h16(l0) | (h16(l1) << 16);
        q = fmaf(v0, v0, q);
        q = fmaf(v1, v1, q);
      }
      *(u32x4*)(lds + L.ch() + ((size_t)b * kVmNc + c) * 16) = u32x4{hw[0], hw[1], hw[2], hw[3]};
      *(u32x4*)(lds + L.cl() + ((size_t)b * kVmNc + c) * 16) = u32x4{lw[0], lw[1], lw[2], lw[3]};
      const float qs = q * (1.0f / kQScale);
      const _Float16 qh = (_Float16)qs, ql = (_Float16)(qs - (float)qh);
      qw = sg == sg ? (h16(qh) | (h16(ql) << 16)) : 0u;
    }
    ((uint32_t*)(lds + L.cq()))[((size_t)(b >> 2) * kVmNc + c) * 4 + (b & 3)] = qw;
  }
  __syncthreads();

  const int n = lane & 15, kg = lane >> 4;  // MFMA coordinates: token / centroid row n, k-group kg
  // LDS addressing in 32 bits
  typedef __attribute__((address_space(3))) uint8_t LdsByte;
  typedef const __attribute__((address_space(3))) u32x4 LdsU32x4;
  typedef const __attribute__((address_space(3))) f32x4 LdsF32x4;
  LdsByte* const lds3 = (LdsByte*)lds;
  // this lane's token: y hi [8] | y lo [8] in K-slot order; the lane owns
  // slots 2kg, 2kg + 1 of each half
  const uint32_t ys_tok = (uint32_t)(L.ys() + (size_t)w * 16 * 32 + n * 32);
  // B operand source (k-group 0 / 2: y hi, 1: y lo, 3: the |C|^2 pair row)
  const uint32_t b_src = kg == 3 ? (uint32_t)L.bq() : ys_tok + (kg == 1 ? 16u : 0u);
  // A rows: centroid 16t + n; k-group 0 / 1 read ch, 2 reads cl, 3 the q row
  const uint32_t a_src = kg < 2 ? (uint32_t)(L.ch() + n * 16) : (kg == 2 ? (uint32_t)(L.cl() + n * 16) : (uint32_t)(L.cq() + n * 16));
  const uint32_t a_blk = kg < 3 ? (uint32_t)(kVmNc * 16) : 0u;  // A bytes per block (q rows: per 4 blocks)
  unsigned ties = 0;
  const int64_t n_tiles = (rows + 15) / 16;
  const int64_t stride = (int64_t)gridDim.x * kVmWaves;
  int64_t tile = (int64_t)blockIdx.x * kVmWaves + w;
  auto key_row = [&](int64_t t) -> const T* {
    const int64_t row = t * 16 + n;
    return k + map.offset(row < rows ? row : rows - 1);
  };
  // (key_row clamps past-the-end rows, so the prefetch past the last tile
  // reads a valid row)
  const T* kr = key_row(tile);
  KeyBlock<T> next;
  next.load(kr);
  for (; tile < n_tiles; tile += stride) {
    const int64_t row = tile * 16 + n;
    const bool valid = row < rows;
    uint8_t* const out = idx_out + map.out_row(valid ? row : 0) * nb;
    const T* const kr_next = key_row(tile + stride);
    for (int b = 0; b < nb; ++b) {
      float kv[kVmBd];
      next.unpack(kv);
      // the next key block of this lane's token (or the next tile's first)
      next.load(b + 1 < nb ? kr + (b + 1) * kVmBd : kr_next);
      // rows kg and kg + 4 of E_b, 16-byte reads
      const LdsF32x4* er = (const LdsF32x4*)(lds3 + L.es() + (size_t)b * 256 + kg * 32);
      const f32x4 ea0 = er[0], ea1 = er[1], eb0 = er[8], eb1 = er[9];  // row kg + 4: 128 bytes on
      const float ea[kVmBd] = {ea0[0], ea0[1], ea0[2], ea0[3], ea1[0], ea1[1], ea1[2], ea1[3]};
      const float eb[kVmBd] = {eb0[0], eb0[1], eb0[2], eb0[3], eb1[0], eb1[1], eb1[2], eb1[3]};
      // x_kg and x_{kg+4}: the reference's chain, bit for bit
      float xa = 0.0f, xb = 0.0f;
#pragma unroll
      for (int d = 0; d < kVmBd; ++d) {
        xa = fmaf(kv[d], ea[d], xa);
        xb = fmaf(kv[d], eb[d], xb);
      }
      const float sg = sig_all[b];
      const float ya = xa * (-2.0f * sg), yb = xb * (-2.0f * sg);  // exact (powers of two)
      const bool ok = fabsf(ya) < kYMax && fabsf(yb) < kYMax;     // false for NaN
      const _Float16 yah = (_Float16)ya, ybh = (_Float16)yb;
      const _Float16 yal = (_Float16)(ya - (float)yah), ybl = (_Float16)(yb - (float)ybh);
      *(__attribute__((address_space(3))) uint32_t*)(lds3 + ys_tok + 4 * kg) = h16(yah) | (h16(ybh) << 16);
      *(__attribute__((address_space(3))) uint32_t*)(lds3 + ys_tok + 16 + 4 * kg) = h16(yal) | (h16(ybl) << 16);
      float sq = ok ? xa * xa + xb * xb : __builtin_nanf("");
      sq = sum_kgroups(sq);
      const float delta = kDeltaRel * (sq + smax_all[b]);
      const float s2 = sg * sg;
      const float init = (sq + delta) * s2;  // |x|^2 + delta, scaled
      const float delta_s = delta * s2;
      wave_sync();
      // B: k-group 0 / 2 take y hi, 1 takes y lo, 3 the 2^14 pair of block b
      const f16x8 bv = __builtin_bit_cast(
          f16x8, *(LdsU32x4*)(lds3 + b_src + (kg == 3 ? (uint32_t)(b & 3) * 16u : 0u)));
      const LdsU32x4* ap =
          (LdsU32x4*)(lds3 + a_src + (kg < 3 ? (uint32_t)b * a_blk : (uint32_t)(b >> 2) * (uint32_t)(kVmNc * 16)));
      const f32x4 acc0 = {init, init, init, init};
      uint32_t best = 0xffffffffu, second = 0xffffffffu;
      // software pipelined: the product of tile t + 1 is issued before the
      // keys of tile t are reduced, and the A operand of tile t + 3 is read
      // then (two tiles of LDS latency covered)
      u32x4 a_n1 = ap[16], a_n2 = ap[32];
      f32x4 acc_next = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ap[0]), bv, acc0, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const f32x4 acc = acc_next;
        if (t + 1 < 16) {
          acc_next = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a_n1), bv, acc0, 0, 0, 0);
          a_n1 = a_n2;
          if (t + 3 < 16) a_n2 = ap[16 * (t + 3)];
        }
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          // centroids 16t + 4kg + i, i + 1 of token n; low 6 bits = (t, i)
          const uint32_t k0 = (fbits(acc[i]) & 0xffffffc0u) | (uint32_t)(4 * t + i);
          const uint32_t k1 = (fbits(acc[i + 1]) & 0xffffffc0u) | (uint32_t)(4 * t + i + 1);
          second = min(second, med3_u32(best, k0, k1));
          best = min3_u32(best, k0, k1);
        }
      }
      // merge the four k-group lanes of each token
      uint32_t gbest = best, gsecond = second;
#pragma unroll
      for (int step = 0; step < 2; ++step) {  // lanes l ^ 16, then l ^ 32
        const LanePair pb = step == 0 ? pair_x16(gbest) : pair_x32(gbest);
        const LanePair ps = step == 0 ? pair_x16(gsecond) : pair_x32(gsecond);
        gsecond = min3_u32(ps.a, ps.b, max(pb.a, pb.b));
        gbest = min(pb.a, pb.b);
      }
      const float vb = bitsf(gbest & 0xffffffc0u), vs = bitsf(gsecond & 0xffffffc0u);
      // clear winner: the runner-up more than delta behind (keys are
      // truncated by at most 2^-17 relative); distances positive and finite
      const bool clear = (vs - vb * (1.0f + 0x1p-16f) > delta_s) && vb > 0.0f && vb < 3.0e38f &&
                         delta_s < 3.0e38f;
      const int kw = best == gbest ? kg : 4;  // the lane holding the winner
      int kwin = kw;
      {
        const LanePair p = pair_x16((uint32_t)kwin);
        const LanePair q = pair_x32(min(p.a, p.b));
        kwin = (int)min(q.a, q.b);
      }
      const int tag = (int)(gbest & 63u);
      int idx = 16 * (tag >> 2) + 4 * kwin + (tag & 3);
      // exact recount of the unclear tokens, one at a time by the whole wave
      uint64_t todo = __ballot(!clear && valid && kg == 0);
      while (todo) {
        const int t0 = __builtin_ctzll(todo);
        todo &= todo - 1;
        float x[kVmBd];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] = __shfl(xa, t0 + 16 * e, 64);
          x[e + 4] = __shfl(xb, t0 + 16 * e, 64);
        }
        float xsq = 0.0f;
#pragma unroll
        for (int e = 0; e < kVmBd; ++e) xsq = xsq + x[e] * x[e];  // x.pow(2).sum(-1) order
        bool tie;
        const int ci = exact_argmin(x, xsq, C + (int64_t)b * kVmNc * kVmBd, lane, &tie);
        if (n == t0) idx = ci;
        if (lane == t0) ties += tie ? 1u : 0u;
      }
      if (valid && kg == 0) out[b] = (uint8_t)idx;
    }
    kr = kr_next;
  }
  add_count(tie_count, ties);
}

}  // namespace

bool encode_blockvq_mfma_supported(int nb, int bd, int nc, const void* k, int kdtype,
                                   long long s_outer, long long s_inner) {
  const int esz = kdtype == SMAQ_F32 ? 4 : 2;
  return bd == kVmBd && nc == kVmNc && nb >= 1 && nb <= kVmMaxBlocks &&
         // 16-byte loads of each 8-value block
         (((uintptr_t)k | (uintptr_t)(s_outer * esz) | (uintptr_t)(s_inner * esz)) & 15) == 0;
}

size_t encode_blockvq_mfma_lds(int nb) {
  return VmLds{nb}.bytes();
}

int launch_encode_blockvq_mfma(int kdtype, const void* k, RowMap map, int64_t rows, int nb,
                               const float* E_blocks, const float* C, uint8_t* idx,
                               unsigned long long* ties, hipStream_t st) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t n_tiles = (rows + 15) / 16;
  const int64_t want = (n_tiles + kVmWaves - 1) / kVmWaves;
  const unsigned grid = (unsigned)(want < cus ? want : cus);
  const size_t lds = encode_blockvq_mfma_lds(nb);
  // the split codebook takes more than the default 64 KB of dynamic LDS
  switch (kdtype) {
    case SMAQ_F32:
      hipFuncSetAttribute((const void*)encode_blockvq_mfma_kernel<float>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      break;
    case SMAQ_F16:
      hipFuncSetAttribute((const void*)encode_blockvq_mfma_kernel<_Float16>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      break;
    default:
      hipFuncSetAttribute((const void*)encode_blockvq_mfma_kernel<bf16>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      break;
  }
  switch (kdtype) {
    case SMAQ_F32:
      hipLaunchKernelGGL(encode_blockvq_mfma_kernel<float>, dim3(grid), dim3(kVmThreads), lds, st,
                         (const float*)k, map, rows, nb, E_blocks, C, idx, ties);
      break;
    case SMAQ_F16:
      hipLaunchKernelGGL(encode_blockvq_mfma_kernel<_Float16>, dim3(grid), dim3(kVmThreads), lds, st,
                         (const _Float16*)k, map, rows, nb, E_blocks, C, idx, ties);
      break;
    default:
      hipLaunchKernelGGL(encode_blockvq_mfma_kernel<bf16>, dim3(grid), dim3(kVmThreads), lds, st,
                         (const bf16*)k, map, rows, nb, E_blocks, C, idx, ties);
      break;
  }
  return launch_status("smaq_encode_blockvq(mfma)");
}

}  // namespace smaq
