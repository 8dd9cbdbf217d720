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
// codebook in LDS (16-byte rows, conflict-free ds_read_b128).  A wave encodes
// sets of 64 tokens, block after block: the set's four groups of 16 tokens
// are the columns of four MFMA products per codebook tile, which share the
// tile's one LDS read, and the key blocks of the next block are in flight
// meanwhile.  Each lane keeps, per
// group, the running minimum of its 64 distances as the distance bits with
// the low 8 bits replaced by the centroid's position in the lane (tile, row),
// so one v_min3_u32 tracks value and index of two distances (distances are
// positive: delta is added to every one) and a v_med3_u32 / v_min_u32 pair the
// runner-up.  The four k-group lanes of every token are then merged by
// v_permlane32_swap / v_permlane16_swap reduce-scatters (the k-group goes into
// tag bits 7:6), leaving token l of the set in lane l for the clear test, the
// index, the store and the exact recount.
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

// Cross-row exchanges without LDS.  A set of 64 tokens in MFMA layout: value
// v[g] of lane (row r, column n) belongs to token (g, n), k-group r.  With
// operands x, y,
// v_permlane32_swap leaves {x rows 0-1 | y rows 0-1} and {x rows 2-3 | y
// rows 2-3}, and v_permlane16_swap {x r0, y r0, x r2, y r2} and {x r1, y r1,
// x r3, y r3}: swapping groups (0, 2) and (1, 3) across the halves, then the
// two results across row pairs, hands lane (r, n) the four k-group values of
// token (r, n).
//
// Sum over the four k-groups of token (r, n), delivered to lane (r, n):
// (v[kg 0] + v[kg 2]) + (v[kg 1] + v[kg 3]).
__device__ __forceinline__ float reduce_scatter_kgroups(const float* v) {
  const auto p = __builtin_amdgcn_permlane32_swap(fbits(v[0]), fbits(v[2]), false, false);
  const auto q = __builtin_amdgcn_permlane32_swap(fbits(v[1]), fbits(v[3]), false, false);
  const float s02 = bitsf(p[0]) + bitsf(p[1]);  // rows 0-1: token (0, n), rows 2-3: (2, n)
  const float s13 = bitsf(q[0]) + bitsf(q[1]);  // rows 0-1: token (1, n), rows 2-3: (3, n)
  const auto r = __builtin_amdgcn_permlane16_swap(fbits(s02), fbits(s13), false, false);
  return bitsf(r[0]) + bitsf(r[1]);
}
// The inverse direction: x of lane (r, n) belongs to token (r, n); every lane
// of column n receives out[g] = x of token (g, n).
__device__ __forceinline__ void all_gather_kgroups(float x, float* out) {
  const auto a = __builtin_amdgcn_permlane16_swap(fbits(x), fbits(x), false, false);
  // a[0]: token (0, n) on rows 0-1, (2, n) on rows 2-3; a[1]: (1, n) / (3, n)
  const auto c0 = __builtin_amdgcn_permlane32_swap(a[0], a[0], false, false);
  const auto c1 = __builtin_amdgcn_permlane32_swap(a[1], a[1], false, false);
  out[0] = bitsf(c0[0]);
  out[1] = bitsf(c1[0]);
  out[2] = bitsf(c0[1]);
  out[3] = bitsf(c1[1]);
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
  // A wave encodes sets of 64 tokens.  Group g (0..3) of a set is its tokens
  // 16g + n, one MFMA column n each; the four groups share every codebook
  // tile (one A read feeds four products).  The k-group partial results are
  // then reduce-scattered so that lane l holds token l of the set, and the
  // per-token tail (clear test, index, store, exact recount) runs once per
  // token instead of once per k-group lane.
  const int64_t n_sets = (rows + 63) / 64;
  const int64_t stride = (int64_t)gridDim.x * kVmWaves;
  int64_t set = (int64_t)blockIdx.x * kVmWaves + w;
  auto key_row = [&](int64_t s, int g) -> const T* {
    const int64_t row = s * 64 + 16 * g + n;
    return k + map.offset(row < rows ? row : rows - 1);
  };
  // (key_row clamps past-the-end rows, so the prefetch past the last set
  // reads a valid row)
  const T* kp[4];
  KeyBlock<T> kb[4];  // this group's token: the key block in flight
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    kp[g] = key_row(set, g);
    kb[g].load(kp[g]);
  }
  const uint32_t kg_tag = (uint32_t)kg << 6;
  for (; set < n_sets; set += stride) {
    const int64_t row = set * 64 + lane;  // the token this lane finishes
    const bool valid = row < rows;
    uint8_t* const out = idx_out + map.out_row(valid ? row : 0) * nb;
    // the token's indices, byte b in word b / 4, stored together after the
    // last block (one store per block and token leaves 16 partial writes of
    // a row to reach HBM separately once the set's rows fall out of L2)
    uint32_t ob[kVmMaxBlocks / 4] = {0u, 0u, 0u, 0u};
    for (int b = 0; b < nb; ++b) {
      // rows kg and kg + 4 of E_b, 16-byte reads
      const LdsF32x4* er = (const LdsF32x4*)(lds3 + L.es() + (size_t)b * 256 + kg * 32);
      const f32x4 ea0 = er[0], ea1 = er[1], eb0 = er[8], eb1 = er[9];  // row kg + 4: 128 bytes on
      const float ea[kVmBd] = {ea0[0], ea0[1], ea0[2], ea0[3], ea1[0], ea1[1], ea1[2], ea1[3]};
      const float eb[kVmBd] = {eb0[0], eb0[1], eb0[2], eb0[3], eb1[0], eb1[1], eb1[2], eb1[3]};
      const float sg = sig_all[b];
      const float m2s = -2.0f * sg, s2 = sg * sg, smax_b = smax_all[b];
      // ---- the four groups' B operands (staged one group at a time through
      // the wave's 16-token buffer) and C operands sigma^2 (|x|^2 + delta)
      f16x8 bv[4];
      float sqp[4];  // this k-group's part of |x|^2 of token (g, n)
      // the key blocks loaded next: block b + 1 of these tokens, or block 0
      // of the next set's
      const bool last = b + 1 == nb;
      if (last) {
#pragma unroll
        for (int g = 0; g < 4; ++g) kp[g] = key_row(set + stride, g);
      }
      const int next_off = last ? 0 : (b + 1) * kVmBd;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float kv[kVmBd];
        kb[g].unpack(kv);
        kb[g].load(kp[g] + next_off);
        // x_kg and x_{kg+4}: the reference's chain, bit for bit
        float xa = 0.0f, xb = 0.0f;
#pragma unroll
        for (int d = 0; d < kVmBd; ++d) {
          xa = fmaf(kv[d], ea[d], xa);
          xb = fmaf(kv[d], eb[d], xb);
        }
        const float ya = xa * m2s, yb = xb * m2s;                 // exact (powers of two)
        const bool ok = fabsf(ya) < kYMax && fabsf(yb) < kYMax;  // false for NaN
        const _Float16 yah = (_Float16)ya, ybh = (_Float16)yb;
        const _Float16 yal = (_Float16)(ya - (float)yah), ybl = (_Float16)(yb - (float)ybh);
        *(__attribute__((address_space(3))) uint32_t*)(lds3 + ys_tok + 4 * kg) = h16(yah) | (h16(ybh) << 16);
        *(__attribute__((address_space(3))) uint32_t*)(lds3 + ys_tok + 16 + 4 * kg) = h16(yal) | (h16(ybl) << 16);
        sqp[g] = ok ? xa * xa + xb * xb : __builtin_nanf("");
        wave_sync();
        // B: k-group 0 / 2 take y hi, 1 takes y lo, 3 the 2^14 pair of block b
        bv[g] = __builtin_bit_cast(f16x8, *(LdsU32x4*)(lds3 + b_src + (kg == 3 ? (uint32_t)(b & 3) * 16u : 0u)));
        // the next group's staging stores come after this read: a wave's LDS
        // operations execute in order, so only the compiler must keep them so
        asm volatile("" ::: "memory");
      }
      // ---- |x|^2 of token (kg, n) in this lane (the four k-group parts
      // reduce-scattered), delta and the accumulator start sigma^2 (|x|^2 +
      // delta) once per token, then the four groups' starts gathered back
      const float sq = reduce_scatter_kgroups(sqp);
      const float delta = kDeltaRel * (sq + smax_b);
      const float delta_s = delta * s2;
      float init_g[4];
      all_gather_kgroups((sq + delta) * s2, init_g);
      f32x4 cv[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) cv[g] = f32x4{init_g[g], init_g[g], init_g[g], init_g[g]};
      // ---- distances: tile t of 16 centroids for each group, the product of
      // the next (tile, group) issued before the keys of this one are reduced
      const LdsU32x4* ap =
          (LdsU32x4*)(lds3 + a_src + (kg < 3 ? (uint32_t)b * a_blk : (uint32_t)(b >> 2) * (uint32_t)(kVmNc * 16)));
      uint32_t best[4], second[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) best[g] = second[g] = 0xffffffffu;
      u32x4 a_cur = ap[0], a_nxt = ap[16];
      f32x4 acc_next = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a_cur), bv[0], cv[0], 0, 0, 0);
#pragma unroll
      for (int s = 0; s < 64; ++s) {
        const int t = s >> 2, g = s & 3;
        const f32x4 acc = acc_next;
        if (s + 1 < 64) {
          const int t1 = (s + 1) >> 2, g1 = (s + 1) & 3;
          if (g1 == 0) {
            a_cur = a_nxt;
            if (t1 + 1 < 16) a_nxt = ap[16 * (t1 + 1)];
          }
          acc_next = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a_cur), bv[g1], cv[g1], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          // centroids 16t + 4kg + i, i + 1 of token (g, n); low 8 bits =
          // (0, t, i) now, the k-group goes into bits 6-7 below
          const uint32_t k0 = (fbits(acc[i]) & 0xffffff00u) | (uint32_t)(4 * t + i);
          const uint32_t k1 = (fbits(acc[i + 1]) & 0xffffff00u) | (uint32_t)(4 * t + i + 1);
          second[g] = min(second[g], med3_u32(best[g], k0, k1));
          best[g] = min3_u32(best[g], k0, k1);
        }
      }
      // ---- merge the four k-group lanes of every token, leaving token
      // 16r + n (group r, column n) in lane 16r + n: lanes l ^ 32 for the
      // group pairs (0, 2), (1, 3), then lanes l ^ 16.  With best <= second
      // on both sides, the merged runner-up is min(second_a, second_b,
      // max(best_a, best_b)).
#pragma unroll
      for (int g = 0; g < 4; ++g) best[g] |= kg_tag;
      uint32_t mb[2], ms[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const auto pb = __builtin_amdgcn_permlane32_swap(best[h], best[h + 2], false, false);
        const auto ps = __builtin_amdgcn_permlane32_swap(second[h], second[h + 2], false, false);
        mb[h] = min(pb[0], pb[1]);
        ms[h] = min3_u32(ps[0], ps[1], max(pb[0], pb[1]));
      }
      const auto pb = __builtin_amdgcn_permlane16_swap(mb[0], mb[1], false, false);
      const auto ps = __builtin_amdgcn_permlane16_swap(ms[0], ms[1], false, false);
      const uint32_t gbest = min(pb[0], pb[1]);
      const uint32_t gsecond = min3_u32(ps[0], ps[1], max(pb[0], pb[1]));
      const float vb = bitsf(gbest & 0xffffff00u), vs = bitsf(gsecond & 0xffffff00u);
      // clear winner: the runner-up more than delta behind (keys are
      // truncated by less than 2^-15 relative); distances positive and finite
      const bool clear = (vs - vb * (1.0f + 0x1p-14f) > delta_s) && vb > 0.0f && vb < 3.0e38f &&
                         delta_s < 3.0e38f;
      // tag bits: kg (7:6), t (5:2), i (1:0) -> centroid 16t + 4kg + i
      const uint32_t tag = gbest & 0xffu;
      int idx = (int)(((tag & 0x3cu) << 2) | ((tag >> 4) & 0xcu) | (tag & 3u));
      // exact recount of the unclear tokens, one at a time by the whole wave
      uint64_t todo = __ballot(!clear && valid);
      while (todo) {
        const int t0 = __builtin_ctzll(todo);
        todo &= todo - 1;
        // x of token t0 again (the same chain), from its key block
        const int64_t r0 = set * 64 + t0;
        KeyBlock<T> kx;
        kx.load(k + map.offset(r0) + b * kVmBd);
        float kv[kVmBd], x[kVmBd];
        kx.unpack(kv);
        const float* Eb = E_blocks + b * 64;
#pragma unroll
        for (int e = 0; e < kVmBd; ++e) {
          float a = 0.0f;
#pragma unroll
          for (int d = 0; d < kVmBd; ++d) a = fmaf(kv[d], Eb[e * kVmBd + d], a);
          x[e] = a;
        }
        float xsq = 0.0f;
#pragma unroll
        for (int e = 0; e < kVmBd; ++e) xsq = xsq + x[e] * x[e];  // x.pow(2).sum(-1) order
        bool tie;
        const int ci = exact_argmin(x, xsq, C + (int64_t)b * kVmNc * kVmBd, lane, &tie);
        if (lane == t0) {
          idx = ci;
          ties += tie ? 1u : 0u;
        }
      }
      const uint32_t v = (uint32_t)idx << (8 * (b & 3));
      switch (b >> 2) {  // b is wave-uniform: scalar branches
        case 0: ob[0] |= v; break;
        case 1: ob[1] |= v; break;
        case 2: ob[2] |= v; break;
        default: ob[3] |= v; break;
      }
    }
    if (valid) {
      if (nb == kVmMaxBlocks && ((uintptr_t)out & 15) == 0) {
        *(u32x4*)out = u32x4{ob[0], ob[1], ob[2], ob[3]};
      } else {
        for (int b = 0; b < nb; ++b) out[b] = (uint8_t)(ob[b >> 2] >> (8 * (b & 3)));
      }
    }
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
