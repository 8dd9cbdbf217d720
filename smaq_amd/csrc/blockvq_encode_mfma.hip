// Block-VQ key encoder on the gfx950 matrix cores (8-dim blocks, 256
// centroids per block, up to 16 blocks).
//
// Same indices as encode_blockvq_kernel (blockvq_codec.hip), which follows
// the reference's torch-CPU arithmetic (smaq/block_vq.py:216-244):
//   x_e  = sequential fmaf chain over d of k_d * E_b[e][d]
//   d2_c = fmaf chain over e of (-2 x_e) * C_c[e], + |x|^2, + |C_c|^2,
//          clamp_min(0); index = first minimum of sqrt(d2)  (cdist's matmul form)
// Here x is computed the same way (bit for bit), and all 256 distances of a
// (token, block) come from three v_mfma_f32_16x16x4_f32 per 16 centroids:
// A = [C_c[0..3]], [C_c[4..7]], [|C_c|^2, 1, 0, 0], B = [-2x[0..3]],
// [-2x[4..7]], [1, |x|^2 + delta, 0, 0].  Those values differ from the
// reference's chain only by rounding order, at most 3e-6 * (|x|^2 + max |C|^2)
// for these 12-term sums, so the argmin is the reference's whenever the
// runner-up is more than delta = 1.2e-5 * (|x|^2 + max |C|^2) behind the best.
// Otherwise (about 1e-3 of the (token, block) pairs on SMAQ-shaped keys, or a
// non-finite key) the whole wave recomputes that pair's 256 distances with
// the exact chain and takes the reference's argmin and tie count.
//
// Layout: one persistent workgroup of 16 waves per CU holds the codebook in
// LDS in MFMA A-operand order (8 KB per block, conflict-free dword reads) plus
// |C|^2 and E; each wave encodes 16 tokens at a time, block after block.  The
// running minimum keeps the distance bits with the low 6 bits replaced by the
// centroid's position in the lane (tile, row), so one v_min_u32 tracks value
// and index (distances are positive: delta is added to every one).
#include "encode_internal.h"

namespace smaq {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kVmWaves = 16;                  // waves per workgroup (4 per SIMD)
constexpr int kVmThreads = 64 * kVmWaves;
constexpr int kVmNc = 256;                    // centroids per block
constexpr int kVmBd = 8;                      // block dim
constexpr int kVmMaxBlocks = 16;
constexpr int kCtBlock = 2 * 2 * kVmNc * 2;   // floats of one block's A operands
constexpr float kDeltaRel = 1.2e-5f;

__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bitsf(uint32_t b) { return __builtin_bit_cast(float, b); }

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* out) {
  if constexpr (sizeof(T) == 2) {
    const u32x4 v = *(const u32x4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)v[i]));
      out[2 * i + 1] = Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(v[i] >> 16)));
    }
  } else {
    const u32x4 a = *(const u32x4*)p, b = *(const u32x4*)(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = bitsf(a[i]);
      out[4 + i] = bitsf(b[i]);
    }
  }
}

// Exact distances of one (token, block) by the whole wave (4 centroids per
// lane) and the reference's choice: first index of the smallest sqrt(d2),
// with NaN winning at its first index; `tie` when another centroid is within
// 2e-6 relative of the smallest d2.
__device__ int exact_argmin(const float* x, float xsq, const float* ct, const float* csq, int lane,
                            bool* tie) {
  uint64_t key = ~0ull;
  float dmin = __builtin_inff();
  float d2v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < kVmBd; ++e) {
      const float ce = ct[((e >> 2) * 2 + ((e >> 1) & 1)) * (2 * kVmNc) + 2 * c + (e & 1)];
      a = fmaf(-2.0f * x[e], ce, a);
    }
    a = a + xsq;
    a = a + csq[c];
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
  extern __shared__ float lds[];
  float* const ct_all = lds;                          // [nb][2 steps][2 k-pairs][256][2]
  float* const csq_all = ct_all + nb * kCtBlock;      // [nb][256]
  float* const es_all = csq_all + nb * kVmNc;         // [nb][8][8]
  float* const cmax_all = es_all + nb * 64;           // [nb] max |C|^2
  const int tid = threadIdx.x;
  for (int i = tid; i < nb * kVmNc * kVmBd; i += kVmThreads) {
    const int b = i / (kVmNc * kVmBd), r = i - b * (kVmNc * kVmBd);
    const int c = r / kVmBd, e = r - c * kVmBd;
    ct_all[b * kCtBlock + ((e >> 2) * 2 + ((e >> 1) & 1)) * (2 * kVmNc) + 2 * c + (e & 1)] = C[i];
  }
  for (int i = tid; i < nb * kVmNc; i += kVmThreads) {
    const float* c = C + (int64_t)i * kVmBd;
    float s = 0.0f;
    for (int e = 0; e < kVmBd; ++e) s = s + c[e] * c[e];  // x.pow(2).sum(-1) order
    csq_all[i] = s;
  }
  for (int i = tid; i < nb * 64; i += kVmThreads) es_all[i] = E_blocks[i];
  __syncthreads();
  for (int b = tid; b < nb; b += kVmThreads) {
    float m = 0.0f;
    for (int c = 0; c < kVmNc; ++c) m = fmaxf(m, csq_all[b * kVmNc + c]);
    cmax_all[b] = m;
  }
  __syncthreads();

  const int lane = tid & 63, w = tid >> 6;
  const int n = lane & 15, kg = lane >> 4;  // MFMA coordinates: token / centroid row n, k-group kg
  typedef const __attribute__((address_space(3))) float LdsF;
  unsigned ties = 0;
  const int64_t n_tiles = (rows + 15) / 16;
  for (int64_t tile = (int64_t)blockIdx.x * kVmWaves + w; tile < n_tiles;
       tile += (int64_t)gridDim.x * kVmWaves) {
    const int64_t row = tile * 16 + n;
    const bool valid = row < rows;
    const T* kr = k + map.offset(valid ? row : rows - 1);
    for (int b = 0; b < nb; ++b) {
      float kv[kVmBd];
      load8<T>(kr + b * kVmBd, kv);
      const float* es = es_all + b * 64;
      // x_kg and x_{kg+4}: the reference's chain, bit for bit
      float xa = 0.0f, xb = 0.0f;
#pragma unroll
      for (int d = 0; d < kVmBd; ++d) {
        xa = fmaf(kv[d], es[kg * 8 + d], xa);
        xb = fmaf(kv[d], es[(kg + 4) * 8 + d], xb);
      }
      float sq = xa * xa + xb * xb;
      sq += __shfl_xor(sq, 16, 64);
      sq += __shfl_xor(sq, 32, 64);
      const float delta = kDeltaRel * (sq + cmax_all[b]);
      const float b0 = -2.0f * xa, b1 = -2.0f * xb;
      const float b2 = kg == 0 ? 1.0f : (kg == 1 ? sq + delta : 0.0f);
      const LdsF* ct = (const LdsF*)(ct_all + b * kCtBlock) + (kg >> 1) * (2 * kVmNc) + 2 * n + (kg & 1);
      const LdsF* cs = (const LdsF*)(csq_all + b * kVmNc) + n;
      uint32_t best = 0xffffffffu, second = 0xffffffffu;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const float a0 = ct[32 * t];
        const float a1 = ct[2 * (2 * kVmNc) + 32 * t];
        const float csv = cs[16 * t];
        const float a2 = kg == 0 ? csv : (kg == 1 ? 1.0f : 0.0f);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a2, b2, acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // centroid 16t + 4kg + i of token n; low 6 bits = (t, i)
          const uint32_t key = (fbits(acc[i]) & 0xffffffc0u) | (uint32_t)(4 * t + i);
          second = min(second, max(best, key));
          best = min(best, key);
        }
      }
      // merge the four k-group lanes of each token
      uint32_t gbest = best, gsecond = second;
#pragma unroll
      for (int off = 16; off < 64; off <<= 1) {
        const uint32_t ob = (uint32_t)__shfl_xor((int)gbest, off, 64);
        const uint32_t os = (uint32_t)__shfl_xor((int)gsecond, off, 64);
        gsecond = min(min(gsecond, os), max(gbest, ob));
        gbest = min(gbest, ob);
      }
      const float vb = bitsf(gbest & 0xffffffc0u), vs = bitsf(gsecond & 0xffffffc0u);
      // clear winner: the runner-up more than delta behind (keys are
      // truncated by at most 2^-17 relative); distances positive and finite
      const bool clear = (vs - vb * (1.0f + 0x1p-16f) > delta) && vb > 0.0f && vb < 3.0e38f &&
                         delta < 3.0e38f;
      const int kw = best == gbest ? kg : 4;  // the lane holding the winner
      int kwin = kw;
      kwin = min(kwin, __shfl_xor(kwin, 16, 64));
      kwin = min(kwin, __shfl_xor(kwin, 32, 64));
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
        const int ci = exact_argmin(x, xsq, ct_all + b * kCtBlock, csq_all + b * kVmNc, lane, &tie);
        if (n == t0) idx = ci;
        if (lane == t0) ties += tie ? 1u : 0u;
      }
      if (valid && kg == 0) idx_out[row * nb + b] = (uint8_t)idx;
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
  return (size_t)nb * (kCtBlock + kVmNc + 64 + 1) * sizeof(float);
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
  // the codebook takes more than the default 64 KB of dynamic LDS
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
