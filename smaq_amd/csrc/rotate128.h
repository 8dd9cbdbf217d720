// The decode query rotation at head_dim 128 as one workgroup's work, shared
// by the rotation launch (scalar_codec.hip) and the launch that runs it
// beside the recent window (attention_recent.hip).
//
// out[r][j] = (sum_d x[r][d] * Mt[d][j]) [* s[j]] for ROWS rows per block of
// 256 threads, shaped for latency: thread (dq = t / 32, cg = t % 32) loads
// the 16 x 4 elements Mt[16 dq .. 16 dq + 15][4 cg .. 4 cg + 3] at once (one
// memory round trip), runs a 16-term fmaf chain per row and column, and the
// eight partial chains of an output are summed in a fixed tree,
// ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)).  Every output's rounding
// is thus fixed by the row alone (not by the blocking), and its error bound
// is that of 20 steps (16 products, 3 tree levels, the scale) rather than
// 128.  Mt must be 16-byte aligned.
#pragma once

#include "smaq_common.h"

namespace smaq {

template <int ROWS>
struct __attribute__((aligned(16))) Rot128Lds {  // 16-byte LDS accesses
  float xs[ROWS][128];
  float part[ROWS][8][128];
};

// element i of a query in dtype code xdtype, as fp32
__device__ __forceinline__ float query_elem(const void* x, int xdtype, int64_t i) {
  switch (xdtype) {
    case SMAQ_F32: return ((const float*)x)[i];
    case SMAQ_F16: return Num<_Float16>::to_f(((const _Float16*)x)[i]);
    default: return Num<bf16>::to_f(((const bf16*)x)[i]);
  }
}

// rows [block * ROWS, block * ROWS + ROWS) of the product; t = thread index
template <int ROWS>
__device__ __forceinline__ void rotate128_block(Rot128Lds<ROWS>& L, const void* __restrict__ x, int xdtype,
                                                int64_t rows, const float* __restrict__ Mt,
                                                const float* __restrict__ s, float* __restrict__ out,
                                                int64_t block, int t) {
  const int cg = t & 31, dq = t >> 5;
  const int64_t r0 = block * ROWS;
  float4 m[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) m[i] = *(const float4*)(Mt + (16 * dq + i) * 128 + 4 * cg);
  if (((uintptr_t)x & 15) == 0 && xdtype != SMAQ_F32) {
    // 16-byte loads of 8 fp16 / bf16 elements (c5's 8192 rows: 13.0 -> 10.0 us
    // with 8-row blocks; the same values as element loads)
#pragma unroll
    for (int e = 8 * t; e < ROWS * 128; e += 8 * 256) {
      const int64_t r = r0 + e / 128;
      const uint4 w = r < rows ? *(const uint4*)((const uint16_t*)x + r * 128 + e % 128) : make_uint4(0, 0, 0, 0);
      const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint16_t h = (uint16_t)(wd[k >> 1] >> (16 * (k & 1)));
        L.xs[e / 128][e % 128 + k] = xdtype == SMAQ_F16 ? Num<_Float16>::to_f(__builtin_bit_cast(_Float16, h))
                                                        : Num<bf16>::to_f(__builtin_bit_cast(bf16, h));
      }
    }
  } else if (((uintptr_t)x & 15) == 0) {
#pragma unroll
    for (int e = 4 * t; e < ROWS * 128; e += 4 * 256) {
      const int64_t r = r0 + e / 128;
      const float4 w = r < rows ? *(const float4*)((const float*)x + r * 128 + e % 128) : make_float4(0, 0, 0, 0);
      *(float4*)&L.xs[e / 128][e % 128] = w;
    }
  } else {
#pragma unroll
    for (int e = t; e < ROWS * 128; e += 256) {
      const int64_t r = r0 + e / 128;
      L.xs[e / 128][e % 128] = r < rows ? query_elem(x, xdtype, r * 128 + e % 128) : 0.0f;
    }
  }
  __syncthreads();
#pragma unroll 2
  for (int r = 0; r < ROWS; ++r) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float xv = L.xs[r][16 * dq + i];
      a0 = fmaf(xv, m[i].x, a0);
      a1 = fmaf(xv, m[i].y, a1);
      a2 = fmaf(xv, m[i].z, a2);
      a3 = fmaf(xv, m[i].w, a3);
    }
    *(float4*)&L.part[r][dq][4 * cg] = make_float4(a0, a1, a2, a3);
  }
  __syncthreads();
#pragma unroll
  for (int e = t; e < ROWS * 128; e += 256) {
    const int r = e / 128, j = e % 128;
    if (r0 + r >= rows) continue;
    const float v = ((L.part[r][0][j] + L.part[r][1][j]) + (L.part[r][2][j] + L.part[r][3][j])) +
                    ((L.part[r][4][j] + L.part[r][5][j]) + (L.part[r][6][j] + L.part[r][7][j]));
    out[(r0 + r) * 128 + j] = s ? v * s[j] : v;
  }
}

// blocks of 4 rows up to this many rows (a c3 step's 1024 rows: 256 blocks),
// 8 beyond (fewer copies of the 64 KB matrix read from L2, and still one
// round of blocks at c5's 8192 rows: 10.0 us against 10.3 with 16 rows and
// 10.9 with 4, timed after a 512 MB read sweep)
constexpr int64_t kRot128ManyRows = 2048;

}  // namespace smaq
