// Shared device helpers for the SMAQ HIP kernels (gfx950, wave64).
//
// Arithmetic contract: this library is compiled with -ffp-contract=off, so a
// multiply followed by an add is two IEEE roundings unless fmaf() is written
// explicitly.  The encoders reproduce torch-CPU results bit for bit; every
// place where the order or fusion of operations matters says which torch-CPU
// behaviour it matches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/smaq_hip.h"

namespace smaq {

// ---------------------------------------------------------------- dtypes ---
struct bf16 {
  uint16_t bits;
};

template <typename T>
struct Num;

template <>
struct Num<float> {
  static __device__ __forceinline__ float to_f(float v) { return v; }
  static __device__ __forceinline__ float from_f(float v) { return v; }
  // Rounding of an fp32 result to the storage dtype (identity for fp32).
  static __device__ __forceinline__ float round(float v) { return v; }
};

template <>
struct Num<_Float16> {
  static __device__ __forceinline__ float to_f(_Float16 v) { return (float)v; }
  static __device__ __forceinline__ _Float16 from_f(float v) { return (_Float16)v; }  // RNE
  static __device__ __forceinline__ float round(float v) { return (float)(_Float16)v; }
};

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;  // NaN, as c10::BFloat16
  u += 0x7fffu + ((u >> 16) & 1u);                     // round to nearest even
  return (uint16_t)(u >> 16);
}

template <>
struct Num<bf16> {
  static __device__ __forceinline__ float to_f(bf16 v) { return __uint_as_float((uint32_t)v.bits << 16); }
  static __device__ __forceinline__ bf16 from_f(float v) { return bf16{f32_to_bf16_bits(v)}; }
  static __device__ __forceinline__ float round(float v) {
    return __uint_as_float((uint32_t)f32_to_bf16_bits(v) << 16);
  }
};

// torch's clamp(min=c) converts the bound to the tensor dtype first.
template <typename T>
__device__ __forceinline__ float dtype_const(float c) {
  return Num<T>::round(c);
}

// Round half to even, as torch.round (P3); NaN passes through.
__device__ __forceinline__ float round_half_even(float x) { return __builtin_rintf(x); }

// Row addressing shared by the encoders: logical row r = o * n_inner + i lives
// at element offset o * s_outer + i * s_inner; its last dim is contiguous.
// This covers both contiguous [rows, D] input and the [T, Hkv, D] -> [Hkv, T]
// transpose view that the store hands to the codecs.  Its outputs go to
// output row o * out_outer + i: dense (r itself) when out_outer == n_inner,
// or the tail rows of per-head columns [Hkv, capacity, ...] when out_outer is
// the columns' capacity (the store's encode-on-append).
struct RowMap {
  int64_t n_inner, s_outer, s_inner, out_outer;
  __device__ __forceinline__ int64_t offset(int64_t r) const {
    const int64_t o = r / n_inner;
    const int64_t i = r - o * n_inner;
    return o * s_outer + i * s_inner;
  }
  __device__ __forceinline__ int64_t out_row(int64_t r) const {
    if (out_outer == n_inner) return r;
    return r + (r / n_inner) * (out_outer - n_inner);
  }
};

__device__ __forceinline__ float warp_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float warp_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ unsigned warp_sum_u(unsigned v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Adds a per-thread count to a device counter with one atomic per wave.
__device__ __forceinline__ void add_count(unsigned long long* counter, unsigned local) {
  if (counter == nullptr) return;
  const unsigned tot = warp_sum_u(local);
  if ((threadIdx.x & 63) == 0 && tot) atomicAdd(counter, (unsigned long long)tot);
}

}  // namespace smaq

// ------------------------------------------------------------- host side ---
namespace smaq {
void set_error(const char* fmt, ...);
int launch_status(const char* what);
}  // namespace smaq

#define SMAQ_REQUIRE(cond, ...)        \
  do {                                 \
    if (!(cond)) {                     \
      ::smaq::set_error(__VA_ARGS__);  \
      return SMAQ_EINVAL;              \
    }                                  \
  } while (0)
