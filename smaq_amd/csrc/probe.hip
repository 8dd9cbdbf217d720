// Streaming-read probe (smaq_probe_read): the HBM read rate a plain stream of
// 16-byte non-temporal loads reaches, the ceiling the bandwidth-bound kernels
// are judged against next to the published peak.  Swept on MI355X (1 GiB;
// 2, 4, 8 or 16 loads in flight per lane; 1-16 workgroups of 256 threads per
// CU): nt loads 6.7-7.2 TB/s at 4+ loads in flight, normal loads 5.7-6.5; the
// fastest shape, below, 7.18.
#include "attention_internal.h"

namespace smaq {

constexpr int kProbeThreads = 256;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kProbeUnroll = 4;  // independent 16-byte loads in flight per lane
constexpr int kProbeBlocksPerCu = 2;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const uint4* __restrict__ src, int64_t n,
                                                                   unsigned int* __restrict__ sink) {
  uint4 acc = {0u, 0u, 0u, 0u};
  const int64_t step = (int64_t)gridDim.x * kProbeThreads * kProbeUnroll;
  for (int64_t i = (int64_t)blockIdx.x * kProbeThreads * kProbeUnroll + threadIdx.x; i < n; i += step) {
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int k = 0; k < kProbeUnroll; ++k) {
      const int64_t j = i + (int64_t)k * kProbeThreads;
      const u32x4 x = j < n ? __builtin_nontemporal_load((const u32x4*)(src + j)) : u32x4{0u, 0u, 0u, 0u};
      v[k] = uint4{x[0], x[1], x[2], x[3]};
    }
#pragma unroll
    for (int k = 0; k < kProbeUnroll; ++k) {
      acc.x ^= v[k].x;
      acc.y ^= v[k].y;
      acc.z ^= v[k].z;
      acc.w ^= v[k].w;
    }
  }
  // a data-dependent store the compiler cannot drop, which in practice never
  // happens: the loads stay, the write traffic is zero
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[0] = acc.x;
}

}  // namespace smaq

extern "C" int smaq_probe_read(const void* src, long long bytes, unsigned int* sink, void* stream) {
  SMAQ_REQUIRE(src && sink, "smaq_probe_read: null pointer");
  SMAQ_REQUIRE(bytes >= 0 && bytes % 16 == 0, "smaq_probe_read: bytes must be a non-negative multiple of 16");
  if (bytes == 0) return SMAQ_OK;
  const int64_t n = bytes / 16;
  const int64_t per_block = (int64_t)smaq::kProbeThreads * smaq::kProbeUnroll;
  int64_t blocks = (int64_t)smaq::device_cu_count() * smaq::kProbeBlocksPerCu;
  const int64_t need = (n + per_block - 1) / per_block;
  if (blocks > need) blocks = need;
  hipLaunchKernelGGL(smaq::read_probe_kernel, dim3((unsigned)blocks), dim3(smaq::kProbeThreads), 0,
                     (hipStream_t)stream, (const uint4*)src, n, sink);
  return smaq::launch_status("smaq_probe_read");
}
