// Block-VQ calibration on the device: shaped keys, k-means++ seeding
// distances and Lloyd centroid updates (the assignment step is the block-VQ
// encoder itself, encode_blockvq_kernel / encode_blockvq_mfma_kernel).
//
// The reference runs k-means++ / Lloyd with torch ops on the calibration
// data's device (smaq/block_vq.py:37-79, 190-203); its CPU random stream
// cannot be reproduced on the device, so this path is judged on codebook
// quality (logit MSE), while the host restatement reproduces the CPU stream.
//
//   shape:   x[b][r][i] = sum_d k[r][b*bd + d] * E_b[i][d], one sequential FMA
//            chain over d (the encoder's own x, so assignments see the same
//            shaped keys as quantize)
//   seeding: dmin[b][r] = min(dmin[b][r], |x[b][r] - x[b][pick_b]|^2)
//   update:  centroid (b, j) = mean of the x[b][r] assigned to j (rows in a
//            fixed partition and reduction order, so the result is
//            deterministic); a centroid with no rows keeps its value
#include "smaq_common.h"

namespace smaq {

constexpr int kFitMaxBlockDim = 16;
constexpr int kFitThreads = 256;

template <typename T>
__global__ __launch_bounds__(kFitThreads) void blockvq_shape_kernel(const T* __restrict__ k, int64_t rows,
                                                                    int nb, int bd,
                                                                    const float* __restrict__ E,
                                                                    float* __restrict__ x) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (r >= rows) return;
  const T* kr = k + r * (int64_t)nb * bd + (int64_t)b * bd;
  const float* Eb = E + (int64_t)b * bd * bd;
  float kv[kFitMaxBlockDim];
  for (int d = 0; d < bd; ++d) kv[d] = Num<T>::to_f(kr[d]);
  float* xr = x + ((int64_t)b * rows + r) * bd;
  for (int i = 0; i < bd; ++i) {
    float a = 0.0f;
    for (int d = 0; d < bd; ++d) a = fmaf(kv[d], Eb[i * bd + d], a);
    xr[i] = a;
  }
}

__global__ __launch_bounds__(kFitThreads) void kmeanspp_update_kernel(const float* __restrict__ x, int64_t rows,
                                                                      int bd, const long long* __restrict__ pick,
                                                                      int first, float* __restrict__ dmin) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int b = blockIdx.y;
  if (r >= rows) return;
  const float* xb = x + (int64_t)b * rows * bd;
  const long long pk = pick[b];
  const float* p = xb + (pk < 0 ? 0 : (pk >= rows ? rows - 1 : pk)) * bd;  // (picks are row indices)
  const float* xr = xb + r * bd;
  float d2 = 0.0f;
  for (int i = 0; i < bd; ++i) {
    const float t = xr[i] - p[i];
    d2 = fmaf(t, t, d2);
  }
  float* dm = dmin + (int64_t)b * rows + r;
  *dm = first ? d2 : fminf(*dm, d2);
}

// one workgroup per (centroid j, block b): thread t sums the rows t, t + 256,
// ... assigned to j, then a fixed-order tree reduction
__global__ __launch_bounds__(kFitThreads) void kmeans_update_kernel(const float* __restrict__ x,
                                                                    const uint8_t* __restrict__ idx, int64_t rows,
                                                                    int nb, int bd, float* __restrict__ C) {
  __shared__ float red[kFitThreads][kFitMaxBlockDim + 1];
  const int j = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const float* xb = x + (int64_t)b * rows * bd;
  float acc[kFitMaxBlockDim];
  for (int i = 0; i < kFitMaxBlockDim; ++i) acc[i] = 0.0f;
  float cnt = 0.0f;
  for (int64_t r = t; r < rows; r += kFitThreads) {
    if (idx[r * nb + b] != (uint8_t)j) continue;
    const float* xr = xb + r * bd;
    for (int i = 0; i < bd; ++i) acc[i] += xr[i];
    cnt += 1.0f;
  }
  for (int i = 0; i < bd; ++i) red[t][i] = acc[i];
  red[t][kFitMaxBlockDim] = cnt;
  __syncthreads();
  for (int s = kFitThreads / 2; s > 0; s >>= 1) {
    if (t < s) {
      for (int i = 0; i < bd; ++i) red[t][i] += red[t + s][i];
      red[t][kFitMaxBlockDim] += red[t + s][kFitMaxBlockDim];
    }
    __syncthreads();
  }
  const float n = red[0][kFitMaxBlockDim];
  if (t < bd && n > 0.0f) C[((int64_t)b * gridDim.x + j) * bd + t] = red[0][t] / n;
}

}  // namespace smaq

using namespace smaq;

extern "C" int smaq_blockvq_shape(const void* k, int kdtype, long long rows, int n_blocks, int block_dim,
                                  const float* E_blocks, float* x_out, void* stream) {
  SMAQ_REQUIRE(k && E_blocks && x_out, "smaq_blockvq_shape: null pointer");
  SMAQ_REQUIRE(rows > 0 && n_blocks >= 1 && n_blocks <= 65535, "smaq_blockvq_shape: bad shape");
  SMAQ_REQUIRE(block_dim >= 1 && block_dim <= kFitMaxBlockDim, "smaq_blockvq_shape: block_dim must be 1..%d",
               kFitMaxBlockDim);
  const dim3 grid((unsigned)((rows + kFitThreads - 1) / kFitThreads), (unsigned)n_blocks);
  hipStream_t st = (hipStream_t)stream;
  switch (kdtype) {
    case SMAQ_F32: hipLaunchKernelGGL(blockvq_shape_kernel<float>, grid, dim3(kFitThreads), 0, st, (const float*)k, (int64_t)rows, n_blocks, block_dim, E_blocks, x_out); break;
    case SMAQ_F16: hipLaunchKernelGGL(blockvq_shape_kernel<_Float16>, grid, dim3(kFitThreads), 0, st, (const _Float16*)k, (int64_t)rows, n_blocks, block_dim, E_blocks, x_out); break;
    case SMAQ_BF16: hipLaunchKernelGGL(blockvq_shape_kernel<bf16>, grid, dim3(kFitThreads), 0, st, (const bf16*)k, (int64_t)rows, n_blocks, block_dim, E_blocks, x_out); break;
    default: set_error("smaq_blockvq_shape: unsupported dtype %d", kdtype); return SMAQ_EUNSUPPORTED;
  }
  return launch_status("smaq_blockvq_shape");
}

extern "C" int smaq_kmeanspp_update(const float* x, int n_blocks, long long rows, int block_dim,
                                    const long long* pick, int first, float* dmin, void* stream) {
  SMAQ_REQUIRE(x && pick && dmin, "smaq_kmeanspp_update: null pointer");
  SMAQ_REQUIRE(rows > 0 && n_blocks >= 1 && n_blocks <= 65535, "smaq_kmeanspp_update: bad shape");
  SMAQ_REQUIRE(block_dim >= 1 && block_dim <= kFitMaxBlockDim, "smaq_kmeanspp_update: bad block_dim");
  const dim3 grid((unsigned)((rows + kFitThreads - 1) / kFitThreads), (unsigned)n_blocks);
  hipLaunchKernelGGL(kmeanspp_update_kernel, grid, dim3(kFitThreads), 0, (hipStream_t)stream, x, (int64_t)rows,
                     block_dim, pick, first, dmin);
  return launch_status("smaq_kmeanspp_update");
}

extern "C" int smaq_kmeans_update(const float* x, const unsigned char* idx, int n_blocks, long long rows,
                                  int block_dim, int n_centroids, float* centroids, void* stream) {
  SMAQ_REQUIRE(x && idx && centroids, "smaq_kmeans_update: null pointer");
  SMAQ_REQUIRE(rows > 0 && n_blocks >= 1 && n_blocks <= 65535, "smaq_kmeans_update: bad shape");
  SMAQ_REQUIRE(block_dim >= 1 && block_dim <= kFitMaxBlockDim, "smaq_kmeans_update: bad block_dim");
  SMAQ_REQUIRE(n_centroids >= 1 && n_centroids <= 256, "smaq_kmeans_update: n_centroids must be 1..256");
  const dim3 grid((unsigned)n_centroids, (unsigned)n_blocks);
  hipLaunchKernelGGL(kmeans_update_kernel, grid, dim3(kFitThreads), 0, (hipStream_t)stream, x, idx,
                     (int64_t)rows, n_blocks, block_dim, centroids);
  return launch_status("smaq_kmeans_update");
}
