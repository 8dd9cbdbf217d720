// Internal declarations shared by the attention kernels (not part of the C ABI).
#pragma once

#include "smaq_common.h"

namespace smaq {

struct HistAddr {
  const long long* seq_start;  // NULL: sequence b starts at b * uniform_len
  long long uniform_len;
  long long head_stride;
  const int* table;
  int max_blocks, block_size, n_kv;
  __device__ __forceinline__ int64_t row(int b, int h, int64_t t) const {
    if (table) {
      const int blk = table[(int64_t)b * max_blocks + t / block_size];
      return ((int64_t)blk * n_kv + h) * block_size + (t % block_size);
    }
    return (int64_t)h * head_stride + (seq_start ? seq_start[b] : (int64_t)b * uniform_len) + t;
  }
};

struct Partials {
  float* m;  // [B][Hkv][rows][S]
  float* l;
  float* o;  // [B][Hkv][rows][S][D]
  int S;
  __device__ __forceinline__ int64_t idx(int b, int h, int nkv, int rows, int r, int s) const {
    return (((int64_t)b * nkv + h) * rows + r) * S + s;
  }
};



// MFMA decode path (attention_mfma.hip).  Returns true when it can serve
// these parameters (history only, decode shape, supported formats).
bool mfma_decode_supported(const smaq_attn_params& p);
int64_t mfma_decode_split_len(const smaq_attn_params& p);
int launch_mfma_decode(const smaq_attn_params& p, const HistAddr& a, const Partials& part,
                       int64_t split_len, int n_splits, hipStream_t st);

}  // namespace smaq
