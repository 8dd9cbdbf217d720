// Internal declarations shared by the attention kernels (not part of the C ABI).
#pragma once

#include "smaq_common.h"

namespace smaq {

// Element idx of the plain (unrotated) query as fp32: from the raw query in
// its own dtype when the caller hands one in (p.q_raw), else from q_exact.
__device__ __forceinline__ float exact_query(const smaq_attn_params& p, int64_t idx) {
  if (p.q_raw == nullptr) return p.q_exact[idx];
  switch (p.q_raw_dtype) {
    case SMAQ_F32: return ((const float*)p.q_raw)[idx];
    case SMAQ_F16: return Num<_Float16>::to_f(((const _Float16*)p.q_raw)[idx]);
    default: return Num<bf16>::to_f(((const bf16*)p.q_raw)[idx]);
  }
}

struct HistAddr {
  const long long* seq_start;  // NULL: sequence b starts at b * uniform_len
  long long uniform_len;
  long long head_stride;
  const int* table;
  int max_blocks, block_size, n_kv;
  long long rows = 0;  // rows in each pool array, 0 if unknown
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



// Matrix-core prefill path (attention_prefill.hip).  Each attended part
// (history, recent window) is first decoded into f16 tile images:
// [B][Hkv][Lp / 64] tiles of 48 KB, each the LDS image the kernel copies
// (key hi, key lo, value hi: kPrefillPlanes f16 planes of head_dim x 64;
// layout in attention_prefill.hip), a 16 KB value-lo plane per tile in a
// second array, and per tile the largest error the value hi plane alone
// leaves (fp32; NaN when a value is not finite).
constexpr int kPrefillPlanes = 3;
constexpr int kPrefillLoHalves = 8192;  // halves per value-lo plane
struct PrefillPlanes {
  _Float16* img;
  _Float16* img_lo;
  float* err;  // [B][Hkv][Lp / 64]
  int64_t Lp;  // padded tokens per (sequence, KV head), multiple of 64
};
// workspace bytes of one part's PrefillPlanes
int64_t prefill_planes_bytes(int64_t batch, int64_t n_kv_heads, int64_t Lp);
// the PrefillPlanes of a part at ws (prefill_planes_bytes long)
PrefillPlanes prefill_planes_at(char* ws, int64_t batch, int64_t n_kv_heads, int64_t Lp);

// One part as the prefill kernel reads it.
struct PrefillPart {
  const float* q;               // q_hist or q_exact
  const _Float16* img;
  const _Float16* img_lo;
  const float* err;
  const long long* len;         // [batch] tokens per sequence, NULL: max_len
  int64_t max_len, Lp, split_len;
  long long pos_offset;         // absolute position of token 0
  int s_base;                   // first partials split of this part
};

// compute units of the current device (256 if the query fails)
int device_cu_count();

bool prefill_mfma_supported(const smaq_attn_params& p);
int64_t prefill_padded_len(int64_t L);
int64_t prefill_split_len(const smaq_attn_params& p, int64_t L);
int launch_prefill_planes_hist(const smaq_attn_params& p, const HistAddr& a, const PrefillPlanes& pl,
                               hipStream_t st);
int launch_prefill_planes_recent(const smaq_attn_params& p, const PrefillPlanes& pl, hipStream_t st);
int launch_prefill_mfma(const smaq_attn_params& p, const PrefillPart& pp, int n_splits, const Partials& part,
                        hipStream_t st);

// Recent window of a decode step (attention_recent.hip): one query token per
// sequence, head_dim 128, 1/2/4 query heads per KV head; impl 1 keeps the
// generic kernel.  Writes the same partials as the generic recent kernel
// (splits s_base .. s_base+n_splits-1).
bool recent_decode_supported(const smaq_attn_params& p);
// tokens per split of the decode recent window (one chunk per workgroup)
int64_t recent_decode_split_len();
int launch_recent_decode(const smaq_attn_params& p, const Partials& part, int s_base, int n_splits,
                         int64_t split_len, hipStream_t st);
// The query rotation (phase 8, into q_hist) and the decode recent window
// (phase 2) in one launch; supported when both are (head_dim 128, a 16-byte
// aligned rot_mt, a raw query).
bool rotate_recent_supported(const smaq_attn_params& p);
int launch_rotate_recent(const smaq_attn_params& p, const Partials& part, int s_base, int n_splits,
                         int64_t split_len, hipStream_t st);

// MFMA decode path (attention_mfma.hip).  Returns true when it can serve
// these parameters (history only, decode shape, supported formats).
bool mfma_decode_supported(const smaq_attn_params& p);
// Tokens per step of a decode workgroup (4 waves x 32-token tiles): split and
// piece boundaries are multiples of it.
constexpr int kMfmaDecodeStep = 128;
int64_t mfma_decode_split_len(const smaq_attn_params& p);
// `order` (NULL: sequence b runs as grid row b) lists the sequences in the
// order their workgroups are dispatched; launch_decode_order fills it with
// the sequences by history length, longest first.
int launch_decode_order(const smaq_attn_params& p, int* order, hipStream_t st);
// A work item of the longest-first piece schedule: tokens [t0, t1) of
// sequence seq, piece `meta & 0xffff` of `meta >> 16`.  seq < 0: no work
// (the decode grid is sized for the most items the lengths could need).
struct DecodeItem {
  int seq, t0, t1, meta;
};
// The longest-first order as `n_items` work items (at `items`): the
// sequences ranked first_round and later run in up to max_pieces pieces of
// about piece_len tokens (decode_schedule.hip).
int launch_decode_items(const smaq_attn_params& p, int first_round, int max_pieces, int64_t piece_len,
                        int n_items, void* items, hipStream_t st);
// One launch for the query rotation (p.q_raw by p.rot_mt into p.q_hist, as
// smaq_rotate_rows at head_dim 128) and the decode schedule: the order at
// `sched` when n_items is 0, else the work items.  Supported at head_dim 128
// with a 16-byte aligned rot_mt and a raw fp32/fp16/bf16 query.
bool rotate_schedule_supported(const smaq_attn_params& p);
int launch_rotate_schedule(const smaq_attn_params& p, int first_round, int max_pieces, int64_t piece_len,
                           int n_items, void* sched, hipStream_t st);

// With `direct` (one split and no recent part) the kernel writes the final
// output itself, and no split combine is needed; with `merge` (several
// splits, no recent part, p.arrivals set) the last workgroup of each
// (sequence, KV head) merges the splits and writes the output.  items > 0:
// `order` holds that many work items (launch_decode_items), n_splits is
// the most pieces of a sequence, and `merge` is required.
int launch_mfma_decode(const smaq_attn_params& p, const HistAddr& a, const Partials& part,
                       int n_splits, bool direct, bool merge, const int* order, int items, hipStream_t st);

}  // namespace smaq
