// Dispatch schedules of the matrix-core decode kernel for ragged batches:
// the sequences by history length, longest first (an order), or the same
// ranking as work items whose later sequences run in pieces; and the launch
// that builds either beside the query rotation.
//
// Ranking: a counting sort on 1024 length buckets by one workgroup.  The
// bucket order is deterministic; the order within a bucket is not, and
// changes no result: each decode workgroup computes its own (sequence, KV
// head, piece) partial, and a sequence's pieces follow from its length and
// the bucket counts alone.

#include "attention_internal.h"
#include "rotate128.h"

namespace smaq {

constexpr int kOrderBuckets = 1024;

template <int NT>
struct ScheduleLds {
  int count[kOrderBuckets];  // bucket counts, then the buckets' rank counters
  int start[kOrderBuckets];  // first rank of each bucket
  int extra[kOrderBuckets];  // items before each bucket beyond one per sequence
  int pieces[kOrderBuckets]; // pieces of each bucket's sequences
  int scan[NT];
};

// Exclusive prefix sum over the NT threads of a workgroup: a shuffle scan
// inside each wave, then the waves' totals through LDS (two barriers, where
// a Hillis-Steele scan over the workgroup takes two per step: 6.8 -> 5.4 us
// for the c5 schedule); returns this thread's exclusive sum and the total.
template <int NT>
__device__ int block_exclusive_scan(int* buf, int v, int tid, int& total) {
  constexpr int NW = NT / 64;
  static_assert(NT % 64 == 0 && NW <= 64, "whole waves");
  const int lane = tid & 63, w = tid >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    x += lane >= off ? y : 0;
  }
  if (lane == 63) buf[w] = x;  // the wave's total
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int t = buf[i];
    before += i < w ? t : 0;
    tot += t;
  }
  __syncthreads();  // buf is free for the next scan
  total = tot;
  return before + x - v;
}

// One workgroup of NT threads (thread t owns buckets [t * BPT, t * BPT + BPT)).
// items == nullptr: writes order[rank] = sequence.  Otherwise the schedule as
// work items: buckets that begin within the first `first_round` ranks (the
// sequences whose KV heads fill the first round of workgroup slots) run
// whole; every later sequence runs in g pieces, g = ceil(L_hi / piece_len)
// capped at max_pieces, L_hi the bucket's upper length bound, the boundaries
// at L * k / g rounded down to whole decode steps.  A sequence of rank r in
// bucket k takes items r + E_k + (r - start_k) * (g_k - 1) ..., E_k the extra
// items of the buckets before k; items past the last are written empty.
template <int NT>
__device__ void build_schedule(ScheduleLds<NT>& L, const long long* __restrict__ len, long long max_len,
                               int batch, int first_round, int max_pieces, long long piece_len, int n_items,
                               int* __restrict__ order, DecodeItem* __restrict__ items, int tid) {
  constexpr int BPT = kOrderBuckets / NT;
  static_assert(kOrderBuckets % NT == 0, "buckets per thread");
  auto clamp_len = [&](int b) {
    const long long x = len[b];
    return x < 0 ? 0 : (x > max_len ? max_len : x);
  };
  auto bucket = [&](long long x) {
    return kOrderBuckets - 1 - (int)(x * (kOrderBuckets - 1) / max_len);  // longest -> 0
  };
#pragma unroll
  for (int i = 0; i < BPT; ++i) L.count[tid * BPT + i] = 0;
  __syncthreads();
  for (int b = tid; b < batch; b += NT) atomicAdd(&L.count[bucket(clamp_len(b))], 1);
  __syncthreads();
  int c[BPT], own = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    c[i] = L.count[tid * BPT + i];
    own += c[i];
  }
  int total = 0;
  int run = block_exclusive_scan<NT>(L.scan, own, tid, total);
  int g[BPT], ex_own = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    const int k = tid * BPT + i;
    L.start[k] = run;
    // lengths x with floor(x * 1023 / max) = j lie below (j + 1) * max / 1023
    const long long j = kOrderBuckets - 1 - k;
    const long long hi = ((j + 1) * max_len + (kOrderBuckets - 2)) / (kOrderBuckets - 1);
    long long gk = items ? (hi + piece_len - 1) / piece_len : 1;
    gk = gk < 1 ? 1 : (gk > max_pieces ? max_pieces : gk);
    g[i] = run < first_round ? 1 : (int)gk;
    ex_own += c[i] * (g[i] - 1);
    run += c[i];
  }
  int extra_total = 0;
  int ex = block_exclusive_scan<NT>(L.scan, ex_own, tid, extra_total);
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    const int k = tid * BPT + i;
    L.extra[k] = ex;
    L.pieces[k] = g[i];
    L.count[k] = L.start[k];  // the bucket's rank counter
    ex += c[i] * (g[i] - 1);
  }
  __syncthreads();
  for (int b = tid; b < batch; b += NT) {
    const long long x = clamp_len(b);
    const int k = bucket(x);
    const int r = atomicAdd(&L.count[k], 1);
    if (!items) {
      order[r] = b;
      continue;
    }
    const int gb = L.pieces[k];
    const int base = r + L.extra[k] + (r - L.start[k]) * (gb - 1);
    long long t0 = 0;
    for (int i = 0; i < gb; ++i) {
      const long long t1 = i + 1 == gb ? x : (x * (i + 1) / gb) & ~(long long)(kMfmaDecodeStep - 1);
      items[base + i] = DecodeItem{b, (int)t0, (int)t1, (gb << 16) | i};
      t0 = t1;
    }
  }
  if (items) {
    for (int i = batch + extra_total + tid; i < n_items; i += NT) items[i] = DecodeItem{-1, 0, 0, 0};
  }
}

__global__ __launch_bounds__(kOrderBuckets) void decode_schedule_kernel(
    const long long* __restrict__ len, long long max_len, int batch, int first_round, int max_pieces,
    long long piece_len, int n_items, int* __restrict__ order, DecodeItem* __restrict__ items) {
  __shared__ ScheduleLds<kOrderBuckets> lds;
  build_schedule<kOrderBuckets>(lds, len, max_len, batch, first_round, max_pieces, piece_len, n_items, order,
                                items, (int)threadIdx.x);
}

// Workgroup 0 builds the schedule (256 threads, 4 buckets each), workgroups
// 1.. rotate ROWS query rows each (rotate128_block, the rotation launch's
// own body: the same bits).  c5: 9.63 us against 9.26 + 5.35 us for the two
// launches, step 397.8 against 401.0 us (three alternating rounds); with the
// workgroup-wide Hillis-Steele scans the schedule workgroup outlasted the
// rotation and the fused launch gained nothing.
template <int ROWS>
__global__ __launch_bounds__(256) void rotate_schedule_kernel(
    const void* __restrict__ x, int xdtype, int64_t rows, const float* __restrict__ Mt,
    const float* __restrict__ s, float* __restrict__ out, const long long* __restrict__ len,
    long long max_len, int batch, int first_round, int max_pieces, long long piece_len, int n_items,
    int* __restrict__ order, DecodeItem* __restrict__ items) {
  __shared__ union {
    Rot128Lds<ROWS> rot;
    ScheduleLds<256> sched;
  } lds;
  if (blockIdx.x == 0) {
    build_schedule<256>(lds.sched, len, max_len, batch, first_round, max_pieces, piece_len, n_items, order,
                        items, (int)threadIdx.x);
  } else {
    rotate128_block<ROWS>(lds.rot, x, xdtype, rows, Mt, s, out, (int64_t)blockIdx.x - 1, (int)threadIdx.x);
  }
}

bool rotate_schedule_supported(const smaq_attn_params& p) {
  return p.head_dim == 128 && p.rot_mt && ((uintptr_t)p.rot_mt & 15) == 0 && p.q_raw &&
         (p.q_raw_dtype == SMAQ_F32 || p.q_raw_dtype == SMAQ_F16 || p.q_raw_dtype == SMAQ_BF16);
}

int launch_rotate_schedule(const smaq_attn_params& p, int first_round, int max_pieces, int64_t piece_len,
                           int n_items, void* sched, hipStream_t st) {
  const int64_t rows = (int64_t)p.batch * p.q_len * p.n_q_heads;
  const int rpb = rows > kRot128ManyRows ? 8 : 4;
  const int64_t blocks = (rows + rpb - 1) / rpb + 1;
  SMAQ_REQUIRE(blocks < (1ll << 31), "smaq_attn_hybrid: too many query rows");
  int* order = n_items > 0 ? nullptr : (int*)sched;
  DecodeItem* items = n_items > 0 ? (DecodeItem*)sched : nullptr;
  if (n_items <= 0) first_round = 0, max_pieces = 1, piece_len = 1;
  if (rpb == 8)
    hipLaunchKernelGGL(rotate_schedule_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, st, p.q_raw, p.q_raw_dtype,
                       rows, p.rot_mt, p.rot_scale, (float*)p.q_hist, p.hist_len, (long long)p.max_hist_len,
                       p.batch, first_round, max_pieces, (long long)piece_len, n_items, order, items);
  else
    hipLaunchKernelGGL(rotate_schedule_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, p.q_raw, p.q_raw_dtype,
                       rows, p.rot_mt, p.rot_scale, (float*)p.q_hist, p.hist_len, (long long)p.max_hist_len,
                       p.batch, first_round, max_pieces, (long long)piece_len, n_items, order, items);
  return launch_status("smaq_attn_hybrid(rotation + decode schedule)");
}

int launch_decode_order(const smaq_attn_params& p, int* order, hipStream_t st) {
  hipLaunchKernelGGL(decode_schedule_kernel, dim3(1), dim3(kOrderBuckets), 0, st, p.hist_len,
                     (long long)p.max_hist_len, p.batch, 0, 1, 1LL, 0, order, (DecodeItem*)nullptr);
  return launch_status("smaq_attn_hybrid(decode order)");
}

int launch_decode_items(const smaq_attn_params& p, int first_round, int max_pieces, int64_t piece_len,
                        int n_items, void* items, hipStream_t st) {
  hipLaunchKernelGGL(decode_schedule_kernel, dim3(1), dim3(kOrderBuckets), 0, st, p.hist_len,
                     (long long)p.max_hist_len, p.batch, first_round, max_pieces, (long long)piece_len, n_items,
                     (int*)nullptr, (DecodeItem*)items);
  return launch_status("smaq_attn_hybrid(decode items)");
}

}  // namespace smaq
