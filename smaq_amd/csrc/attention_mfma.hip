// Decode attention over scalar-coded keys on the gfx950 matrix cores.
//
// Serves the common decode shape: head_dim 128, 3- or 4-bit scalar key codes
// (two per byte), 2-bit values in groups of 32, one query token per sequence
// and up to 4 query heads per KV head.  One workgroup = 4 waves over one
// (context split, KV head, sequence); each wave streams 32-token tiles, and
// issues each array's loads for the next tile as soon as it has consumed the
// current tile's copy.  With 16-bit norms and value metadata the kernel fits
// 128 VGPRs, i.e. 4 waves per SIMD (the query operands live in LDS).
//
// Per 32-token tile (two 16-token halves):
//   QK   v_mfma_f32_16x16x32_f16, M = 16 tokens, K = 32 dims, N = 16 columns:
//        columns [0, Q) hold the query hi parts, [8, 8+Q) the lo parts.  The
//        decoded key is split hi/lo as well (q.k ~= qh.kh + ql.kh + qh.kl), so
//        scores keep ~22 bits against fp32.  Key bytes (two codes) go through
//        a 256-entry LDS table whose 8-byte entries hold both codes' f16 hi
//        and lo halves (one ds_read_b64 per byte).
//   soft the hi and lo columns are summed with one DPP add and the 4 x 32
//        (query, token) scores are redistributed two per lane; online softmax
//        in base 2 whose reference maximum is raised only when a score exceeds
//        it by 2^8, so the cross-lane max and the rescale are rare.
//   PV   v_mfma_f32_16x16x32_bf16, M = 16 rows (query head j, value group g),
//        K = 32 tokens, N = 16 dims.  A = p * scale_g split bf16 hi/lo, staged
//        through LDS in MFMA layout.  B: the value codes are spread to 16-bit
//        lanes once per tile (LDS), and step tau takes bit field tau >> 1 of
//        code byte 16*(tau & 1) + n as the bf16 value 128 + (c << 2f) with one
//        and-or per dword; the 128 * sum(A) offset (an MFMA against ones), the
//        2^2f column factor and the zero-point term sum(p * zero) are removed
//        at the end.
// Scores and outputs match the reference fp32 path to ~1e-6 relative; the
// unsupported shapes use the generic kernels in attention.hip.
#include <math.h>

#include <type_traits>

#include "attention_internal.h"

namespace smaq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kMWaves = 4;
constexpr int kMTile = 32;
static_assert(kMWaves * kMTile == kMfmaDecodeStep, "decode step");
constexpr int kVRow = 80;   // bytes per code-byte row of the spread value tile (64 + 16 pad)
constexpr int kARow = 144;  // bytes per row of the staged PV A operand (64 hi + 64 lo + 16 pad)
// The softmax reference maximum is raised only when a score exceeds it by
// this much (log2 units), so weights stay below 2^8 and rescales are rare.
constexpr float kLazyRescale = 8.0f;
// s_waitcnt operand that waits for LDS and scalar loads only (lgkmcnt 0,
// vmcnt and expcnt at their maxima)
constexpr int kWaitLdsOnly = 0xC07F;
// s_waitcnt operand that waits for vector memory operations only (vmcnt 0,
// expcnt and lgkmcnt at their maxima)
constexpr int kWaitVmemOnly = 0x0F70;
// Cache policy of the tile loads (buffer-load aux 2 = nt, streaming).  A
// plain read stream reaches 7.0-7.2 TB/s with nt loads against 6.3-6.45
// without (MI355X, 1 GiB, every unroll and occupancy tried), and the key rows
// (1 KB per load instruction, whole lines read once) and the contiguous
// value rows take it: kernel 179.0-182.2 -> 177.1-180.4 us at c3, 390.4-401.7
// -> 387.9-400.3 us at c5 (keys; five alternating rounds on three boxes,
// rocprofv3 averages over ~1,800-3,600 launches each).  The norms (64-byte
// runs, their lines shared with the neighbouring tile) and the value scales
// and zeros (two whole lines per tile, each 16 bytes read by four lanes)
// stay normal: nt on all three made c3 2-3% slower, on the scales and zeros
// alone 3.6%, on the norms alone 1.1%; so do the paged layout's value loads
// (32-byte pieces of 512-byte pages: +7.6% at c5).
constexpr int kKeyPolicy = 2;
constexpr int kValPolicy = 2;
constexpr int kSidePolicy = 0;

// Split boundaries.  The grid (KV heads, sequences, splits) is dispatched
// split-major, so with one round of workgroups, split s of unit u = head +
// n_kv_heads * sequence runs in round-slot k = (u + units * s) / n_cu of its
// CU.  A CU's memory pipeline serves its earlier-dispatched workgroups first:
// with equal splits (c3 on MI355X, 4 slots per CU) the slots took 147, 154,
// 162 and 169 us.  Split s therefore weighs kSplitWeight - tilt * k, and its
// first token is the sequence length times the weight of the splits before it
// over the total, rounded down to whole 128-token steps.
constexpr int kMaxSlots = 4;
struct SplitRule {
  int n_splits;
  int n_cu;   // workgroups per round-slot (the device's CU count)
  int slots;  // round-slots per CU (at most kMaxSlots)
  int tilt;   // weight step per slot; tilt * (slots - 1) < kSplitWeight
  int direct; // no recent part: a (sequence, KV head) of one split writes
              // the final output
  int merge;  // arrival counters given (several splits, or a recent part
              // whose partials an earlier launch wrote): the last workgroup
              // of each (sequence, KV head) merges and writes the output
  int pieces; // grid rows are work items (DecodeItem), not sequences: the
              // sequences past the first round of workgroup slots run in up
              // to n_splits pieces each
  int items;  // grid rows in item mode
};

constexpr int kSplitWeight = 64;

// The splits of unit u (of `units`) from which on the round-slot is at
// least j, for j = 1 .. slots-1.
struct SlotStarts {
  int first[kMaxSlots];
  __device__ __forceinline__ SlotStarts(const SplitRule& r, int u, int units) {
#pragma unroll
    for (int j = 1; j < kMaxSlots; ++j) {
      const int num = j * r.n_cu - u;
      first[j] = j >= r.slots ? 0x7fffffff
                              : (num <= 0 ? 0 : (int)(((unsigned)num + (unsigned)units - 1u) / (unsigned)units));
    }
  }
  // weight of splits 0 .. s-1
  __device__ __forceinline__ int weight_before(const SplitRule& r, int s) const {
    int c = kSplitWeight * s;
#pragma unroll
    for (int j = 1; j < kMaxSlots; ++j) c -= r.tilt * (s > first[j] ? s - first[j] : 0);
    return c;
  }
};

// Rows of one 32-token tile: tokens 0..15 at rows gA.., 16..31 at gB..
struct TileDesc {
  int64_t gA, gB;
  int last;  // offsets [0, last] are valid tokens
};

__device__ __forceinline__ uint32_t f16_bits(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }

__device__ __forceinline__ f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// exponent e with |x| in [2^e, 2^(e+1)); 0 for x == 0
__device__ __forceinline__ int exponent_of(float x) {
  if (!(x > 0.0f)) return 0;
  int e;
  frexpf(x, &e);
  return e - 1;
}

// Workgroup barrier that waits for this wave's LDS operations only (global
// loads stay in flight).  The compiler barriers on both sides of the wait
// keep every LDS access of the code around it on its side: the wait
// intrinsic itself does not order memory operations.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLdsOnly);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Orders this wave's LDS writes before its later LDS reads of other lanes'
// data (a wave-local exchange; the workgroup's waves run independent tiles).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A wave-uniform 64-bit value, moved to SGPRs.
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// 2^x on the transcendental unit (v_exp_f32); denormal results flush to 0,
// which is harmless for softmax weights.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Value of lane (i + 8) within each 16-lane row (row_shl:8); lanes 8..15 of a
// row read 0.
__device__ __forceinline__ float dpp_row_shl8(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x108, 0xf, 0xf, true));
}

// Lanes of the banks (4-lane groups of a 16-lane row) in BANKS take `src` from
// the lane the DPP control CTRL names (row_shr:k = lane i - k); the others keep
// `old`.
template <int CTRL, int BANKS>
__device__ __forceinline__ float dpp_bank_move(float old, float src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, src),
                                                               CTRL, 0xf, BANKS, false));
}

// Rotation within each 16-lane row (CTRL = row_ror:k); fuses into the
// consuming max / add.
template <int CTRL>
__device__ __forceinline__ float dpp_row_ror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

// Raw buffer descriptor of a wave-uniform base address (no stride, no range
// limit): loads through it take the base from SGPRs and a 32-bit lane offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, -1, 0x00020000);
}
// a descriptor over `bytes` bytes from base (loads past them read zero)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc_n(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// (x & m) | c.  Plain code, not inline asm, so that the compiler sees the VALU
// write and keeps the wait states the matrix core needs before reading the
// result as an operand; with m in an SGPR and c in a VGPR it is one
// v_and_or_b32.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) { return (x & m) | c; }

// Two consecutive storage-dtype values -> fp32 (one 4- or 8-byte load; the
// element index must be even).
template <typename T>
__device__ __forceinline__ void load2(const T* p, float* out) {
  if constexpr (sizeof(T) == 2) {
    const uint32_t v = *(const uint32_t*)p;
    out[0] = Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)v));
    out[1] = Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(v >> 16)));
  } else {
    const float2 v = *(const float2*)p;
    out[0] = v.x; out[1] = v.y;
  }
}

// Eight consecutive storage-dtype values, kept packed as loaded (16 or 32
// bytes; the element index must be a multiple of 8) and widened on use.
template <typename T>
struct Pack8 {
  static constexpr int kWords = sizeof(T) == 2 ? 4 : 8;
  uint32_t w[kWords];
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (sizeof(T) == 2) {
      const uint4 v = *(const uint4*)p;
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
      const uint4 a = *(const uint4*)p, c = *(const uint4*)(p + 4);
      w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
      w[4] = c.x; w[5] = c.y; w[6] = c.z; w[7] = c.w;
    }
  }
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSidePolicy);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
    if constexpr (sizeof(T) == 4) {
      const u32x4 c = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, kSidePolicy);
      w[4] = c[0]; w[5] = c[1]; w[6] = c[2]; w[7] = c[3];
    }
  }
  __device__ __forceinline__ void set(int i, T v) {  // element-wise fill
    if constexpr (sizeof(T) == 2) {
      const uint32_t bits = (uint32_t)__builtin_bit_cast(uint16_t, v);
      w[i >> 1] = (i & 1) ? ((w[i >> 1] & 0xffffu) | (bits << 16)) : ((w[i >> 1] & 0xffff0000u) | bits);
    } else {
      w[i] = __builtin_bit_cast(uint32_t, v);
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (sizeof(T) == 2)
      return Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(w[i >> 1] >> (16 * (i & 1)))));
    else
      return __builtin_bit_cast(float, w[i]);
  }
};

// Waves per SIMD of the decode kernel: 4 (<= 128 VGPRs) with 16-bit norms and
// value metadata; 3 when either is fp32 (more registers per tile).
template <typename TN, typename TV>
constexpr int kDecodeWaves = (sizeof(TN) == 2 && sizeof(TV) == 2) ? 4 : 3;

// Two consecutive key norms, kept as loaded and widened on use.
template <typename T>
struct NormPair {
  uint32_t w[sizeof(T) == 2 ? 1 : 2];
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kSidePolicy);
    // (a second dword load: this toolchain lowers raw_buffer_load_b64 to one dword)
    if constexpr (sizeof(T) == 4) w[1] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 4, kSidePolicy);
  }
  __device__ __forceinline__ void load(const T* p) {  // element index even
    if constexpr (sizeof(T) == 2) {
      w[0] = *(const uint32_t*)p;
    } else {
      const uint2 v = *(const uint2*)p;
      w[0] = v.x; w[1] = v.y;
    }
  }
  __device__ __forceinline__ void set(int i, T v) {
    if constexpr (sizeof(T) == 2) {
      const uint32_t bits = (uint32_t)__builtin_bit_cast(uint16_t, v);
      w[0] = i ? ((w[0] & 0xffffu) | (bits << 16)) : ((w[0] & 0xffff0000u) | bits);
    } else {
      w[i] = __builtin_bit_cast(uint32_t, v);
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (sizeof(T) == 2)
      return Num<T>::to_f(__builtin_bit_cast(T, (uint16_t)(w[0] >> (16 * i))));
    else
      return __builtin_bit_cast(float, w[i]);
  }
};

// Two output elements (o0, o1) at element offset oi of the output.
__device__ __forceinline__ void store_out2(const smaq_attn_params& p, int64_t oi, float o0, float o1) {
  switch (p.out_dtype) {
    case SMAQ_F32: {
      float* o = (float*)p.out + oi;
      o[0] = o0;
      o[1] = o1;
    } break;
    case SMAQ_F16: {
      _Float16* o = (_Float16*)p.out + oi;
      o[0] = Num<_Float16>::from_f(o0);
      o[1] = Num<_Float16>::from_f(o1);
    } break;
    default: {
      bf16* o = (bf16*)p.out + oi;
      o[0] = Num<bf16>::from_f(o0);
      o[1] = Num<bf16>::from_f(o1);
    } break;
  }
}

// NaN test on the bits: this file is built with -fno-honor-nans, under
// which a floating-point self-comparison folds to false.
__device__ __forceinline__ bool is_nan_bits(float x) {
  return (__builtin_bit_cast(uint32_t, x) & 0x7fffffffu) > 0x7f800000u;
}
constexpr float kQuietNaN = __builtin_bit_cast(float, 0x7fc00000u);

// x rounded to the output dtype (kept in fp32).
__device__ __forceinline__ float round_out(const smaq_attn_params& p, float x) {
  switch (p.out_dtype) {
    case SMAQ_F32: return x;
    case SMAQ_F16: return Num<_Float16>::round(x);
    default: return Num<bf16>::round(x);
  }
}

// Agent-coherent (device-scope relaxed atomic) stores and loads: on gfx950
// they carry the sc1 cache policy, so a store is written through the XCD's
// L2 and a load misses a stale L2 line, without cache-wide maintenance.
__device__ __forceinline__ void store_agent(float* a, float v) {
  __hip_atomic_store((uint32_t*)a, __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(float* a, f32x2 v) {
  __hip_atomic_store((uint64_t*)a, __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* a) {
  return __builtin_bit_cast(float, __hip_atomic_load((const uint32_t*)a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ f32x2 load_agent2(const float* a) {
  return __builtin_bit_cast(f32x2, __hip_atomic_load((const uint64_t*)a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// VBUF (16-token pages, a value pool below 4 GB): the value loads address the
// pool through one descriptor with 32-bit lane offsets instead of 64-bit
// per-lane addresses (c5 kernel 398.6-399.1 -> 394.7-395.5 us and
// 378.5-378.9 -> 374.2-374.8 us, three alternating rounds on each of two
// boxes; non-temporal there was slower: 421.5-425.3 us; so were the norms,
// scales and zeros through such descriptors as well: 373.6-373.9 against
// 371.6-371.9 us)
template <int KBITS, typename TN, typename TV, bool SPLIT, bool VBUF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kDecodeWaves<TN, TV>, kDecodeWaves<TN, TV>))) void decode_mfma_kernel(
    smaq_attn_params p, HistAddr addr, Partials part, SplitRule rule, const int* __restrict__ order) {
  // key LUT, one 8-byte entry per code byte: {f16 hi pair, f16 lo pair}
  // (read with ds_read_b64, twice the rate of two dword reads)
  __shared__ __attribute__((aligned(16))) u32x2 lut[256];
  // query B operands (one u32x4 per lane and K step), shared by the 4 waves
  __shared__ __attribute__((aligned(16))) u32x4 bqs[8][64];
  // per wave: value codes spread to 16 bits ([code byte][token pair] dwords)
  // and the PV A operand ([row][hi 32 tokens | lo 32 tokens] bf16)
  __shared__ __attribute__((aligned(16))) uint8_t vsp[kMWaves][32 * kVRow];
  __shared__ __attribute__((aligned(16))) uint8_t ast[kMWaves][16 * kARow];
  __shared__ float red_m[kMWaves][4];
  __shared__ float red_l[kMWaves][4];
  __shared__ int last_split;  // merge: this workgroup is its unit's last arrival
  // per-wave results, laid over the spread tiles once every wave has left its loop
  float (*const red_o)[4][128] = (float (*)[4][128])&vsp[0][0];

  // Thread and workgroup ids come from the hardware registers directly: this
  // file is built without IEEE mode, which keeps the device library's
  // accessors (threadIdx, blockIdx) from being inlined.
  const int tid = (int)__builtin_amdgcn_workitem_id_x();
  const int gx = (int)__builtin_amdgcn_workgroup_id_x(), gy = (int)__builtin_amdgcn_workgroup_id_y();
  const int gz = (int)__builtin_amdgcn_workgroup_id_z();
  const int lane = tid & 63, w = tid >> 6;
  const int wu = __builtin_amdgcn_readfirstlane(w);  // wave index, in an SGPR
  const int n = lane & 15, kg = lane >> 4;           // MFMA lane coordinates
  const int bank = n >> 2, qq = n & 3;               // softmax layout: bank, query row
  // this lane's two softmax tokens: C-layout values 2*bank, 2*bank + 1
  const int tokA = bank < 2 ? 4 * kg + 2 * bank : 16 + 4 * kg + 2 * (bank - 2);
  const int tq = lane & 7, pq = lane >> 3;           // value loader: tokens 4tq.., bytes 4pq..
  // per-sequence lookups go through the scalar cache (no vector-memory wait
  // in the prologue)
  typedef const __attribute__((address_space(4))) int* ConstIntPtr;
  typedef const __attribute__((address_space(4))) int64_t* ConstI64Ptr;
  // Longest-first dispatch (one split per unit): the KV heads of a sequence
  // share cache lines of the pools (a 16-token page's norms, scales and
  // zeros are runs shorter than a line, next to the other heads' runs), and
  // workgroup f runs on XCD f mod 8.  So each group of 8 sequences (in
  // dispatch order) takes 8 * Hkv consecutive workgroups f = base + 8 h + i,
  // which puts every head of sequence i on one XCD and its shared lines in
  // one L2 (c5: HBM traffic +6.0% -> +0.8% over the algorithmic bytes).
  // In item mode the same grouping runs over work items (the pieces of a
  // sequence are consecutive items).
  int hsel = gx, osel = gy;
  if (order) {
    const int hk = p.n_kv_heads;
    const int f = gx + hk * gy;
    const int rows = rule.pieces ? rule.items : p.batch;
    if (f < (rows / 8) * 8 * hk) {
      const int grp = f / (8 * hk), rem = f - grp * 8 * hk;
      hsel = rem >> 3;
      osel = 8 * grp + (rem & 7);
    }
  }
  const int h = __builtin_amdgcn_readfirstlane(hsel);
  int b, s, nsplit;
  int64_t s0 = 0, s1 = 0;
  if (rule.pieces) {
    const ConstIntPtr it = (ConstIntPtr)order + 4 * __builtin_amdgcn_readfirstlane(osel);
    const int seq = it[0], t0 = it[1], t1 = it[2], meta = it[3];  // one 16-byte scalar load
    b = __builtin_amdgcn_readfirstlane(seq);
    // b < 0: no work (uniform over the workgroup).  The range checks keep a
    // stale schedule (phase 16 on a workspace the lengths no longer match)
    // inside the buffers; its results are then undefined.
    if ((unsigned)b >= (unsigned)p.batch) return;
    s1 = min((int64_t)__builtin_amdgcn_readfirstlane(t1), p.max_hist_len);
    s0 = min((int64_t)__builtin_amdgcn_readfirstlane(t0), s1);
    s0 = s0 < 0 ? 0 : s0;
    nsplit = __builtin_amdgcn_readfirstlane(meta >> 16);
    nsplit = nsplit < 1 ? 1 : (nsplit > rule.n_splits ? rule.n_splits : nsplit);
    s = __builtin_amdgcn_readfirstlane(meta & 0xffff);
    s = s < nsplit ? s : nsplit - 1;
  } else {
    b = order ? ((ConstIntPtr)order)[__builtin_amdgcn_readfirstlane(osel)] : gy;
    if (order && (unsigned)b >= (unsigned)p.batch) return;  // a stale order (as above)
    s = gz;
    nsplit = rule.n_splits;
  }
  const int Q = p.n_q_heads / p.n_kv_heads;  // query rows (decode: one token)
  constexpr uint32_t kMask = (1u << KBITS) - 1u;
  constexpr float kLog2e = 1.4426950408889634f;

  // The prologue's two global reads (the query rows, the key centroids) are
  // issued together: the query rows first, as vector loads; the centroids as
  // scalar loads, each lane taking its table entries from them by index.
  const int qrow = n < Q ? n : ((n >= 8 && n < 8 + Q) ? n - 8 : -1);
  const int64_t qrow0 = (int64_t)b * p.n_q_heads + h * Q;  // first query row of this KV head
  const float* qsrc = p.q_hist + (qrow0 + (qrow < 0 ? 0 : qrow)) * 128;
  // (padding columns read query row 0 and drop it: loads without a branch)
  float qv[32];
#pragma unroll
  for (int i = 0; i < 32; i += 4) {
    const float4 v4 = *(const float4*)(qsrc + 32 * kg + i);
    qv[i] = v4.x; qv[i + 1] = v4.y; qv[i + 2] = v4.z; qv[i + 3] = v4.w;
  }
  // (nothing below is scheduled above the query loads: they need only the
  // query pointer and the head counts, and go out before the other argument
  // reads and their waits)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 32; ++i) qv[i] = qrow < 0 ? 0.0f : qv[i];
  float cent[1 << KBITS];
  typedef const __attribute__((address_space(4))) float* ConstFloatPtr;
  const ConstFloatPtr klut = (ConstFloatPtr)p.key_lut;
#pragma unroll
  for (int i = 0; i < (1 << KBITS); ++i) cent[i] = klut[i];

  // ---- split range: split s of this sequence and head holds
  // tokens [s0, s1) (wave-uniform values are pinned to SGPRs so the tile
  // loop's control flow and address arithmetic stay scalar); an item
  // carries its range
  if (!rule.pieces) {
    s1 = uniform64(p.hist_len ? min(((ConstI64Ptr)p.hist_len)[b], (int64_t)p.max_hist_len) : p.max_hist_len);
  }
  if (!rule.pieces && rule.n_splits > 1) {
    const int64_t len = s1;
    // (a shared boundary is computed by the same expression for both of its
    // splits, so rounding cannot open a gap or an overlap)
    const int units = p.n_kv_heads * p.batch, u = h + p.n_kv_heads * gy;
    const SlotStarts starts(rule, u, units);
    const double per_weight = (double)len / (double)starts.weight_before(rule, rule.n_splits);
    constexpr int64_t kStepMask = ~(int64_t)(kMWaves * kMTile - 1);
    if (s > 0) s0 = (int64_t)(per_weight * starts.weight_before(rule, s)) & kStepMask;
    if (s + 1 < rule.n_splits) s1 = (int64_t)(per_weight * starts.weight_before(rule, s + 1)) & kStepMask;
  }
  s0 = uniform64(s0);
  s1 = uniform64(s1);
  const uint8_t* kbytes = (const uint8_t*)p.key_bytes;
  const uint8_t* vbytes = (const uint8_t*)p.val_bytes;
  // (VBUF: the value pool, 32-byte rows, as one range-checked descriptor)
  const auto vpool = buf_rsrc_n(vbytes, VBUF ? (uint32_t)addr.rows * 32u : 0u);
  const TN* norms = (const TN*)p.key_norms;
  const TV* vsc = (const TV*)p.val_scales;
  const TV* vzr = (const TV*)p.val_zeros;

  // row of history token t0g (a multiple of 16): rows t0g .. t0g + 15 are
  // consecutive in both layouts (paged blocks hold a multiple of 16 tokens)
  const int64_t contig_base = uniform64(addr.table ? 0
      : (int64_t)h * addr.head_stride + (addr.seq_start ? ((ConstI64Ptr)addr.seq_start)[b] : (int64_t)b * addr.uniform_len));
  // block table row of this sequence, read through the scalar cache
  const bool paged = __builtin_amdgcn_readfirstlane(addr.table != nullptr ? 1 : 0) != 0;
  const ConstIntPtr tbl =
      (ConstIntPtr)uniform64(paged ? (int64_t)(uintptr_t)(addr.table + (int64_t)b * addr.max_blocks) : 0);
  const int bsz = addr.block_size;          // a power of two (checked on the host)
  const int n_kv = addr.n_kv;
  const int bshift = __builtin_ctz((unsigned)bsz);
  if (rule.pieces && paged) {
    // (a stale item's range stays inside the block-table row)
    s1 = uniform64(min(s1, (int64_t)addr.max_blocks << bshift));
    s0 = uniform64(min(s0, s1));
  }
  auto group_row = [&](int64_t t0g) -> int64_t {
    if (!paged) return contig_base + t0g;
    const uint32_t tg = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)t0g);
    const uint32_t blk_i = tg >> bshift;
    const int blk = __builtin_amdgcn_readfirstlane(tbl[blk_i]);
    return ((int64_t)blk * n_kv + h) * bsz + (tg & (uint32_t)(bsz - 1));
  };

  // Tile t (first token; a multiple of 32 past the split start): its rows and
  // validity.  Offsets [0, last] are valid tokens; a tail tile clamps rows onto
  // the last valid token.
  auto describe = [&](int64_t t) -> TileDesc {
    TileDesc d;
    d.last = __builtin_amdgcn_readfirstlane((int)min((int64_t)31, s1 - 1 - t));
    d.gA = uniform64(group_row(t));
    d.gB = uniform64(d.last >= 16 ? group_row(t + 16) : d.gA);
    return d;
  };
  auto rowof = [&](const TileDesc& d, int i) -> int64_t {
    const int c = min(i, d.last);
    return c < 16 ? d.gA + c : d.gB + (c - 16);
  };

  // Full tiles with even rows.  Without SPLIT the second 16-token group
  // follows the first (gB = gA + 16): every array is read through a buffer
  // descriptor of the tile's first row (SGPRs) plus a constant lane offset, so
  // a tile costs no vector address arithmetic.  With SPLIT (16-token pages)
  // the lanes of the second group read from another block and take 64-bit
  // row addresses.
  const uint32_t offK = (uint32_t)(n * 64 + 16 * kg);
  const uint32_t offV = (uint32_t)(128 * tq + 4 * pq);  // rows 4tq.. (both groups when gB = gA + 16)
  auto fast_values = [&](const TileDesc& d, uint32_t* vd) {
    if constexpr (SPLIT && VBUF) {
      // (the rows fit 32 bits: the pool is below 4 GB)
      const uint32_t vo = ((uint32_t)(tq < 4 ? d.gA : d.gB) + 4u * (uint32_t)(tq & 3)) * 32u + 4u * (uint32_t)pq;
#pragma unroll
      for (int i = 0; i < 4; ++i) vd[i] = __builtin_amdgcn_raw_buffer_load_b32(vpool, vo, 32 * i, 0);
    } else if constexpr (SPLIT) {
      const uint8_t* vrow = vbytes + ((tq < 4 ? d.gA : d.gB) + 4 * (tq & 3)) * 32 + 4 * pq;
#pragma unroll
      for (int i = 0; i < 4; ++i) vd[i] = *(const uint32_t*)(vrow + 32 * i);
    } else {
      const auto rv = buf_rsrc(vbytes + d.gA * 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) vd[i] = __builtin_amdgcn_raw_buffer_load_b32(rv, offV, 32 * i, kValPolicy);
    }
  };
  auto fast_keys = [&](const TileDesc& d, u32x4& kqa, u32x4& kqb) {
    kqa = __builtin_amdgcn_raw_buffer_load_b128(buf_rsrc(kbytes + d.gA * 64), offK, 0, kKeyPolicy);
    kqb = __builtin_amdgcn_raw_buffer_load_b128(buf_rsrc(kbytes + d.gB * 64), offK, 0, kKeyPolicy);
  };
  // this lane's first softmax token row (tokens tokA, tokA + 1 are consecutive rows)
  auto rowA = [&](const TileDesc& d) -> int64_t { return tokA < 16 ? d.gA + tokA : d.gB + (tokA - 16); };
  auto fast_norms = [&](const TileDesc& d, NormPair<TN>& nrm) {
    if constexpr (SPLIT) nrm.load(norms + rowA(d));
    else nrm.load_buf(buf_rsrc(norms + d.gA), (uint32_t)(tokA * sizeof(TN)));
  };
  auto fast_side = [&](const TileDesc& d, Pack8<TV>& sv, Pack8<TV>& zv) {
    if constexpr (SPLIT) {
      const int64_t r = rowA(d);
      sv.load(vsc + r * 4);
      zv.load(vzr + r * 4);
    } else {
      const uint32_t o = (uint32_t)(tokA * 4 * sizeof(TV));
      sv.load_buf(buf_rsrc(vsc + d.gA * 4), o);
      zv.load_buf(buf_rsrc(vzr + d.gA * 4), o);
    }
  };
  // Any tile (tail or odd rows): element loads with clamped rows.
  auto slow_loads = [&](const TileDesc& d, u32x4& kqa, u32x4& kqb, uint32_t* vd, NormPair<TN>& nrm,
                        Pack8<TV>& sv, Pack8<TV>& zv) {
#pragma unroll
    for (int i = 0; i < 4; ++i) vd[i] = *(const uint32_t*)(vbytes + rowof(d, 4 * tq + i) * 32 + 4 * pq);
    kqa = *(const u32x4*)(kbytes + rowof(d, n) * 64 + 16 * kg);
    kqb = *(const u32x4*)(kbytes + rowof(d, 16 + n) * 64 + 16 * kg);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t r = rowof(d, tokA + i);
      nrm.set(i, norms[r]);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        sv.set(4 * i + g, vsc[r * 4 + g]);
        zv.set(4 * i + g, vzr[r * 4 + g]);
      }
    }
  };

  u32x4 kqa, kqb;
  uint32_t vd[4];
  NormPair<TN> nrm;
  Pack8<TV> sv, zv;
  auto none = [] {};
  int64_t t0 = s0 + (int64_t)wu * kMTile;
  // Pipelined loops over full tiles with even rows (paged rows always are;
  // contiguous rows when the head's first row is even).  Each iteration
  // issues the next tile's loads once this tile's registers are consumed, so
  // every load has one iteration to arrive; the last iteration reloads its
  // own rows (cache hits) to keep the load sequence identical.
  const bool even_rows = paged || (contig_base & 1) == 0;
  // Contiguous rows: the split's full 128-token steps (one 32-token tile per
  // wave) in a rotated order whose start differs between workgroups.  Every
  // split starts at the same offset of its sequence's arrays, so without the
  // rotation concurrent workgroups stream the same address phase; measured on
  // MI355X, the rotation alone takes the load stream from 5.6 to 5.9 TB/s.
  // The next row is formed without a branch: with a branch at the loop top
  // the compiler waits for every load of the tile there instead of for each
  // array when it is first used.  The start follows from the (KV head,
  // sequence, split) only, not from the grid position, which a longest-first
  // order assigns by atomics within a length bucket: the summation order, so
  // the output bits, must not depend on the schedule.
  const int64_t n_steps = (s1 - s0) / (kMWaves * kMTile);
  constexpr int64_t kStep = kMWaves * kMTile;
  const bool rot = !paged && even_rows && n_steps > 0;
  const int K = __builtin_amdgcn_readfirstlane((int)(rot ? n_steps : 1));
  const int r = __builtin_amdgcn_readfirstlane(
      (int)(((unsigned)h * 7u + (unsigned)b * 13u + (unsigned)s * 5u) % (unsigned)K));
  const int64_t base = uniform64(contig_base + s0 + (int64_t)wu * kMTile);  // step 0 of this wave
  const int64_t wrap = (int64_t)K * kStep;
  const int64_t rot_end = base + wrap;
  int64_t row = uniform64(base + (int64_t)r * kStep);
  // The rotated loop's first tile is pulled into the caches here, ahead of
  // the prologue's own work, so that its loads after the prologue hit L2
  // instead of paying a full memory round trip: one dword per lane, every
  // 128-byte line of the tile's five arrays touched by some lane (a point
  // every 128 bytes from each array's first byte, the last at its last dword).
  // Other paths read the query row instead: the load is issued on every path,
  // because a load under a branch makes the compiler wait for every load
  // where the paths join.
  uint32_t warm;
  {
    constexpr int kKeyPts = 17, kValPts = 9, kNrmPts = 2;  // 2 KB, 1 KB, <= 128 B
    constexpr int kSidePts = sizeof(TV) == 2 ? 3 : 5;      // 256 or 512 B each
    constexpr int kBytesSide = 32 * 4 * (int)sizeof(TV);
    const uint8_t* pt = (const uint8_t*)qsrc;
    int k = lane;
    auto point = [&](const void* arr, int bytes, int npts) {
      if (k >= 0 && k < npts) pt = (const uint8_t*)arr + min(128 * k, bytes - 4);
      k -= npts;
    };
    point(kbytes + row * 64, 32 * 64, kKeyPts);
    point(vbytes + row * 32, 32 * 32, kValPts);
    point(norms + row, 32 * (int)sizeof(TN), kNrmPts);
    point(vsc + row * 4, kBytesSide, kSidePts);
    point(vzr + row * 4, kBytesSide, kSidePts);
    if (!rot) pt = (const uint8_t*)qsrc;
    warm = *(const uint32_t*)pt;
  }

  // ---- key LUT: byte (c0 | c1 << KBITS) -> packed f16 hi / lo of both codes,
  // centroids pre-scaled by 2^-e_lut so the largest has magnitude in [1, 2)
  float cmax = 0.0f;
#pragma unroll
  for (int i = 0; i < (1 << KBITS); ++i) cmax = fmaxf(cmax, fabsf(cent[i]));
  const int e_lut = exponent_of(cmax);
  const float lut_scale = ldexpf(1.0f, -e_lut);
  {
    const int v = tid;  // 256 threads, one entry each
    float c0 = cent[0], c1 = cent[0];
#pragma unroll
    for (int i = 1; i < (1 << KBITS); ++i) {
      c0 = (v & kMask) == (uint32_t)i ? cent[i] : c0;
      c1 = ((v >> KBITS) & kMask) == (uint32_t)i ? cent[i] : c1;
    }
    c0 *= lut_scale;
    c1 *= lut_scale;
    const _Float16 h0 = (_Float16)c0, h1 = (_Float16)c1;
    const _Float16 l0 = (_Float16)(c0 - (float)h0), l1 = (_Float16)(c1 - (float)h1);
    lut[v] = u32x2{f16_bits(h0) | (f16_bits(h1) << 16), f16_bits(l0) | (f16_bits(l1) << 16)};
  }

  // ---- query B operands: columns [0, Q) hold the hi parts of query rows
  // 0..Q-1, columns [8, 8+Q) their lo parts, the rest zero
  float qmax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) qmax = fmaxf(qmax, fabsf(qv[i]));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 16, 64));
  qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
  const int e_q = exponent_of(qmax);
  const float q_scale = ldexpf(1.0f, -e_q);
  // Step st (0..7) covers dims d = 32kg + 4st + {0..3}; its 8 k-elements are
  // [x(d0) x(d1) y(d0) y(d1) x(d2) x(d3) y(d2) y(d3)], matched on the key side by
  // [hi(d0) hi(d1) lo(d0) lo(d1) hi(d2) hi(d3) lo(d2) lo(d3)] (two LUT pairs).
  // x = q hi (columns < Q) or q lo (columns 8..8+Q), y = q hi (columns < Q), so
  // column j + column 8+j = qh.kh + qh.kl + ql.kh.
  if (w == 0) {
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      uint32_t xw[2], yw[2];
#pragma unroll
      for (int pr2 = 0; pr2 < 2; ++pr2) {
        uint32_t xx = 0, yy = 0;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const float x = qv[4 * st + 2 * pr2 + hh] * q_scale;
          const _Float16 hi = (_Float16)x;
          const _Float16 lo = (_Float16)(x - (float)hi);
          const uint32_t hb = f16_bits(hi), lb = f16_bits(lo);
          xx |= (n < Q ? hb : (qrow >= 0 ? lb : 0u)) << (16 * hh);
          yy |= (n < Q ? hb : 0u) << (16 * hh);
        }
        xw[pr2] = xx;
        yw[pr2] = yy;
      }
      bqs[st][lane] = u32x4{xw[0], yw[0], xw[1], yw[1]};
    }
  }
  // score factor of query row qq: scale * log2(e) * 2^(e_q + e_lut), taken
  // from column qq (its hi column)
  const float rfac = __shfl(p.scale * kLog2e * ldexpf(1.0f, e_q + e_lut), qq, 64);
  // LDS-only barrier: the first tile's global loads stay in flight
  lds_barrier();

  // reference max / running sum of query row qq (max replicated over its 16
  // lanes; the sum is this lane's share, reduced once at the end)
  float m_run = -__builtin_inff(), l_run = 0.0f;
  f32x4 acc_o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc_o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 acc_s = {0.f, 0.f, 0.f, 0.f};  // sum of A per row (query kg, group v)
  float zacc[4] = {0.f, 0.f, 0.f, 0.f};  // this lane's share of sum p * zero, query qq
  const u32x4 kOnesBf16 = u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  // bf16 128.0 in both halves, and the four 2-bit field masks of a spread
  // code byte; hidden from constant folding so that each B operand dword is a
  // single v_and_or_b32 (mask from an SGPR, base from a VGPR) rather than an
  // and plus an or with two literals
  uint32_t bf16_base = 0x43004300u;
  asm volatile("" : "+v"(bf16_base));
  uint32_t fmask[4] = {0x00030003u, 0x000c000cu, 0x00300030u, 0x00600060u};
#pragma unroll
  for (int f = 0; f < 4; ++f) asm volatile("" : "+s"(fmask[f]));

  // LDS addresses (lane constants)
  uint8_t* const vw = &vsp[w][kVRow * 4 * pq + 8 * tq];       // spread writer, code byte 4pq
  const uint8_t* const vr = &vsp[w][kVRow * n + 16 * kg];     // B reader: byte n (+16 rows: 16+n)
  uint8_t* const aw = &ast[w][kARow * 4 * qq + 4 * (tokA >> 1)];  // A writer: row (qq, group 0)
  const uint8_t* const ar = &ast[w][kARow * n + 16 * kg];     // A reader: row n, tokens 8kg..

  float m_thr = -__builtin_inff();  // m_run + kLazyRescale
  // One tile.  The hooks run right after the tile's copy of the matching
  // registers has been consumed (the pipelined loop loads the next tile there).
  auto tile = [&](auto tail_tag, int last, u32x4& kqa, u32x4& kqb, uint32_t* vd, NormPair<TN>& nrm,
                  Pack8<TV>& sv, Pack8<TV>& zv, auto&& after_values, auto&& after_keys,
                  auto&& after_norms, auto&& after_side) {
    constexpr bool TAIL = decltype(tail_tag)::value;
    // -- value codes spread to 16 bits: dword (byte j, tokens 2i, 2i+1) =
    // [code byte of token 2i, 0, code byte of token 2i+1, 0]
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + j) << 16) | (uint32_t)j;
      uint2 pr2;
      pr2.x = __builtin_amdgcn_perm(vd[1], vd[0], sel);
      pr2.y = __builtin_amdgcn_perm(vd[3], vd[2], sel);
      *(uint2*)(vw + kVRow * j) = pr2;
    }
    after_values();
    // -- QK: per step two key bytes -> two LUT pairs -> one A operand
    f32x4 ca = {0.f, 0.f, 0.f, 0.f}, cb = {0.f, 0.f, 0.f, 0.f};
    typedef const __attribute__((address_space(3))) u32x4 LdsU32x4;
    const LdsU32x4* bqp = (const LdsU32x4*)&bqs[0][lane];
    asm volatile("" : "+v"(bqp));  // read each tile (keeps the operands out of registers)
    // The matrix sections run at raised wave priority: the four waves of a
    // SIMD drift apart (no workgroup barrier in the loop), and letting the
    // wave in its MFMA chain issue first while the others fill in VALU work
    // measured 2% faster (0.1928 -> 0.1884 ms at c3).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const u32x4 bqv = bqp[64 * st];
      const uint32_t wa = kqa[st >> 1] >> (16 * (st & 1)), wb = kqb[st >> 1] >> (16 * (st & 1));
      const uint32_t a0 = wa & 0xffu, a1 = (wa >> 8) & 0xffu;
      const uint32_t b0 = wb & 0xffu, b1 = (wb >> 8) & 0xffu;
      const u32x2 pa0 = lut[a0], pa1 = lut[a1], pb0 = lut[b0], pb1 = lut[b1];
      const u32x4 av = u32x4{pa0[0], pa0[1], pa1[0], pa1[1]};
      const u32x4 bv = u32x4{pb0[0], pb0[1], pb1[0], pb1[1]};
      ca = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(av), as_f16x8(bqv), ca, 0, 0, 0);
      cb = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_f16x8(bv), as_f16x8(bqv), cb, 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    after_keys();
    // -- scores.  C layout: lane (kg, n) holds column n for tokens 4kg + v (ca)
    // and 16 + 4kg + v (cb).  Add the lo column n + 8 (row_shl:8), then move
    // values 2*bank, 2*bank + 1 of column qq into bank `bank` of the same row.
    float sc[8];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sc[v] = ca[v] + dpp_row_shl8(ca[v]);
      sc[4 + v] = cb[v] + dpp_row_shl8(cb[v]);
    }
    float x0 = sc[0], x1 = sc[1];
    x0 = dpp_bank_move<0x114, 0x2>(x0, sc[2]);  // row_shr:4 into bank 1
    x1 = dpp_bank_move<0x114, 0x2>(x1, sc[3]);
    x0 = dpp_bank_move<0x118, 0x4>(x0, sc[4]);  // row_shr:8 into bank 2
    x1 = dpp_bank_move<0x118, 0x4>(x1, sc[5]);
    x0 = dpp_bank_move<0x11c, 0x8>(x0, sc[6]);  // row_shr:12 into bank 3
    x1 = dpp_bank_move<0x11c, 0x8>(x1, sc[7]);
    x0 *= nrm.get(0);  // score / rfac (rfac > 0 is applied in the exponent)
    x1 *= nrm.get(1);
    after_norms();
    if constexpr (TAIL) {
      if (tokA > last) x0 = -__builtin_inff();
      if (tokA + 1 > last) x1 = -__builtin_inff();
    }
    // -- online softmax (base 2) of query row qq over its 16 lanes, with a
    // lazily raised reference maximum: weights may grow to 2^kLazyRescale
    // before the row maximum is reduced and the accumulators rescaled.
    const float tmax = fmaxf(x0, x1) * rfac;
    if (__any(tmax > m_thr)) {
      float mt = tmax;
      mt = fmaxf(mt, dpp_row_ror<0x124>(mt));
      mt = fmaxf(mt, dpp_row_ror<0x128>(mt));
      mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float m_new = fmaxf(m_run, mt);
      // rows qq >= Q are padding: their factor stays 1
      const float alpha = qq >= Q ? 1.0f : ((m_run == -__builtin_inff()) ? 0.0f : fast_exp2(m_run - m_new));
      const float a_o = __shfl(alpha, kg, 64);  // O rows: query kg (lane kg holds row kg)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc_o[i] *= a_o;
      acc_s *= a_o;
#pragma unroll
      for (int g = 0; g < 4; ++g) zacc[g] *= alpha;
      l_run *= alpha;
      m_run = m_new;
      m_thr = m_new + kLazyRescale;
    }
    // exp2(-inf) = 0 covers masked tokens; only a row with no valid token yet
    // (m_run = -inf, possible in a tail tile) needs the guard against inf - inf
    float p0, p1;
    if constexpr (TAIL) {
      const bool dead = m_run == -__builtin_inff();
      p0 = dead ? 0.0f : fast_exp2(fmaf(x0, rfac, -m_run));
      p1 = dead ? 0.0f : fast_exp2(fmaf(x1, rfac, -m_run));
    } else {
      p0 = fast_exp2(fmaf(x0, rfac, -m_run));
      p1 = fast_exp2(fmaf(x1, rfac, -m_run));
    }
    l_run += p0 + p1;
    // -- PV A operand (row (qq, g), tokens tokA, tokA + 1): p * scale split into
    // a bf16 hi part (truncation, exact remainder) and a rounded bf16 lo part
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float ps0 = p0 * sv.get(g), ps1 = p1 * sv.get(4 + g);
      const uint32_t h0 = __builtin_bit_cast(uint32_t, ps0) & 0xffff0000u;
      const uint32_t h1 = __builtin_bit_cast(uint32_t, ps1) & 0xffff0000u;
      const f32x2 lo2 = {ps0 - __builtin_bit_cast(float, h0), ps1 - __builtin_bit_cast(float, h1)};
      const uint32_t hp = __builtin_amdgcn_perm(h1, h0, 0x07060302u);
      const uint32_t lp = __builtin_bit_cast(uint32_t, __builtin_convertvector(lo2, bf16x2));
      *(uint32_t*)(aw + kARow * g) = hp;
      *(uint32_t*)(aw + kARow * g + 64) = lp;
      zacc[g] = fmaf(p1, zv.get(4 + g), fmaf(p0, zv.get(g), zacc[g]));
    }
    after_side();
    wave_sync();
    // -- PV.  A: rows (query kg', group g') x tokens 8kg..8kg+7.  B: column n of
    // step tau is code byte 16*(tau & 1) + n, bit field f = tau >> 1 (dim
    // 4 * byte + f), as the bf16 value 128 + (c << 2f) (f = 3: 128 + 32c), so
    // each step is one and-or per dword.
    const u32x4 ahi = *(const u32x4*)(ar);
    const u32x4 alo = *(const u32x4*)(ar + 64);
    const u32x4 w0 = *(const u32x4*)(vr);
    const u32x4 w1 = *(const u32x4*)(vr + kVRow * 16);
    __builtin_amdgcn_s_setprio(1);
    acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ahi), as_bf16x8(kOnesBf16), acc_s, 0, 0, 0);
    acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(alo), as_bf16x8(kOnesBf16), acc_s, 0, 0, 0);
#pragma unroll
    for (int tau = 0; tau < 8; ++tau) {
      const u32x4 wv = (tau & 1) ? w1 : w0;
      const int f = tau >> 1;
      u32x4 bv;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        bv[i] = f < 3 ? and_or(wv[i], fmask[f], bf16_base) : and_or(wv[i] >> 1, fmask[3], bf16_base);
      acc_o[tau] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ahi), as_bf16x8(bv), acc_o[tau], 0, 0, 0);
      acc_o[tau] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(alo), as_bf16x8(bv), acc_o[tau], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    wave_sync();  // this tile's LDS reads complete before the next tile's writes
  };

  if (rot) {
    const TileDesc dc{row, row + 16, 31};
    fast_values(dc, vd);
    fast_keys(dc, kqa, kqb);
    fast_norms(dc, nrm);
    fast_side(dc, sv, zv);
    asm volatile("" ::"v"(warm));  // keeps the warm-up load (done by now)
    for (int i = 0;;) {
      ++i;
      const bool more = i < K;
      int64_t rn = row + (more ? kStep : 0);
      rn = uniform64(rn >= rot_end ? rn - wrap : rn);
      const TileDesc dn{rn, rn + 16, 31};
      tile(std::false_type{}, 31, kqa, kqb, vd, nrm, sv, zv, [&] { fast_values(dn, vd); },
           [&] { fast_keys(dn, kqa, kqb); }, [&] { fast_norms(dn, nrm); }, [&] { fast_side(dn, sv, zv); });
      row = rn;
      if (!more) break;
    }
    t0 += n_steps * kStep;
  } else if (paged && t0 + kMTile <= s1) {
    // Paged rows: a counted loop over this wave's full tiles.  The block
    // table entries of a tile are loaded (scalar loads) one iteration before
    // its rows are formed, so the loop never waits on a table lookup, and
    // the row is (block * Hkv + h) << log2(block_size) + offset with the
    // block-times-head product in 32 bits (the pool has < 2^32 block-heads).
    constexpr int64_t kStep = kMWaves * kMTile;
    const int K = __builtin_amdgcn_readfirstlane((int)((s1 - t0 - kMTile) / kStep + 1));
    const uint32_t t_first = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)t0);
    const uint32_t bmask = (uint32_t)bsz - 1u;
    auto entries = [&](int k, uint32_t& ea, uint32_t& eb) {
      const uint32_t t = t_first + (uint32_t)k * (uint32_t)kStep;
      ea = (uint32_t)__builtin_amdgcn_readfirstlane(tbl[t >> bshift]);
      eb = (uint32_t)__builtin_amdgcn_readfirstlane(tbl[(t + 16u) >> bshift]);
    };
    auto rows_of = [&](int k, uint32_t ea, uint32_t eb) -> TileDesc {
      const uint32_t t = t_first + (uint32_t)k * (uint32_t)kStep;
      const int64_t ga = (int64_t)((uint64_t)(ea * (uint32_t)n_kv + (uint32_t)h) << bshift) + (int64_t)(t & bmask);
      const int64_t gb = (int64_t)((uint64_t)(eb * (uint32_t)n_kv + (uint32_t)h) << bshift) +
                         (int64_t)((t + 16u) & bmask);
      return TileDesc{uniform64(ga), uniform64(gb), 31};
    };
    uint32_t ea, eb, na, nb;
    entries(0, ea, eb);
    const TileDesc d0 = rows_of(0, ea, eb);
    fast_values(d0, vd);
    fast_keys(d0, kqa, kqb);
    fast_norms(d0, nrm);
    fast_side(d0, sv, zv);
    entries(K > 1 ? 1 : 0, na, nb);  // the tile after the first
    for (int i = 0;;) {
      ++i;
      const bool more = i < K;
      const int kn = more ? i : i - 1;   // the last tile reloads its own rows
      const TileDesc dn = rows_of(kn, na, nb);
      uint32_t fa, fb;
      entries(i + 1 < K ? i + 1 : K - 1, fa, fb);  // one more tile ahead
      tile(std::false_type{}, 31, kqa, kqb, vd, nrm, sv, zv, [&] { fast_values(dn, vd); },
           [&] { fast_keys(dn, kqa, kqb); }, [&] { fast_norms(dn, nrm); }, [&] { fast_side(dn, sv, zv); });
      na = fa;
      nb = fb;
      if (!more) break;
    }
    t0 += (int64_t)K * kStep;
  } else if (even_rows && t0 + kMTile <= s1) {
    TileDesc dc = describe(t0);
    fast_values(dc, vd);
    fast_keys(dc, kqa, kqb);
    fast_norms(dc, nrm);
    fast_side(dc, sv, zv);
    for (;;) {
      t0 = uniform64(t0);
      const int64_t tn = t0 + kMWaves * kMTile;
      const bool more = __builtin_amdgcn_readfirstlane((int)(tn + kMTile <= s1)) != 0;
      const TileDesc dn = more ? describe(tn) : dc;
      tile(std::false_type{}, 31, kqa, kqb, vd, nrm, sv, zv, [&] { fast_values(dn, vd); },
           [&] { fast_keys(dn, kqa, kqb); }, [&] { fast_norms(dn, nrm); }, [&] { fast_side(dn, sv, zv); });
      t0 = tn;
      dc = dn;
      if (!more) break;
    }
  }
  // Remaining tiles (the tail, or rows of odd parity): loads at the top.
  for (; t0 < s1; t0 += kMWaves * kMTile) {
    t0 = uniform64(t0);
    const TileDesc d = describe(t0);
    slow_loads(d, kqa, kqb, vd, nrm, sv, zv);
    tile(std::true_type{}, d.last, kqa, kqb, vd, nrm, sv, zv, none, none, none, none);
  }

  // ---- per-wave result.  Sum the per-lane shares of query qq (banks, rows).
  l_run += dpp_row_ror<0x124>(l_run);
  l_run += dpp_row_ror<0x128>(l_run);
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  float zq[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float z = zacc[g];
    z += dpp_row_ror<0x124>(z);
    z += dpp_row_ror<0x128>(z);
    z += __shfl_xor(z, 16, 64);
    z += __shfl_xor(z, 32, 64);
    zq[g] = __shfl(z, kg, 64);  // query kg
  }
  __syncthreads();  // red_o overlays the spread tiles of every wave
  if (kg < Q) {
    // C element (row (kg, g), column n) of step tau: dim 4 * (16 * (tau & 1) + n) + (tau >> 1),
    // which lies in group g = 2 * (tau & 1) + (n >> 3)
#pragma unroll
    for (int tau = 0; tau < 8; ++tau) {
      const int hb = tau & 1, f = tau >> 1;
      const bool hi8 = n >= 8;
      const float acc = hi8 ? acc_o[tau][2 * hb + 1] : acc_o[tau][2 * hb];
      const float sg = hi8 ? acc_s[2 * hb + 1] : acc_s[2 * hb];
      const float zg = hi8 ? zq[2 * hb + 1] : zq[2 * hb];
      const float inv = f < 3 ? 1.0f / (float)(1 << (2 * f)) : 1.0f / 32.0f;
      red_o[w][kg][4 * (16 * hb + n) + f] = (acc - 128.0f * sg) * inv + zg;
    }
  }
  if (lane < Q) {
    red_m[w][lane] = m_run;
    red_l[w][lane] = l_run;
  }
  __syncthreads();
  // a (sequence, KV head) of one split and no recent part: the final output
  const bool direct = rule.direct && nsplit == 1;
  // ---- merge the 4 waves into this split's partial (natural-log units).
  // Each thread takes two adjacent dims of one query row and reads all its
  // LDS operands before using any (waves without tokens, l = 0, are skipped).
  for (int i = tid; i < Q * 64; i += 256) {
    const int j = i >> 6, d = 2 * (i & 63);
    float mw[kMWaves], lw[kMWaves];
    f32x2 ow[kMWaves];
#pragma unroll
    for (int ww = 0; ww < kMWaves; ++ww) {
      mw[ww] = red_m[ww][j];
      lw[ww] = red_l[ww][j];
      ow[ww] = *(const f32x2*)&red_o[ww][j][d];
    }
    float M = -__builtin_inff();
#pragma unroll
    for (int ww = 0; ww < kMWaves; ++ww) M = lw[ww] > 0.0f ? fmaxf(M, mw[ww]) : M;
    float L = 0.0f;
    f32x2 O = {0.0f, 0.0f};
    bool poisoned = false;  // a NaN score reached some wave's sum
#pragma unroll
    for (int ww = 0; ww < kMWaves; ++ww) {
      const bool live = lw[ww] > 0.0f;
      poisoned |= is_nan_bits(lw[ww]);
      const float f = live ? exp2f(mw[ww] - M) : 0.0f;
      L = live ? fmaf(lw[ww], f, L) : L;
      O[0] = live ? fmaf(ow[ww][0], f, O[0]) : O[0];
      O[1] = live ? fmaf(ow[ww][1], f, O[1]) : O[1];
    }
    // a NaN score makes the reference's softmax row NaN: the partial's sum
    // carries it to the merge (which would otherwise drop the partial)
    if (poisoned) L = kQuietNaN;
    if (direct) {
      // the output itself: the split combine's arithmetic for one partial
      // (o * (1 / l), zero without tokens), in the output dtype
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      const float r0 = poisoned ? kQuietNaN : O[0] * inv, r1 = poisoned ? kQuietNaN : O[1] * inv;
      store_out2(p, (qrow0 + j) * 128 + d, r0, r1);
    } else {
      const int64_t pi = part.idx(b, h, p.n_kv_heads, Q, j, s);
      const float Mn = M == -__builtin_inff() ? M : M * 0.6931471805599453f;
      if (rule.merge) {
        // agent-coherent stores (written through this XCD's L2), read back by
        // the merging workgroup with agent-coherent loads
        store_agent(&part.o[pi * 128 + d], O);
        if (d == 0) {
          store_agent(&part.m[pi], Mn);
          store_agent(&part.l[pi], L);
        }
      } else {
        *(f32x2*)&part.o[pi * 128 + d] = O;
        if (d == 0) {
          part.m[pi] = Mn;
          part.l[pi] = L;
        }
      }
    }
  }
  if (direct || !rule.merge) return;
  // ---- split merge.  Once every thread has seen its agent-coherent partial
  // stores complete (vmcnt 0), one thread counts the workgroup in with a
  // vector atomic; the workgroup that completes the count is the unit's
  // last, resets the counter for the next call and merges all splits in
  // split order with the combine kernel's arithmetic, so the result does not
  // depend on which workgroup arrives last.  No cache-wide fence: a device-
  // scope release / acquire writes back / invalidates the whole L2 of the
  // XCD in every workgroup (measured: 178 -> 313 us at c3).
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitVmemOnly);
  asm volatile("" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    int* const cnt = p.arrivals + ((int64_t)b * p.n_kv_heads + h);
    const int before = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = before == nsplit - 1 ? 1 : 0;
    if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_split = last;
  }
  __syncthreads();
  if (!last_split) return;
  const int S = part.S;
  for (int i = tid; i < Q * 64; i += 256) {
    const int j = i >> 6, d = 2 * (i & 63);
    const int64_t base = part.idx(b, h, p.n_kv_heads, Q, j, 0);
    // history splits [0, n_splits) sum into o, the recent window's splits
    // (written by the recent launch before this kernel) into r
    float M = -__builtin_inff(), L = 0.0f, o0 = 0.0f, o1 = 0.0f, r0 = 0.0f, r1 = 0.0f;
    bool poisoned = false;  // a partial whose sum is NaN (a NaN score)
    for (int c0 = 0; c0 < S; c0 += 8) {
      // a chunk's loads are all issued before any is used
      float mv[8], lv[8];
      f32x2 ov[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        lv[k] = 0.0f;
        mv[k] = -__builtin_inff();
        ov[k] = f32x2{0.0f, 0.0f};
        // history partials [0, nsplit) (an item's sequence may fill fewer
        // than the n_splits slots), recent ones [n_splits, S)
        if (c0 + k < S && (c0 + k < nsplit || c0 + k >= rule.n_splits)) {
          lv[k] = load_agent(&part.l[base + c0 + k]);
          mv[k] = load_agent(&part.m[base + c0 + k]);
          ov[k] = load_agent2(&part.o[(base + c0 + k) * 128 + d]);
        }
      }
      float Mc = M;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (lv[k] > 0.0f) Mc = fmaxf(Mc, mv[k]);
        poisoned |= is_nan_bits(lv[k]);
      }
      if (Mc > M) {
        const float c = __expf(M - Mc);
        L *= c;
        o0 *= c;
        o1 *= c;
        r0 *= c;
        r1 *= c;
        M = Mc;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (!(lv[k] > 0.0f)) continue;
        const float wk = __expf(mv[k] - M);
        L = fmaf(lv[k], wk, L);
        const float v0 = ov[k][0] * wk, v1 = ov[k][1] * wk;
        if (c0 + k < rule.n_splits) {
          o0 += v0;
          o1 += v1;
        } else {
          r0 += v0;
          r1 += v1;
        }
      }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    o0 *= inv;
    o1 *= inv;
    if (S > rule.n_splits) {
      // history and recent outputs each in the output dtype, then added (the
      // combine kernel's order, as compute_hybrid_attention adds them)
      o0 = round_out(p, round_out(p, o0) + round_out(p, r0 * inv));
      o1 = round_out(p, round_out(p, o1) + round_out(p, r1 * inv));
    }
    if (poisoned) o0 = o1 = kQuietNaN;
    store_out2(p, (qrow0 + j) * 128 + d, o0, o1);
  }
}

bool mfma_decode_supported(const smaq_attn_params& p) {
  const int g = p.n_q_heads / p.n_kv_heads;
  return p.has_history && p.q_len == 1 && !p.q_positions && p.head_dim == 128 &&
         p.key_format == SMAQ_KEY_SCALAR && (p.key_bits == 3 || p.key_bits == 4) &&
         p.key_row_bytes == 64 && p.val_bits == 2 && p.val_group == 32 && p.val_row_bytes == 32 &&
         g >= 1 && g <= 4 &&
         (!p.block_table || (p.block_size >= 16 && (p.block_size & (p.block_size - 1)) == 0)) &&
         // vector loads of rows, row pairs and query rows assume 16-byte
         // aligned arrays
         (((uintptr_t)p.key_bytes | (uintptr_t)p.val_bytes | (uintptr_t)p.key_norms |
           (uintptr_t)p.val_scales | (uintptr_t)p.val_zeros | (uintptr_t)p.q_hist) & 15) == 0;
}

// Contexts are split so that the grid fills one round of the device's
// workgroup slots (kDecodeWaves workgroups of 4 waves per CU): a workgroup's
// fixed costs (its prologue and first tile's latency, the 4-wave merge) are
// then paid once per slot (c3: 4 splits, 1024 workgroups, 0.177 ms against
// 0.183 ms for two rounds of half the length).  The length returned sets the
// number of splits; the kernel places the boundaries (SplitRule).
int64_t mfma_decode_split_len(const smaq_attn_params& p) {
  const int64_t units = (int64_t)p.batch * p.n_kv_heads;
  const bool wide = p.norm_dtype == SMAQ_F32 || p.val_dtype == SMAQ_F32;
  const int64_t slots = (int64_t)device_cu_count() * (wide ? 3 : 4);
  const int64_t want = units >= slots ? 1 : (slots + units - 1) / units;
  int64_t split = (p.max_hist_len + want - 1) / want;
  const int64_t q = kMWaves * kMTile;
  split = ((split + q - 1) / q) * q;
  return split < 4 * q ? 4 * q : split;
}

// Weight step per round-slot with 4 slots per CU: splits weigh 64, 54, 44, 34
// (c3 on MI355X, kernel alone, three alternating rounds on one box: steps
// of 6 / 8 / 10 / 12 took 173.9 / 172.3 / 171.1 / 173.0 us; equal splits
// were 2-3% slower than a step of 10 on other boxes, 14 and above slower
// still).  With 3 slots (fp32 metadata) the splits stay equal (not measured).
constexpr int kSplitTilt4 = 10;
static_assert(kSplitTilt4 * 3 < kSplitWeight, "split weights must stay positive");

template <int KB, typename TN, bool SPLIT, bool VBUF>
static void launch_v(const smaq_attn_params& p, const HistAddr& a, const Partials& part, const SplitRule& rule,
                     int n_splits, const int* order, hipStream_t st) {
  // heads fastest, then sequences (the longest-first order when given), then
  // splits: split-major, so that a one-round grid runs split s in round-slot s;
  // in item mode, heads fastest, then items
  const dim3 grid(p.n_kv_heads, rule.pieces ? rule.items : p.batch, rule.pieces ? 1 : n_splits);
  switch (p.val_dtype) {
    case SMAQ_F32: hipLaunchKernelGGL((decode_mfma_kernel<KB, TN, float, SPLIT, VBUF>), grid, dim3(256), 0, st, p, a, part, rule, order); break;
    case SMAQ_F16: hipLaunchKernelGGL((decode_mfma_kernel<KB, TN, _Float16, SPLIT, VBUF>), grid, dim3(256), 0, st, p, a, part, rule, order); break;
    default: hipLaunchKernelGGL((decode_mfma_kernel<KB, TN, bf16, SPLIT, VBUF>), grid, dim3(256), 0, st, p, a, part, rule, order); break;
  }
}

template <int KB, typename TN>
static void launch_s(const smaq_attn_params& p, const HistAddr& a, const Partials& part, const SplitRule& rule,
                     int n_splits, const int* order, hipStream_t st) {
  // 16-token pages put a tile's two 16-token groups in different blocks
  // (value rows of 32 bytes: the pool's bytes as a 32-bit descriptor range)
  const bool vbuf = a.rows > 0 && a.rows <= (int64_t)(0xFFFFFFFFu / 32u);
  if (p.block_table && p.block_size == 16) {
    if (vbuf) launch_v<KB, TN, true, true>(p, a, part, rule, n_splits, order, st);
    else launch_v<KB, TN, true, false>(p, a, part, rule, n_splits, order, st);
  } else {
    launch_v<KB, TN, false, false>(p, a, part, rule, n_splits, order, st);
  }
}

template <int KB>
static void launch_n(const smaq_attn_params& p, const HistAddr& a, const Partials& part, const SplitRule& rule,
                     int n_splits, const int* order, hipStream_t st) {
  switch (p.norm_dtype) {
    case SMAQ_F32: launch_s<KB, float>(p, a, part, rule, n_splits, order, st); break;
    case SMAQ_F16: launch_s<KB, _Float16>(p, a, part, rule, n_splits, order, st); break;
    default: launch_s<KB, bf16>(p, a, part, rule, n_splits, order, st); break;
  }
}

int launch_mfma_decode(const smaq_attn_params& p, const HistAddr& a, const Partials& part,
                       int n_splits, bool direct, bool merge, const int* order, int items, hipStream_t st) {
  const bool wide = p.norm_dtype == SMAQ_F32 || p.val_dtype == SMAQ_F32;
  SplitRule rule;
  rule.n_splits = n_splits;
  rule.n_cu = device_cu_count();
  rule.slots = wide ? 3 : 4;
  rule.tilt = wide ? 0 : kSplitTilt4;
  rule.pieces = items > 0 ? 1 : 0;
  rule.items = items;
  // item mode: the sequences of one piece write the output when there is no
  // recent part; the others merge their pieces (arrival counters required)
  rule.direct = direct && (rule.pieces || n_splits == 1) ? 1 : 0;
  rule.merge = merge && p.arrivals && (rule.pieces || !rule.direct) ? 1 : 0;
  SMAQ_REQUIRE(!rule.merge || part.S >= n_splits, "smaq_attn_hybrid: merge partials missing");
  SMAQ_REQUIRE(!rule.pieces || (order && rule.merge && n_splits <= 0xffff),
               "smaq_attn_hybrid: decode pieces need items and arrival counters");
  if (p.key_bits == 3) launch_n<3>(p, a, part, rule, n_splits, order, st);
  else launch_n<4>(p, a, part, rule, n_splits, order, st);
  return launch_status("smaq_attn_hybrid(mfma decode)");
}

}  // namespace smaq
