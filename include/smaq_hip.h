/*
 * smaq_hip.h -- C ABI of libsmaq_hip.so, the MI355X (gfx950) kernels behind the
 * SMAQ quantized-KV hot path.
 *
 * Conventions
 *  - Every entry point is extern "C", takes plain device pointers, element
 *    counts and strides, and an opaque hipStream_t (void*), and returns an int
 *    status: SMAQ_OK (0) or a negative code.  smaq_last_error() returns a
 *    thread-local message for the last failure on the calling thread.
 *  - The caller allocates every output and workspace (torch does, on the
 *    Python side).  Entry points never allocate, never synchronise the stream,
 *    and keep no mutable global state (re-entrant), except
 *    smaq_attn_hybrid_noalloc, whose workspace is one built-in array per GPU.
 *  - dtype codes: SMAQ_F32 = 0, SMAQ_F16 = 1, SMAQ_BF16 = 2.
 *  - "rows" inputs are addressed as row r = o * n_inner + i at element offset
 *    o * s_outer + i * s_inner with a contiguous last dim.  This covers the
 *    [1, Hkv, T, D] transpose views the reference's store passes to its codecs
 *    (smaq/store.py:86-87).  The encoders write row r to output row
 *    o * out_outer + i: out_outer = 0 means n_inner (dense, row-major in r
 *    order); a larger out_outer writes into the tail rows of per-head columns
 *    [Hkv][capacity][...] (pass the column base offset by the first new row
 *    and out_outer = capacity), so an appended chunk is encoded in place.
 *
 * Each declaration names the reference interface (file:line under
 * gauravsaini/smaq) whose arithmetic it replaces.
 */
#ifndef SMAQ_HIP_H_
#define SMAQ_HIP_H_

#ifdef __cplusplus
extern "C" {
#endif

enum { SMAQ_F32 = 0, SMAQ_F16 = 1, SMAQ_BF16 = 2 };
enum { SMAQ_OK = 0, SMAQ_EINVAL = -1, SMAQ_EUNSUPPORTED = -2, SMAQ_ELAUNCH = -3 };

/* Library version (major * 10000 + minor * 100 + patch). */
int smaq_version(void);
/* Message for the last non-zero status returned on this thread. */
const char* smaq_last_error(void);

/*
 * Value bit-packer.  Replaces quantize_values (smaq/kv_cache.py:50-91):
 * per group of `group` elements, scale = max((max-min)/(2^bits-1), 1e-10),
 * zero = min, code = clamp(round_half_even((v-zero)/scale), 0, 2^bits-1),
 * every op rounded to the value dtype.  2-bit codes pack 4 per byte, 4-bit 2
 * per byte (low bits first), other widths 1 per byte.
 *   data_out   [rows, D/vpb] uint8     scales_out, zeros_out [rows, D/group] vdtype
 */
int smaq_pack_values(const void* v, int vdtype, long long n_outer, long long n_inner,
                     long long s_outer, long long s_inner, long long out_outer, int D, int bits,
                     int group, void* data_out, void* scales_out, void* zeros_out, void* stream);

/*
 * Value dequantiser.  Replaces unpack_values + dequantize_values
 * (smaq/kv_cache.py:29-47,94-103): out = float(code) * scale + zero (fp32).
 */
int smaq_dequant_values(const void* data, const void* scales, const void* zeros, int sdtype,
                        long long rows, int D, int bits, int group, float* out, void* stream);

/*
 * Weighted sum over packed values.  Replaces the compressed term of
 * SMAQKVCache.attend (smaq/kv_cache.py:247-252), torch.matmul(w,
 * dequantize_values(vq)): out[b][q][d] = sum_n w[b][q][n] * v[b][n][d] with
 * v = float(code) * scale + zero (smaq/kv_cache.py:94-103), summed in fp32
 * without writing v out.  Deterministic: fixed token splits summed in order.
 *   w fp32, element (b, q, n) at w[b * w_bstride + q * w_qstride + n];
 *   data: row n of batch b at data + b * d_bstride + n * (D / vpb) bytes
 *   (vpb = 4, 2, 1 codes per byte for 2-, 4-, other-bit codes);
 *   scales, zeros: row n of batch b at b * s_bstride + n * (D / group)
 *   elements, in sdtype; out [batch][nq][D] fp32, overwritten.
 *   workspace: smaq_apply_values_workspace_bytes(batch, nq, N, D) bytes
 *   (0: none needed).
 * Layouts: a value row must be a power-of-two number (<= 64) of 4-byte words,
 * each inside one group (D = 128: 2-bit with group % 16 == 0, 4-bit with
 * group % 8 == 0, 8-bit with group % 4 == 0); others return
 * SMAQ_EUNSUPPORTED.
 */
long long smaq_apply_values_workspace_bytes(long long batch, long long nq, long long N, int D);
int smaq_apply_values(const float* w, long long w_bstride, long long w_qstride, long long batch, long long nq,
                      long long N, int D, const void* data, long long d_bstride, int bits, int group,
                      const void* scales, const void* zeros, long long s_bstride, int sdtype, float* out,
                      void* workspace, long long workspace_bytes, void* stream);

/*
 * Scalar key encoder.  Replaces SMAQQuantizer.quantize (smaq/quantizer.py:138-145)
 * and RotationAdapter.quantize (smaq/weighted_scalar.py:347-355):
 * n = ||k|| (key dtype), u = k / (n + 1e-10) (key dtype), y = u @ M^T (fp32),
 * optionally y *= coord_scales, code = #{bounds[i] < y}, packed
 * max(1, 8/bits) codes per byte.  Mt is M transposed, [D][D] fp32 row-major.
 *   codes_out [rows, ceil(D/vpb)] uint8    norms_out [rows] kdtype
 *   tie_count (nullable): += number of y within 1e-6 (relative) of a bound.
 */
int smaq_encode_scalar(const void* k, int kdtype, long long n_outer, long long n_inner,
                       long long s_outer, long long s_inner, long long out_outer, int D, const float* Mt,
                       const float* coord_scales, const float* bounds, int n_bounds, int bits,
                       void* codes_out, void* norms_out, unsigned long long* tie_count,
                       void* stream);

/*
 * Row transform y = (x @ M^T) [* coord_scales] in fp32 with a sequential FMA
 * chain over D.  Replaces SMAQQuantizer.rotate_query (smaq/quantizer.py:131-136)
 * and RotationAdapter.rotate_query (smaq/weighted_scalar.py:342-345).
 */
int smaq_rotate_rows(const void* x, int xdtype, long long rows, int D, const float* Mt,
                     const float* coord_scales, float* out, void* stream);

/*
 * Scalar key dequantiser.  Replaces SMAQQuantizer.dequantize
 * (smaq/quantizer.py:147-152; inv_scales = NULL, Mt = E_inv^T) and
 * RotationAdapter.dequantize (smaq/weighted_scalar.py:357-363; Mt = R):
 * k_hat = ((c[code] [* inv_scales]) @ Mt) * norm, written as odtype.
 */
int smaq_dequant_scalar(const void* codes, const void* norms, int ndtype, long long rows, int D,
                        int bits, const float* centroids, const float* inv_scales, const float* Mt,
                        void* out, int odtype, void* stream);

/*
 * Scores against scalar-coded keys.  Replaces the score path of
 * SMAQQuantizer.attention_score / smaq_attention_scores
 * (smaq/quantizer.py:154-184, smaq/triton_kernels.py:102-114,190-208):
 * out[b, r, t] = ((qrot[b, r] . c[code[b, t]]) * norm[b, t]) [* scale].
 *   qrot [batch, nq, D] fp32; codes [batch, N, P] uint8; norms [batch, N];
 *   out [batch, nq, N] in odtype.  has_scale = 0 skips the scale multiply.
 */
int smaq_scores_scalar(const float* qrot, long long batch, long long nq, long long N, int D,
                       const void* codes, int bits, const void* norms, int ndtype,
                       const float* centroids, int has_scale, float scale, void* out, int odtype,
                       void* stream);

/*
 * Block-VQ key encoder.  Replaces SMAQBlockVQ.quantize (smaq/block_vq.py:216-244):
 * per block b, x = k_b @ E_b^T, d = sqrt(clamp_min(-2 x.c + |x|^2 + |c|^2, 0))
 * (torch.cdist's matmul form), index = first argmin.
 *   E_blocks [nb][bd][bd]; centroids [nb][nc][bd] fp32; idx_out [rows, nb] uint8.
 *   tie_count (nullable): += number of (row, block) whose two best distances
 *   are within 1e-6 (relative).
 */
int smaq_encode_blockvq(const void* k, int kdtype, long long n_outer, long long n_inner,
                        long long s_outer, long long s_inner, long long out_outer, int n_blocks, int block_dim,
                        int n_centroids, const float* E_blocks, const float* centroids,
                        void* idx_out, unsigned long long* tie_count, void* stream);

/*
 * Block-VQ dequantiser.  Replaces SMAQBlockVQ.dequantize (smaq/block_vq.py:246-267):
 * k_hat[r, b*bd + i] = decoded[b][idx[r, b]][i] (fp32).
 */
int smaq_dequant_blockvq(const void* idx, long long rows, int n_blocks, int block_dim,
                         int n_centroids, const float* decoded, float* out, void* stream);

/*
 * Block-VQ calibration on the device.  The reference fits its codebook with
 * torch ops on the calibration data's device (smaq/block_vq.py:37-79 _kmeans,
 * :190-203 fit); these three steps are that fit's arithmetic, with the
 * assignment step done by smaq_encode_blockvq:
 *
 * smaq_blockvq_shape replaces `calibration_keys[:, bj].float() @ E.T`
 * (smaq/block_vq.py:196) for every block: x[b][r][i] = sum_d k[r][b*bd+d] *
 * E_b[i][d] (sequential FMA over d, the encoder's own shaped keys).
 *   k [rows][n_blocks*block_dim] contiguous; x_out [n_blocks][rows][block_dim] fp32.
 */
int smaq_blockvq_shape(const void* k, int kdtype, long long rows, int n_blocks, int block_dim,
                       const float* E_blocks, float* x_out, void* stream);

/*
 * k-means++ seeding distances (smaq/block_vq.py:54-61, the squared distance
 * of every point to its nearest chosen centroid): dmin[b][r] =
 * |x[b][r] - x[b][pick[b]]|^2 when `first`, else the minimum of that and
 * dmin[b][r].  pick: [n_blocks] row indices (device int64).
 */
int smaq_kmeanspp_update(const float* x, int n_blocks, long long rows, int block_dim,
                         const long long* pick, int first, float* dmin, void* stream);

/*
 * Lloyd centroid update (smaq/block_vq.py:70-77): centroid (b, j) = mean of
 * the x[b][r] with idx[r][b] == j; centroids with no rows keep their value.
 * idx [rows][n_blocks] uint8 (smaq_encode_blockvq's output); centroids
 * [n_blocks][n_centroids][block_dim] fp32, updated in place.  Deterministic.
 */
int smaq_kmeans_update(const float* x, const unsigned char* idx, int n_blocks, long long rows,
                       int block_dim, int n_centroids, float* centroids, void* stream);

/*
 * Fused quantized-KV attention (decode and prefill).  Replaces
 * compute_hybrid_attention (smaq/score.py:23-72) with its per-head score loop
 * (smaq/score.py:75-96), value dequantisation (smaq/kv_cache.py:94-103) and
 * weighted sums (smaq/score.py:113-124): one softmax over [history; recent]
 * logits, each part cast to the output dtype before the sum.
 *
 * History token t of sequence b, KV head h, lives at row
 *   contiguous: h * hist_head_stride + hist_seq_start[b] + t
 *   paged:      (block_table[b * max_blocks + t / block_size] * Hkv + h) * block_size
 *               + t % block_size
 * and every per-token array (key bytes, norms, value bytes, scales, zeros) is
 * indexed by that row.  Rows of queries: (b, t, hq) with hq -> KV head hq / g.
 */
enum { SMAQ_KEY_SCALAR = 0, SMAQ_KEY_BLOCKVQ = 1 };

typedef struct smaq_attn_params {
  /* shapes */
  int batch;        /* sequences */
  int q_len;        /* query tokens per sequence (T) */
  int n_q_heads;    /* Hq */
  int n_kv_heads;   /* Hkv */
  int head_dim;     /* D */
  float scale;      /* softmax scale (1/sqrt(D) when the caller passes None) */
  /* queries, fp32 [batch][q_len][Hq][D]: q_hist is the query as the history
     codec scores it (rotated for scalar codes), q_exact the plain query.
     With q_raw set (below) the recent window reads q_raw instead, and
     q_exact is a scratch row buffer the library fills from q_raw when a
     multi-token query takes the recent prefill path. */
  const float* q_hist;
  const float* q_exact;
  /* causal extension: NULL = no mask (reference semantics); else int64
     [batch][q_len] absolute positions; key j is visible iff pos_j <= q_pos. */
  const long long* q_positions;
  /* history (compressed) segment */
  int has_history;
  int key_format;          /* SMAQ_KEY_SCALAR or SMAQ_KEY_BLOCKVQ */
  const void* key_bytes;   /* [rows][key_row_bytes] uint8 */
  int key_row_bytes;
  int key_bits;            /* scalar: bits per code */
  const void* key_norms;   /* scalar: [rows], norm_dtype */
  int norm_dtype;
  const float* key_lut;    /* scalar: centroids [2^bits]; block-VQ: decoded [nb][nc][bd] */
  int vq_blocks, vq_block_dim, vq_centroids;
  const void* val_bytes;   /* [rows][val_row_bytes] uint8 */
  int val_row_bytes;
  int val_bits, val_group;
  const void* val_scales;  /* [rows][D/group], val_dtype */
  const void* val_zeros;
  int val_dtype;
  const long long* hist_len;        /* [batch] history tokens per sequence; NULL: all
                                       sequences hold max_hist_len tokens */
  const long long* hist_seq_start;  /* contiguous layout: [batch] start row; NULL:
                                       sequence b starts at row b * max_hist_len */
  long long hist_head_stride;       /* contiguous layout: rows between heads */
  const int* block_table;           /* paged layout, NULL for contiguous */
  int max_blocks;
  int block_size;
  long long hist_pos_offset;        /* absolute position of history token 0 */
  /* recent (exact) segment: [batch][recent_stride_t][Hkv][D] in recent_dtype */
  int has_recent;
  const void* recent_k;
  const void* recent_v;
  int recent_dtype;
  const long long* recent_len;      /* [batch]; NULL: all hold max_recent_len */
  long long recent_batch_stride;    /* elements between sequences */
  long long recent_pos_offset;      /* absolute position of recent token 0 */
  /* output [batch][q_len][Hq][D] in out_dtype */
  void* out;
  int out_dtype;
  /* workspace from smaq_attn_workspace_bytes */
  void* workspace;
  long long workspace_bytes;
  /* max history length over the batch (sizes the split grid) */
  long long max_hist_len;
  long long max_recent_len;
  /* 0 = run everything; else a bit mask of phases to launch, so a caller can
     time them apart: 8 = query rotation (with rot_mt), 1 = history
     partials, 2 = recent partials, 4 = combine.
     Phases communicate through the workspace, launched in order on one
     stream.  When the matrix-core decode kernel serves the history as one
     split per (sequence, KV head) and there is no recent part, phase 1
     writes the output itself and phase 4 launches nothing; with arrival
     counters (below) it merges several splits itself, and, when one call
     launches phases 1 and 2, the recent partials too (the recent phase then
     runs first).  For ragged batches that kernel runs in a longest-first
     schedule which phase 1 builds first (inside the rotation's launch when
     phases 8 and 1 run in one call); with 16 added,
     phase 1 reuses the schedule an earlier call on this workspace built for
     the same lengths, so the decode kernel can be timed alone (with any
     other workspace contents the output is undefined). */
  int phases;
  /* kernel choice: 0 = automatic (matrix-core decode kernel when the shape
     allows, generic kernels otherwise), 1 = generic kernels only, 2 = the
     matrix-core decode kernel, 3 = the matrix-core prefill kernel
     (SMAQ_EUNSUPPORTED if the shape does not fit).  Automatic choice: the
     decode kernel for single-token queries, the prefill kernel for
     q_len >= 16 at head_dim 128, the generic kernels otherwise. */
  int impl;
  /* Optional split merge inside the matrix-core decode kernel (NULL: a
     combine launch merges the splits).  int32 [batch * Hkv] arrival
     counters, zero before the first call; every call leaves them zero.
     When the decode kernel serves the history in several splits, or with a
     recent part whose partials the same call's recent phase wrote first,
     each workgroup counts itself in once its partial is written and the
     last one of its (sequence, KV head) merges the partials in split order
     (the combine launch's arithmetic) and writes the output: phase 1 then
     writes the output and phase 4 launches nothing.  Calls sharing the
     counters must not overlap. */
  int* arrivals;
  /* Optional query rotation (rot_mt NULL: q_hist is read as given).  With
     rot_mt set, phase 8 writes q_hist = (q_raw @ M^T) [* rot_scale]
     (smaq_rotate_rows, one launch), the codec-space query that
     SMAQQuantizer.rotate_query (smaq/quantizer.py:131-136) and
     RotationAdapter.rotate_query (smaq/weighted_scalar.py:342-345) form
     before scoring; q_hist must then be a writable fp32 buffer.
       q_raw [batch][q_len][Hq][D] in q_raw_dtype; rot_mt = M^T [D][D] fp32;
       rot_scale [D] fp32 or NULL. */
  const void* q_raw;
  int q_raw_dtype;
  const float* rot_mt;
  const float* rot_scale;
  /* Rows in each history pool array (key codes, norms, values, scales,
     zeros share the row index; paged layout: blocks * n_kv_heads *
     block_size), or 0 if unknown.  Lets the decode kernel address a paged
     value pool below 4 GB through one buffer descriptor; it must cover
     every row the block table reaches (the descriptor is range-checked:
     value rows past it read as zero).  0 keeps 64-bit per-lane addresses.
     Added last, so a zero-initialised struct keeps its earlier meaning. */
  long long hist_rows;
} smaq_attn_params;

/* Bytes of workspace smaq_attn_hybrid needs for these parameters. */
long long smaq_attn_workspace_bytes(const smaq_attn_params* p);
int smaq_attn_hybrid(const smaq_attn_params* p, void* stream);

/*
 * Allocation-free smaq_attn_hybrid.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid hipMalloc).  Same kernels and results as
 * smaq_attn_hybrid; p->workspace and p->workspace_bytes are ignored and the
 * workspace is a built-in device array of SMAQ_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends.  Parameters whose smaq_attn_workspace_bytes
 * exceeds that size are rejected with SMAQ_EINVAL (decode batches fit; the
 * matrix-core prefill's tile images generally do not).  Nothing in the array
 * needs clearing between calls (every partial a call reads it writes first),
 * but calls that overlap on one GPU -- on two streams, or two threads --
 * share the array and race.  The first call on a device looks up the array's
 * address there (hipGetSymbolAddress); no call allocates or frees memory.
 */
#define SMAQ_NOALLOC_SCRATCH_BYTES (32ll << 20)
int smaq_attn_hybrid_noalloc(const smaq_attn_params* p, void* stream);

/*
 * Streaming-read probe.  No counterpart in the reference: a measurement
 * utility that reads `bytes` (a multiple of 16) from `src` once in 16-byte
 * loads over the whole device and writes nothing unless the XOR of
 * everything read equals a fixed sentinel (then one word of `sink`); its
 * duration gives the HBM read rate a plain stream reaches on this GPU, the
 * practical ceiling next to the published peak.
 */
int smaq_probe_read(const void* src, long long bytes, unsigned int* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SMAQ_HIP_H_ */
