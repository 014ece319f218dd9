/* insitu.h -- C ABI of the MI355X compressed-KV decode-attention block.
 *
 * The boundary is the reference's seam (kernel.py:253-258 in, :348-353 out):
 * post-RoPE q/k/v arrive as Q8.16 integers, the block rotates them, appends
 * the compressed k/v row to an HBM-resident cache, scores the query heads on
 * the codes, runs the fixed-point softmax and returns Q16 in the rotated
 * basis, head-major (merge_heads order, ops/project.py:67-74).
 *
 * Conventions
 *   - Every call returns an int status; 0 is OK. The status set follows
 *     host/attn_proto.py:41 (OK, EBADLEN, ERANGE, EDMA -> EHIP) plus the
 *     reference's raise sites (capacity, bad format).
 *   - Pointers named *_dev are device pointers (hipMalloc / torch cuda
 *     tensors); *_host are host pointers. Device work is ordered on the
 *     context's stream; a call does not synchronise unless it says so.
 *   - A handle is not thread-safe. append must precede attend on the same
 *     stream: the current token attends to itself (hw/vectors.py:22-30).
 *   - Lengths and the plane layout are owned by the cache handle, as the host
 *     owns cache_base/head_stride/plane_span in host/attn_proto.h:16-24.
 */
#ifndef INSITU_H
#define INSITU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    INSITU_OK = 0,
    INSITU_EBADLEN = 1,    /* shape/length mismatch (attn_proto.py:41 EBADLEN)         */
    INSITU_ERANGE = 2,     /* value outside the format (attn_proto.py:41 ERANGE)       */
    INSITU_EHIP = 3,       /* HIP runtime failure (stands where EDMA stood)            */
    INSITU_EINVAL = 4,     /* unsupported format / bad argument (config.py:45-61,178-207) */
    INSITU_ECAPACITY = 5,  /* append past capacity (cache/base.py:67-73)               */
    INSITU_ENOMEM = 6,
    INSITU_EFAULT = 7      /* a kernel reported an internal error flag                 */
};

enum {
    INSITU_SEQUENTIAL = 0, /* CompressedAttention.attend_online, bit-exact (attention.py:451-513) */
    INSITU_TWO_PASS = 1,   /* CompressedAttention.attend_two_pass, bit-exact (attention.py:429-449) */
    INSITU_SPLIT = 2,      /* context-split flash-decoding; <= 2 Q16 LSB of SEQUENTIAL */
    INSITU_SERIAL = 3      /* SEQUENTIAL computed one token at a time per head (slow; reference path) */
};

typedef struct insitu_ctx insitu_ctx;
typedef struct insitu_cache insitu_cache;

/* The fixed-point contract (config.py:132-254 QuantConfig + FixedFormat). */
typedef struct {
    int32_t head_dim;       /* 64 or 128                                   */
    int32_t key_bits;       /* 1..8 (config.py:179-181)                    */
    int32_t value_bits;     /* 1..8                                        */
    int32_t norm_bits;      /* 16                                          */
    int32_t norm_frac;      /* 9                                           */
    int32_t qk_frac;        /* 16                                          */
    int32_t qk_width;       /* 24                                          */
    int32_t centroid_frac;  /* 15                                          */
    int32_t acc_frac;       /* 16                                          */
    int32_t acc_width;      /* 32                                          */
    int32_t score_width;    /* 48                                          */
    int32_t prob_frac;      /* 15                                          */
    int32_t exp_lut_bits;   /* 8                                           */
    int32_t rot_rounds;     /* 1 (config.py:169); 0 is the identity         */
    uint64_t rot_signs[8][2]; /* per round, bit i set = negate channel i (tb/vectors/rot_signs.hex) */
} insitu_format;

/* cache/compressed.py:42-66 + hw/ddr_layout.py:110-124. Codebooks are the
 * integers Codebook.build produced (ops/codebook.py:67-120), as the RTL
 * receives them: centroids 2^bits, boundaries 2^bits - 1, Q(centroid_frac). */
typedef struct {
    int64_t capacity;       /* tokens per sequence                         */
    int32_t batch;          /* sequences                                   */
    int32_t n_kv_heads;
    int32_t n_q_heads;      /* multiple of n_kv_heads (config.py:49-53)     */
    int32_t chunk_tokens;   /* tokens per chunk of the chunked attend: 0 or 1024, or 512; no
                               counterpart in the reference (an MI355X tuning of this build) */
    insitu_format fmt;
    const int64_t *key_centroids_host;
    const int64_t *key_bounds_host;
    const int64_t *value_centroids_host;
    const int64_t *value_bounds_host;
} insitu_cache_desc;

/* hw/ddr_layout.py:261-274 describe(), per sequence region. */
typedef struct {
    int32_t row_bytes, n_planes;
    int32_t plane_lo[16], plane_width[16];
    int64_t plane_span, head_stride, seq_stride, total_bytes;
    uint64_t device_base;   /* device address of sequence 0, head 0, plane 0 */
} insitu_layout;

/* AttentionStats (attention.py:257-274), merged over heads and sequences as
 * AttentionStats.merge does, plus device flags. */
typedef struct {
    int64_t n_tokens, rescale_events, score_overflows, acc_overflows;
    int64_t max_abs_score, max_abs_acc;
    int64_t range_errors;      /* q_rot outside the supported +-2^27 range */
    int64_t serial_fallbacks;  /* heads recomputed on the exact serial path */
} insitu_stats;

/* --- context ------------------------------------------------------------- */
/* Binds a device and a stream (NULL = the default stream); holds the exp LUT constants. */
int insitu_ctx_create(int32_t device, void *hip_stream, insitu_ctx **out);
int insitu_ctx_destroy(insitu_ctx *ctx);
int insitu_ctx_sync(insitu_ctx *ctx);
void *insitu_ctx_stream(insitu_ctx *ctx);

/* Attend kernel timing: the measurement hook of the benchmark (no counterpart
 * in the reference, whose attend is a Python loop). While enabled, every attend
 * on the context's caches attaches a pair of HIP events to its kernel dispatches
 * (start of the first, end of the last; hipExtLaunchKernelGGL), which adds no
 * packets to the stream. _read
 * waits for the last pair and returns the summed kernel time in milliseconds
 * and the number of attends since the previous read. Disabling drops what has
 * not been read. */
int insitu_ctx_timing(insitu_ctx *ctx, int32_t enable);
int insitu_ctx_timing_read(insitu_ctx *ctx, double *total_ms, int64_t *n_attends);
/* The same, one time per attend in launch order: ms_each (cap) receives n_attends values
 * (EBADLEN when more than cap were timed). */
int insitu_ctx_timing_read_each(insitu_ctx *ctx, double *ms_each, int64_t cap, int64_t *n_attends);

/* --- rotation: Rotation.apply (ops/rotate.py:170-197) -------------------- */
/* x_dev, y_dev: int32 (n_vec, d). y may alias x. */
int insitu_rotate(insitu_ctx *ctx, const int32_t *x_dev, int32_t *y_dev, int64_t n_vec,
                  const insitu_format *fmt);

/* --- encoder: KVQuantizer._norm_wire/_encode_plane (ops/quantize.py:164-196) */
/* x_dev int32 (n_vec, d) rotated; norm_dev int32 (n_vec); codes_dev uint8 (n_vec, d). */
int insitu_encode(insitu_ctx *ctx, const int32_t *x_dev, int64_t n_vec, const insitu_format *fmt,
                  const int64_t *bounds_host, int32_t bits, int32_t *norm_dev, uint8_t *codes_dev);

/* --- qtab: T[h][ch][i] = q_rot[h][ch] * c[i] (hw/vectors.py:485-509) ---------- */
int insitu_qtab(insitu_ctx *ctx, const int32_t *q_rot_dev, int32_t n_heads, int32_t d,
                const int64_t *centroids_host, int32_t n_centroids, int64_t *table_dev);

/* --- exp LUT: ExpLut.__call__ (attention.py:153-159) ----------------------- */
int insitu_exp_lut(insitu_ctx *ctx, const int64_t *delta_dev, int64_t n, int32_t *p_dev);

/* --- finalize: reciprocal + _finalize (attention.py:197-250, 873-880) ----- */
int insitu_finalize(insitu_ctx *ctx, const int64_t *acc_dev, const int64_t *l_dev, int32_t rows,
                    int32_t d, int64_t *out_dev, int64_t *recip_dev, int32_t *shift_dev);

/* --- the cache: CompressedCache (cache/compressed.py:42-132) -------------- */
int insitu_cache_create(insitu_ctx *ctx, const insitu_cache_desc *desc, insitu_cache **out);
int insitu_cache_destroy(insitu_cache *cache);
int insitu_cache_reset(insitu_cache *cache);                       /* base.py:64 */
int insitu_cache_length(const insitu_cache *cache, int32_t seq, int64_t *len);
int insitu_cache_set_length(insitu_cache *cache, int32_t seq, int64_t len);
int insitu_cache_layout(const insitu_cache *cache, insitu_layout *out);

/* append_rotated (compressed.py:64-86): encode, pack and write n_tok rows at
 * each sequence's length. k/v_rot_dev int32 (batch, n_tok, n_kv_heads, d). */
int insitu_append(insitu_cache *cache, const int32_t *k_rot_dev, const int32_t *v_rot_dev,
                  int32_t n_tok);
/* The same for one sequence: k/v_rot_dev int32 (n_tok, n_kv_heads, d). */
int insitu_append_seq(insitu_cache *cache, int32_t seq, const int32_t *k_rot_dev,
                      const int32_t *v_rot_dev, int32_t n_tok);
/* kernel.py:271-272 + :283-284 in one pass: rotate wire k/v rows (Rotation.apply,
 * rotate.py:170-197, with the cache format's rotation) and append them as insitu_append
 * does, without the rotated copies. seq = -1: every sequence, k/v_wire_dev int32 (batch,
 * n_tok, n_kv_heads, d); else that sequence, (n_tok, n_kv_heads, d). Rotated values beyond
 * int32 count as range errors. */
int insitu_append_wire(insitu_cache *cache, int32_t seq, const int32_t *k_wire_dev,
                       const int32_t *v_wire_dev, int32_t n_tok);

/* attend_online / attend_two_pass over every sequence's cache (kernel.py:337-345,
 * attention.py:429-513). q_rot_dev int32 (batch, n_q_heads, d) rotated;
 * out_dev int32 (batch, n_q_heads, d) Q16. stats_host may be NULL: then nothing
 * synchronises and no statistics are gathered. */
int insitu_attend(insitu_cache *cache, const int32_t *q_rot_dev, int32_t *out_dev, int32_t mode,
                  insitu_stats *stats_host);

/* A prefill's queries against one sequence's cache (attend_online_batch,
 * ops/attention.py:794-871, in SEQUENTIAL mode; attend_causal_batch, :517-670, in
 * TWO_PASS mode): query i (i < n_q) attends rows 0 .. base + i, exactly as a
 * decode step would (the prompt's rows are appended first). q_rot_dev int32
 * (n_q, n_q_heads, d) rotated; out_dev int32 (n_q, n_q_heads, d) Q16.
 * EBADLEN when base + n_q exceeds the sequence's length. stats_host may be NULL. */
int insitu_attend_causal(insitu_cache *cache, int32_t seq, int64_t base, int64_t n_q,
                         const int32_t *q_rot_dev, int32_t *out_dev, int32_t mode,
                         insitu_stats *stats_host);

/* The same for the G query heads of one KV head (CompressedAttention holds one KV
 * head's cache in the reference: attend_online / attend_two_pass, ops/attention.py:
 * 429-513, called from kernel.py:385-392 with kv = cache.view(h).select(slice(0, ctx));
 * attend_online_batch / attend_causal_batch, :517-871, called from kernel.py:317-331).
 * Query i (i < n_q) of (seq, kv_head) attends that head's rows 0 .. base + i; a decode
 * step over rows 0 .. n - 1 is base = n - 1, n_q = 1. q_rot_dev int32 (n_q, G, d)
 * rotated; out_dev int32 (n_q, G, d) Q16; the statistics are this head's alone.
 * EBADLEN when base + n_q exceeds the sequence's length. */
int insitu_attend_causal_head(insitu_cache *cache, int32_t seq, int32_t kv_head, int64_t base,
                              int64_t n_q, const int32_t *q_rot_dev, int32_t *out_dev, int32_t mode,
                              insitu_stats *stats_host);

/* insitu_attend_causal without allocating: no counterpart in the reference; for callers
 * that cannot call hipMalloc (tight serving loops, harnesses that forbid it). The same
 * launches and results as insitu_attend_causal, but the chunk scratch and the lengths of
 * the virtual batch live in a fixed device array of the library (64 MiB, one per device,
 * set up by insitu_ctx_create) instead of buffers the cache allocates. A launch takes as
 * many queries as fit it; EBADLEN when a single query's scratch does not (its size is in
 * the message). No statistics (nothing is copied back) and no timing events. Every call on
 * a device shares that device's array: calls that overlap on one device (two streams, two
 * threads) race and must not. Stream-ordered on the cache's context. Not for HIP graph
 * capture: each call takes its scratch epoch from a host counter into the launch's
 * arguments, so a replayed graph would run every replay under the captured epoch. */
int insitu_attend_causal_static(insitu_cache *cache, int32_t seq, int64_t base, int64_t n_q,
                                const int32_t *q_rot_dev, int32_t *out_dev, int32_t mode);

/* -- the host half either side of the seam (kernel.py:198-249, 348-356) -------------- */

/* A projection (ops/project.py:21-52, numerics/fp.py:25-44): y_dev fp32 (n, out_f) =
 * fp16(x_dev) (n, in_f) @ w_dev^T + bias_dev, fp16 weights (out_f, in_f) in the
 * checkpoint's layout, fp32 accumulation. x_dev fp32 is rounded to fp16 (nearest
 * even) first. bias_dev (out_f) fp32 may be NULL. Stream-ordered on the context. */
int insitu_project(insitu_ctx *ctx, const uint16_t *w_dev, int32_t out_f, int32_t in_f,
                   const float *x_dev, int64_t n, const float *bias_dev, float *y_dev);

/* The seam (kernel.py:209-249): p_dev fp32 (n, (n_q + 2 n_kv) d), the q|k|v projections
 * of n tokens, bias_dev fp32 ((n_q + 2 n_kv) d) or NULL, added in fp32; q times
 * attn_scale in float64; then cast_after_rope = 0: to_fixed (ops/convert.py:44-57) and
 * RoPE in fixed point (ops/rope.py:144-174), or 1: RoPE in float64 (:176-198) and
 * to_fixed. cos/sin_dev int64 (max_pos, d/2) Q(frac); pos_dev int64 (n), or NULL for the
 * consecutive positions pos0 .. pos0 + n - 1 (a decode step needs no upload). Writes the
 * wire rows q_dev (n, n_q, d), k/v_dev (n, n_kv, d) int32 Q8.16 (RoPE's output is
 * not clamped, as in the reference). counts_host (2) may be NULL; otherwise the call
 * synchronises and returns {values saturated by to_fixed, rows whose position is
 * beyond the table}, and ERANGE when the second is not 0. With counts_host NULL the
 * call is stream-ordered and checks nothing on the device: the caller keeps every
 * position in [0, max_pos) (a q/k row at a position beyond it is left unwritten). */
int insitu_seam_wire(insitu_ctx *ctx, const float *p_dev, const float *bias_dev, int64_t n, int32_t n_q,
                     int32_t n_kv, int32_t d, const int64_t *pos_dev, int64_t pos0, const int64_t *cos_dev,
                     const int64_t *sin_dev, int64_t max_pos, int32_t frac, double attn_scale,
                     int32_t cast_after_rope, int32_t *q_dev, int32_t *k_dev, int32_t *v_dev,
                     unsigned long long *counts_host);

/* insitu_project then insitu_seam_wire (kernel.py:198-249) in one launch where the decode
 * projection takes it (n <= 4 tokens, in_f a multiple of 8, d even): the q|k|v
 * projections of x_dev fp32 (n, in_f) by w_dev fp16 ((n_q + 2 n_kv) d, in_f) into p_dev
 * fp32 (n, (n_q + 2 n_kv) d), unbiased, then the seam as insitu_seam_wire (bias_dev added
 * there) into q/k/v_dev, and counts_host as there. Elsewhere the two calls. */
int insitu_project_seam(insitu_ctx *ctx, const uint16_t *w_dev, int32_t in_f, const float *x_dev, int64_t n,
                        const float *bias_dev, int32_t n_q, int32_t n_kv, int32_t d, const int64_t *pos_dev,
                        int64_t pos0, const int64_t *cos_dev, const int64_t *sin_dev, int64_t max_pos,
                        int32_t frac, double attn_scale, int32_t cast_after_rope, float *p_dev, int32_t *q_dev,
                        int32_t *k_dev, int32_t *v_dev, unsigned long long *counts_host);

/* The output side (kernel.py:348-356): out_dev int32 (n, width) Q(frac) -> float ->
 * fp16, then y_dev fp32 (n, hidden) = that @ wo_dev^T + bias_dev with W_o' fp16
 * (hidden, width), R^-1 folded in (ops/output.py:49-78). bias_dev may be NULL. */
int insitu_output_projection(insitu_ctx *ctx, const int32_t *out_dev, int64_t n, int32_t width,
                             int32_t frac, const uint16_t *wo_dev, int32_t hidden, const float *bias_dev,
                             float *y_dev);

/* One decode step from the wire (CMD_STEP, host/attn_proto.py:65-72; kernel.py:256-353):
 * q/k/v_dev int32 Q8.16 (batch, heads, d) -> rotate -> append -> attend -> out_dev. */
int insitu_step(insitu_cache *cache, const int32_t *q_dev, const int32_t *k_dev,
                const int32_t *v_dev, int32_t *out_dev, int32_t mode, insitu_stats *stats_host);

/* Byte-exact rows (view_from_buffer, compressed.py:123-129; CMD_LOAD, attn_proto.py:75-78).
 * rows_host uint8 (n, row_bytes). Synchronous. */
int insitu_read_rows(insitu_cache *cache, int32_t seq, int32_t head, int64_t t0, int64_t n,
                     uint8_t *rows_host);
int insitu_load_rows(insitu_cache *cache, int32_t seq, int32_t head, int64_t t0, int64_t n,
                     const uint8_t *rows_host);

/* The raw plane image of one sequence (DdrLayout.image / CMD_LOAD, ddr_layout.py:227-248):
 * nbytes must equal insitu_layout.seq_stride. Synchronous. */
int insitu_read_image(insitu_cache *cache, int32_t seq, uint8_t *image_host, int64_t nbytes);
int insitu_load_image(insitu_cache *cache, int32_t seq, const uint8_t *image_host, int64_t nbytes);

/* -- measurement probes (no counterpart in the reference's path: the analogue of its
 *    DDR bandwidth probe, rtl/ddr_probe.sv) ------------------------------------- */

/* Read nbytes (a positive multiple of 64) of src_dev with n_wg workgroups of 256 threads,
 * 16-byte loads; layout 0 grid-stride, 1 one contiguous span per workgroup. Writes nothing
 * of use to sink_dev (uint32 [256]). Stream-ordered; timed like an attend while
 * insitu_ctx_timing is on. */
int insitu_probe_read(insitu_ctx *ctx, const void *src_dev, int64_t nbytes, int32_t n_wg,
                      int32_t layout, uint32_t *sink_dev);
/* An empty kernel of n_wg workgroups: the launch floor. */
int insitu_probe_empty(insitu_ctx *ctx, int32_t n_wg, uint32_t *sink_dev);

/* -- test hooks (no counterpart in the reference) ----------------------------------- */
enum {
    INSITU_DEBUG_DECODE_CALLS = 1,   /* attends the decode scratch has served (its epoch counter) */
    INSITU_DEBUG_PREFILL_CALLS = 2,  /* the same for the prefill scratch                         */
    INSITU_DEBUG_SPIN_LIMIT = 3,     /* polls before a wait on another workgroup gives up; 0 gives
                                        up at once, sending every chain with a predecessor to the
                                        exact serial path                                       */
    INSITU_DEBUG_PATH = 4,           /* the kernel of a sequential-mode attend: 0 automatic (the
                                        decode step on its own kernel where it handles the cache,
                                        the chunked attend where it handles the cache, the scan
                                        attend elsewhere), 1 the scan attend, 2 the chunked attend
                                        (the decode step too), 3 the decode step's own kernel;
                                        INSITU_EINVAL if the kernel does not handle the cache   */
    INSITU_DEBUG_APPEND = 5          /* the append's kernel: 0 automatic (lane = row where it
                                        handles the format: d = 64, 4/2- or 2/2-bit codes), 1 the
                                        lane-per-channel kernel for every format                */
};
int insitu_cache_debug(insitu_cache *cache, int32_t what, int64_t value);
/* The statistics the cache's kernels have gathered since they were last cleared (an
 * attend that returns statistics clears them first; an append's range errors are
 * otherwise seen nowhere), copied into stats_host and then cleared. Synchronises. */
int insitu_cache_stats(insitu_cache *cache, insitu_stats *stats_host);
/* The invariants of a scratch layout, computed on the host without a GPU: kernel 0 the
 * chunked attend (1,024-token chunks), 1 the chunked attend (512), 2 the decode step's own
 * kernel (d = 64), for a cache of `capacity` tokens, batch sequences and n_kv KV heads of
 * dimension d, 4 query heads per KV head. facts (n >= 11): chunks per sequence, run slots
 * per head, slots per chunk after chunk 0, one past the last chunk's slots, runs the replay
 * lists per head, most chunks per sequence, scratch bytes, bytes of the epoch-checked front,
 * 1 when every area is 256-aligned and ends before the next begins, tokens per chunk, the
 * slot id limit. */
int insitu_debug_scratch_layout(int32_t kernel, int64_t capacity, int32_t batch, int32_t n_kv, int32_t d,
                                int64_t *facts, int32_t n);

/* Message of the last failing call on this thread. */
const char *insitu_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
