/*
 * dfattn.h — C ABI of the MI355X (gfx950) fused causal attention library.
 *
 * This is the drop-in boundary for Dark Forest's attention path. The library
 * (libdfattn.so) exports two groups of symbols:
 *
 *  1. The reference's own launcher symbols, with identical C signatures and
 *     semantics, so a binary that linked the reference's `darkforest_kernels`
 *     attention object links this library instead:
 *       launch_fused_attention     darkforest-cuda/kernels/attention_fused.cu:223
 *       launch_fused_mha_forward   darkforest-cuda/kernels/attention_fused.cu:233
 *       launch_attention_backward  darkforest-cuda/kernels/attention_fused.cu:361
 *       launch_fused_mha_backward  darkforest-cuda/kernels/attention_fused.cu:518
 *       darkforest_sync            darkforest-cuda/kernels/matmul.cu:21
 *     The Rust wrappers that bind them are darkforest-cuda/src/kernels.rs:689-885
 *     (cuda_fused_attention, cuda_attention_backward, cuda_fused_mha_forward,
 *     cuda_fused_mha_backward) and kernels.rs:9-20 (cuda_sync).
 *
 *  2. The fast path, which the reference does not have: a forward that also
 *     writes the natural-log logsumexp of every query row, and a backward that
 *     recomputes P from that logsumexp with an O(H*S*D) workspace instead of
 *     the reference's H*2*S*S probability scratch. These take an explicit HIP
 *     stream and return a status code; nothing aborts.
 *
 * Tensor layout (both groups), as in attention_fused.cu:60-66 and :404-414:
 * every tensor is fp32, contiguous, row-major [seq_len, n_heads * d_head];
 * head h occupies columns [h*d_head, (h+1)*d_head). Batch is 1. The
 * single-head launchers use [seq_len, d_head]. Logsumexp is fp32 [n_heads,
 * seq_len]: lse[h*seq_len + i] = ln sum_{j visible to i} exp(scale * q_i . k_j).
 *
 * `causal != 0` restricts query i to keys j <= i. `scale` multiplies q . k
 * before the softmax (the reference's callers pass 1/sqrt(d_head)).
 */
#ifndef DFATTN_H
#define DFATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Status codes of the fast-path entry points ------------------------ */
typedef enum dfattn_status {
  DFATTN_OK = 0,
  DFATTN_ERR_NULL_POINTER = -1,   /* a required pointer is NULL                 */
  DFATTN_ERR_MISALIGNED = -2,     /* a tensor pointer is not 4-byte aligned     */
  DFATTN_ERR_SHAPE = -3,          /* n_heads == 0 or seq_len == 0               */
  DFATTN_ERR_HEAD_DIM = -4,       /* d_head outside 1..=128                     */
  DFATTN_ERR_OVERFLOW = -5,       /* seq_len*n_heads*d_head does not fit, or    */
                                  /* seq_len > 2^30 or n_heads > 65535          */
  DFATTN_ERR_WORKSPACE = -6,      /* workspace NULL or smaller than required    */
  DFATTN_ERR_HIP = -7,            /* a HIP launch failed (see dfattn_last_error) */
  DFATTN_ERR_FLAGS = -8           /* unknown bits in a flags argument           */
} dfattn_status;

/* Flags of dfattn_bwd_preprocess. */
#define DFATTN_BWD_QKV_SAVED 1u /* the workspace holds dfattn_fwd_train's copies */

/* KV-cache element types of dfattn_decode. */
#define DFATTN_KV_F32 0u  /* fp32 rows                                        */
#define DFATTN_KV_BF16 1u /* bf16 bit patterns in uint16 (the reference's      */
                          /* __nv_bfloat16 pools)                             */

/* ---- Group 1: the reference's launcher symbols ---------------------------
 * Same signatures as the reference. Launches go to the legacy default (null)
 * stream; the functions return nothing. Argument errors that the reference
 * would turn into a device trap (d_head > 128) or a failed launch are recorded
 * instead and reported by darkforest_sync(), which, like the reference,
 * prints the error and aborts.                                              */

/* attention_fused.cu:223 — single-head forward, tensors [seq_len, d_head].  */
void launch_fused_attention(const float *q, const float *k, const float *v,
                            float *out, uint32_t seq_len, uint32_t d_head,
                            float scale, uint32_t causal);

/* attention_fused.cu:233 — multi-head forward, tensors [seq_len, H*d_head].
 * Writes O only (the reference has no logsumexp output).                   */
void launch_fused_mha_forward(const float *q, const float *k, const float *v,
                              float *out, uint32_t n_heads, uint32_t seq_len,
                              uint32_t d_head, float scale, uint32_t causal);

/* attention_fused.cu:361 — single-head backward. `probabilities` is the
 * caller's [seq_len, seq_len] fp32 scratch; it is used as workspace for O,
 * logsumexp and row statistics when large enough. dQ, dK, dV are fully
 * overwritten (the reference zeroes dK and dV itself, :367-369).           */
void launch_attention_backward(const float *q, const float *k, const float *v,
                               const float *d_out, float *d_q, float *d_k,
                               float *d_v, float *probabilities,
                               uint32_t seq_len, uint32_t d_head, float scale,
                               uint32_t causal);

/* attention_fused.cu:518 — multi-head backward. `probabilities` is the
 * caller's [n_heads, 2, seq_len, seq_len] fp32 scratch (lib.rs:2023).      */
void launch_fused_mha_backward(const float *q, const float *k, const float *v,
                               const float *d_out, float *d_q, float *d_k,
                               float *d_v, float *probabilities,
                               uint32_t n_heads, uint32_t seq_len,
                               uint32_t d_head, float scale, uint32_t causal);

/* Decode: one query row q [H*d_head] against the first cur_seq_len rows of a
 * KV cache, out [H*d_head] (nothing written when cur_seq_len is 0, as the
 * reference's kernels return early). d_head 1..=128. Contiguous caches are
 * [max_seq_len, H*d_head]; paged pools are [n_blocks * page_size,
 * H*d_head] with row t at block_table[t / page_size] * page_size +
 * t % page_size. The split-K variants take the caller's partial buffers in
 * the reference's layout (m, l: [H, n_chunks]; o: [H, n_chunks, d_head],
 * n_chunks = ceil(cur_seq_len / chunk_size)) and, like the reference, do not
 * split when cur_seq_len <= chunk_size; chunk_size 0 and page_size 0 are
 * recorded as argument errors (the reference divides by them).             */

/* attention_fused.cu:617 — contiguous fp32 cache.                          */
void launch_fused_mha_decode_kv(const float *q, const float *k_cache,
                                const float *v_cache, float *out,
                                uint32_t n_heads, uint32_t cur_seq_len,
                                uint32_t d_head, float scale);
/* attention_fused.cu:762 — contiguous fp32 cache, split over the keys.     */
void launch_fused_mha_decode_kv_splitk(const float *q, const float *k_cache,
                                       const float *v_cache, float *partial_m,
                                       float *partial_l, float *partial_o,
                                       float *out, uint32_t n_heads,
                                       uint32_t cur_seq_len, uint32_t d_head,
                                       float scale, uint32_t chunk_size);
/* attention_fused.cu:1028 — paged fp32 pool.                               */
void launch_paged_mha_decode_kv(const float *q, const float *k_pool,
                                const float *v_pool, const int32_t *block_table,
                                float *out, uint32_t n_heads,
                                uint32_t cur_seq_len, uint32_t d_head,
                                float scale, uint32_t page_size);
/* attention_fused.cu:1045 — paged fp32 pool, split over the keys.          */
void launch_paged_mha_decode_kv_splitk(const float *q, const float *k_pool,
                                       const float *v_pool,
                                       const int32_t *block_table,
                                       float *partial_m, float *partial_l,
                                       float *partial_o, float *out,
                                       uint32_t n_heads, uint32_t cur_seq_len,
                                       uint32_t d_head, float scale,
                                       uint32_t page_size, uint32_t chunk_size);
/* attention_fused.cu:1075 — paged bf16 pool (bit patterns as uint16).      */
void launch_paged_mha_decode_kv_bf16(const float *q, const uint16_t *k_pool,
                                     const uint16_t *v_pool,
                                     const int32_t *block_table, float *out,
                                     uint32_t n_heads, uint32_t cur_seq_len,
                                     uint32_t d_head, float scale,
                                     uint32_t page_size);

/* The elementwise kernels that share the reference's attention object. All
 * run on the null stream; argument errors are recorded for darkforest_sync. */

/* attention_fused.cu:1123 — out [d_model] := row pos of the trained table
 * [trained_ctx_len, d_model] when pos < trained_ctx_len and max_ctx_len <=
 * trained_ctx_len; otherwise the linear interpolation at position
 * pos * (trained_ctx_len - 1) / (max_ctx_len - 1). A position past the
 * table's last row (where the reference reads out of bounds) gives the last
 * row. trained_ctx_len 0 is an argument error.                             */
void launch_pos_embed_interpolate(const float *pos_table, float *out,
                                  uint32_t pos, uint32_t trained_ctx_len,
                                  uint32_t max_ctx_len, uint32_t d_model);
/* attention_fused.cu:1164 — rotary embedding of one row qk [n_heads *
 * d_head] in place: values (2i, 2i+1) of each head rotated by the angle
 * pos * base_freq^(-2i / d_head). n_heads 0 and d_head < 2 (an invalid
 * launch in the reference) are argument errors.                            */
void launch_apply_rope(float *qk, uint32_t pos, uint32_t n_heads,
                       uint32_t d_head, float base_freq);
/* attention_fused.cu:1192 — row phys_block * page_size + page_offset of a
 * paged pool [n_blocks * page_size, d_model] := src [d_model]. A negative
 * phys_block or page_offset >= page_size is an argument error.            */
void launch_paged_copy_row(const float *src, float *pool, int32_t phys_block,
                           uint32_t page_offset, uint32_t page_size,
                           uint32_t d_model);
/* attention_fused.cu:1219 — the same into a bf16 pool (bit patterns as
 * uint16), each value rounded to nearest even.                             */
void launch_paged_copy_row_f32_to_bf16(const float *src, uint16_t *pool,
                                       int32_t phys_block, uint32_t page_offset,
                                       uint32_t page_size, uint32_t d_model);

/* matmul.cu:21 — device synchronize; on a HIP error, or on an argument
 * error of one of the launchers above since the last sync, print
 * "[darkforest] ..." to stderr and abort(), as the reference does. Errors
 * the status-returning entry points below already returned do not abort.   */
void darkforest_sync(void);

/* ---- Group 2: fast path -------------------------------------------------
 * `stream` is a hipStream_t passed as an opaque pointer (NULL = the null
 * stream). All validation happens on the host before any HIP call; on error
 * nothing is launched and a negative dfattn_status is returned.
 * d_head = 64 runs on fp16 MFMA operands: scale*log2(e)*q, k and v are
 * rounded to fp16, so their magnitudes must stay below 65504 (fp16's largest
 * finite value); beyond it they overflow and the outputs are not finite.
 * d_out needs no such bound (each 64-row block is scaled by a power of two
 * before rounding, and dK, dV are summed in the units of the block of
 * largest magnitude). Other d_head values run in fp32 like the reference. */

/* Forward: O [S, H*D] and lse [H, S] (lse may be NULL to skip it).
 * No allocation: only the caller's Q, K, V, O and lse are touched.
 * Reference counterpart: launch_fused_mha_forward (attention_fused.cu:233),
 * plus the logsumexp output that the reference does not produce.           */
int dfattn_fwd(const float *q, const float *k, const float *v, float *o,
               float *lse, uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
               float scale, uint32_t causal, void *stream);

/* Forward of a training step: everything dfattn_fwd does (lse required),
 * and, on the d_head = 64 fast path, the backward's fp16 copies of
 * scale*log2(e)*Q, K and V written into `workspace` (which must hold
 * dfattn_bwd_workspace_bytes()), rounded exactly as the backward rounds
 * them. A later dfattn_bwd_preprocess with DFATTN_BWD_QKV_SAVED on the same
 * q, k, v, scale and workspace then converts only dO (about 56 MB less
 * traffic at H = 12, S = 4096). No reference counterpart: the reference's
 * backward recomputes the forward from scratch (attention_fused.cu:390-516). */
int dfattn_fwd_train(const float *q, const float *k, const float *v, float *o,
                     float *lse, void *workspace, size_t workspace_bytes,
                     uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
                     float scale, uint32_t causal, void *stream);

/* Bytes of device workspace dfattn_bwd needs: O(n_heads * seq_len * d_head)
 * (a power-of-two dO scale per 64-row block, the row statistics -lse*log2(e)
 * and -Delta_i (Delta_i = dO_i . O_i) as the main phase's products take
 * them, fp16 copies of the scaled Q, K, V and dO that the main phase
 * reads, and the fp16 rounding residues of the first 64 rows of the scaled
 * Q, K and dO, 24 KB per head; about 8 bytes per element of one input,
 * 25 MB at H = 12, S = 4096, D = 64).
 * Returns 0 when the arguments are invalid.                                */
size_t dfattn_bwd_workspace_bytes(uint32_t n_heads, uint32_t seq_len,
                                  uint32_t d_head);

/* Backward from the forward's O and lse: writes dQ, dK, dV [S, H*D] (all
 * fully overwritten). `workspace` must hold dfattn_bwd_workspace_bytes().
 * Reference counterpart: launch_fused_mha_backward (attention_fused.cu:518),
 * which recomputes the softmax from scratch with an O(S^2) buffer instead. */
int dfattn_bwd(const float *q, const float *k, const float *v, const float *o,
               const float *d_o, const float *lse, float *d_q, float *d_k,
               float *d_v, void *workspace, size_t workspace_bytes,
               uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
               float scale, uint32_t causal, void *stream);

/* The two phases of dfattn_bwd, for callers that schedule or time them
 * separately (dfattn_bwd is exactly preprocess then main, on one stream,
 * with one workspace). Preprocess reads Q, K, V, O, dO and lse and fills
 * the workspace (row statistics and the fp16 operand copies); main reads
 * the workspace and writes dQ, dK, dV. Pass both phases the same
 * q, k, v, o, d_o, lse, workspace and scale. flags: 0, or
 * DFATTN_BWD_QKV_SAVED when a dfattn_fwd_train with the same q, k, v,
 * scale and workspace has run and neither q, k, v nor the workspace has
 * changed since (preprocess then converts only dO). No reference
 * counterpart: the
 * reference backward is one kernel without saved statistics
 * (attention_fused.cu:390-516).                                             */
int dfattn_bwd_preprocess(const float *q, const float *k, const float *v,
                          const float *o, const float *d_o, const float *lse,
                          void *workspace, size_t workspace_bytes, uint32_t n_heads,
                          uint32_t seq_len, uint32_t d_head, float scale, uint32_t flags,
                          void *stream);
int dfattn_bwd_main(const float *q, const float *k, const float *v,
                    const float *o, const float *d_o, const float *lse, float *d_q,
                    float *d_k, float *d_v, void *workspace, size_t workspace_bytes,
                    uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
                    float scale, uint32_t causal, void *stream);

/* The training pair with row strides. No counterpart in the reference (its
 * engine keeps Q, K, V and their gradients in separate [S, H*D] tensors):
 * for callers whose Q, K, V are the three column blocks of one fused
 * projection [S, 3*H*D] and whose gradients go back into one such tensor,
 * which saves splitting and re-interleaving them. Same semantics and
 * results, bit for bit, as dfattn_fwd_train, dfattn_bwd_preprocess and
 * dfattn_bwd_main with contiguous tensors, except that row i of q, k and v
 * starts qkv_row_stride floats after row i-1 (each buffer must hold
 * (seq_len-1)*stride + n_heads*d_head floats), and likewise d_q, d_k, d_v
 * with grad_row_stride; o, d_o and lse stay contiguous. d_head must be 64,
 * every tensor 16-byte aligned, and a stride at least n_heads*d_head, a
 * multiple of 4 and at most 2^21 (else DFATTN_ERR_HEAD_DIM,
 * DFATTN_ERR_MISALIGNED or DFATTN_ERR_SHAPE). The main phase reads only the
 * workspace, lse and its outputs, so it takes no q, k, v.                  */
int dfattn_fwd_train_strided(const float *q, const float *k, const float *v, float *o,
                             float *lse, void *workspace, size_t workspace_bytes,
                             uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
                             float scale, uint32_t causal, uint32_t qkv_row_stride,
                             void *stream);
int dfattn_bwd_preprocess_strided(const float *q, const float *k, const float *v,
                                  const float *o, const float *d_o, const float *lse,
                                  void *workspace, size_t workspace_bytes,
                                  uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
                                  float scale, uint32_t flags, uint32_t qkv_row_stride,
                                  void *stream);
int dfattn_bwd_main_strided(const float *lse, float *d_q, float *d_k, float *d_v,
                            void *workspace, size_t workspace_bytes, uint32_t n_heads,
                            uint32_t seq_len, uint32_t d_head, float scale, uint32_t causal,
                            uint32_t grad_row_stride, void *stream);

/* Backward that allocates nothing. No counterpart in the reference: it is
 * for callers that cannot call hipMalloc or take a workspace (code under
 * HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). Same arguments, semantics and results as dfattn_bwd without
 * the workspace: the workspace lives in a static device array of
 * DFATTN_NOALLOC_SCRATCH_BYTES per GPU, held from the library's load until
 * the process ends. Shapes whose dfattn_bwd_workspace_bytes() exceeds it
 * (for d_head = 64: n_heads * seq_len above about 63,900, e.g. H = 12,
 * S = 4096 fits) return DFATTN_ERR_WORKSPACE before any HIP call. Every
 * call on one GPU uses that GPU's one array: calls that overlap on one GPU
 * (different streams, or threads) race and give wrong results; serialise
 * them. Nothing in the array needs to be cleared between calls. The first
 * call on a device, which places the array, may itself run under stream
 * capture: it enqueues nothing beyond the backward's kernels.              */
#define DFATTN_NOALLOC_SCRATCH_BYTES (32u << 20)
int dfattn_bwd_noalloc(const float *q, const float *k, const float *v,
                       const float *o, const float *d_o, const float *lse,
                       float *d_q, float *d_k, float *d_v, uint32_t n_heads,
                       uint32_t seq_len, uint32_t d_head, float scale,
                       uint32_t causal, void *stream);

/* Decode on a stream with a status: the five launchers above in one entry
 * point. block_table NULL: contiguous cache (page_size ignored); kv_dtype
 * DFATTN_KV_F32 or DFATTN_KV_BF16 (k_cache, v_cache then point to uint16
 * bf16 bit patterns). lse [H] (natural log of the sum of exp(scale*q.k),
 * may be NULL) lets callers merge decodes over sharded caches. With a
 * workspace of dfattn_decode_workspace_bytes the keys are split over enough
 * workgroups to fill the GPU; with workspace NULL one workgroup per head
 * walks them all. cur_seq_len 0 returns DFATTN_OK and writes nothing.
 * Reference counterparts: attention_fused.cu:617, 762, 1028, 1045, 1075
 * (the reference's launchers have no stream, no status and no lse).       */
size_t dfattn_decode_workspace_bytes(uint32_t n_heads, uint32_t cur_seq_len,
                                     uint32_t d_head);
int dfattn_decode(const float *q, const void *k_cache, const void *v_cache,
                  const int32_t *block_table, uint32_t page_size,
                  uint32_t kv_dtype, float *out, float *lse, uint32_t n_heads,
                  uint32_t cur_seq_len, uint32_t d_head, float scale,
                  void *workspace, size_t workspace_bytes, void *stream);

/* ---- Group 3: the reference's per-layer attention context ---------------
 * Mirror of AttentionContext (darkforest-cuda/src/lib.rs:1949-2368), the
 * object each layer of the reference's static GPT-2 engine owns
 * (static_gpt2.rs:401-406). All device buffers it needs (logsumexp [H, S]
 * and the backward workspace, O(H*S*D)) are allocated by create; the reference
 * instead allocates an H*2*S*S scratch on the first backward (lib.rs:2019).
 * The context is internally locked, like the reference's Mutex fields.    */
typedef struct dfattn_context dfattn_context;

/* lib.rs:1966 AttentionContext::new (and :1975 new_shared): d_head in
 * 1..=128, n_heads*d_head and seq_len*d_model must not overflow.            */
int dfattn_context_create(uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
                          dfattn_context **out);
void dfattn_context_destroy(dfattn_context *ctx);
int dfattn_context_dims(const dfattn_context *ctx, uint32_t *n_heads, uint32_t *seq_len,
                        uint32_t *d_head, uint32_t *d_model);
/* The context's logsumexp buffer [n_heads, seq_len], written by every
 * forward (device pointer; NULL for a NULL context).                        */
const float *dfattn_context_lse(const dfattn_context *ctx);

/* Opt-in forward reuse for the backward (no reference counterpart; the
 * reference always recomputes). enable != 0 promises that between a
 * forward_device_into and the backward_device_into on the same q, k, v,
 * neither q, k, v nor that forward's `out` is modified or freed — the
 * reference's static engine keeps them in its arena untouched
 * (static_gpt2.rs:1329-1336, 1500-1510). Breaking the promise gives stale
 * gradients (or reads freed memory as O); it is not detected.              */
int dfattn_context_set_reuse_forward(dfattn_context *ctx, uint32_t enable);

/* lib.rs:2042 forward_device_into: O [seq_len, d_model] from device Q, K, V;
 * out_elems must equal seq_len * d_model ("attention output shape
 * mismatch"). Also writes the context's logsumexp and remembers q, k, v and
 * out for the backward.                                                     */
int dfattn_context_forward_device_into(dfattn_context *ctx, const float *q, const float *k,
                                       const float *v, float scale, uint32_t causal,
                                       float *out, size_t out_elems, void *stream);

/* lib.rs:2240 backward_device_into: dQ, dK, dV (each seq_len * d_model =
 * grad_elems), computed from the current contents of q, k, v and d_out: by
 * default the forward is recomputed first, as the reference does. With
 * reuse enabled (dfattn_context_set_reuse_forward) and the same q, k, v
 * pointers, scale and causal flag as the last forward_device_into, the O,
 * logsumexp and fp16 operand copies of that forward are reused instead.    */
int dfattn_context_backward_device_into(dfattn_context *ctx, const float *q, const float *k,
                                        const float *v, const float *d_out, float scale,
                                        uint32_t causal, float *d_q, float *d_k, float *d_v,
                                        size_t grad_elems, void *stream);

/* The two calls above with row strides: q, k, v read at qkv_row_stride
 * floats per row, d_q, d_k, d_v written at grad_row_stride (out and d_out
 * contiguous), through the strided training pair above. No counterpart in
 * the reference: for an engine whose Q/K/V projection is one fused GEMM
 * with an [S, 3*H*D] output and whose Q/K/V gradients feed one such GEMM.
 * A stride of exactly n_heads*d_head is the contiguous layout and takes
 * the unstrided call (any d_head). A reused forward
 * (dfattn_context_set_reuse_forward) must have had the same q, k, v
 * pointers and row stride.                                               */
int dfattn_context_forward_device_into_strided(dfattn_context *ctx, const float *q,
                                               const float *k, const float *v, float scale,
                                               uint32_t causal, float *out, size_t out_elems,
                                               uint32_t qkv_row_stride, void *stream);
int dfattn_context_backward_device_into_strided(dfattn_context *ctx, const float *q,
                                                const float *k, const float *v,
                                                const float *d_out, float scale, uint32_t causal,
                                                float *d_q, float *d_k, float *d_v,
                                                size_t grad_elems, uint32_t qkv_row_stride,
                                                uint32_t grad_row_stride, void *stream);

/* lib.rs:2295 forward / :2328 backward: host slices of seq_len * d_head
 * floats uploaded into context buffers and run on the single-head path, as
 * the reference does; backward differentiates the last host forward's
 * q, k, v. Synchronous.                                                     */
int dfattn_context_forward(dfattn_context *ctx, const float *q, const float *k, const float *v,
                           size_t len, float scale, uint32_t causal, float *out);
int dfattn_context_backward(dfattn_context *ctx, const float *d_out, size_t len, float scale,
                            uint32_t causal, float *d_q, float *d_k, float *d_v);

/* lib.rs:2371 fused_attention_forward and :2421 attention_backward: one
 * head [seq_len, d_head] from host slices through device buffers allocated
 * for the call. Synchronous.                                                */
int dfattn_fused_attention_forward(const float *q, const float *k, const float *v, size_t len,
                                   uint32_t seq_len, uint32_t d_head, float scale,
                                   uint32_t causal, float *out);
int dfattn_attention_backward(const float *q, const float *k, const float *v,
                              const float *d_out, size_t len, uint32_t seq_len,
                              uint32_t d_head, float scale, uint32_t causal, float *d_q,
                              float *d_k, float *d_v);

/* Human-readable name of a dfattn_status value.                             */
const char *dfattn_status_string(int status);

/* The last error recorded by any entry point of this library on any thread
 * (0 if none), and a message for it; dfattn_clear_error() resets it and the
 * launcher error darkforest_sync() would report.                          */
int dfattn_last_error(void);
const char *dfattn_last_error_message(void);
void dfattn_clear_error(void);

/* Library version string and the device architecture the kernels target.   */
const char *dfattn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DFATTN_H */
