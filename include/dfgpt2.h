/* dfgpt2.h — C ABI of the GPT-2 step's non-attention kernels in libdfattn.so (gfx950).
 *
 * The reference engine's training step (darkforest-core/src/engine/static_gpt2.rs:1375-1696)
 * calls these CUDA launchers around its attention; the reference symbols below keep their
 * signatures and semantics (null stream, void return, argument errors reported by
 * darkforest_sync, declared in dfattn.h). The dfgpt2_* entry points are the same kernels on an
 * explicit stream with a dfattn_status return. Every reduction adds in a fixed order (no
 * floating-point atomics), so results are bitwise reproducible from run to run.
 */
#ifndef DFGPT2_H
#define DFGPT2_H

#include "dfattn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* darkforest-cuda/kernels/layernorm.cu:97. out = (x - mean) * rstd * gamma + beta per row of
 * [batch, features], eps 1e-5; gamma / beta NULL mean 1 / 0; means / rstds ([batch]) may be NULL. */
void launch_layernorm(const float *x, const float *gamma, const float *beta, float *out, float *means,
                      float *rstds, uint32_t batch, uint32_t features);
/* layernorm.cu:187. grad_x overwritten; grad_gamma and grad_beta ([features], each may be NULL)
 * ACCUMULATE the column sums of grad_out * x_hat and of grad_out (the reference adds them with
 * atomics), so the caller zeroes them first. */
void launch_layernorm_backward(const float *grad_out, const float *x, const float *gamma, const float *means,
                               const float *rstds, float *grad_x, float *grad_gamma, float *grad_beta,
                               uint32_t batch, uint32_t features);
/* elementwise.cu:195, 217: tanh GELU, 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))). */
void launch_gelu(const float *x, float *out, uint32_t n);
void launch_gelu_backward(const float *grad_out, const float *x, float *grad_x, uint32_t n);
/* elementwise.cu:242: out[r, c] = input[r, c] + bias[c] over [batch, features] (out may be input),
 * the bias add after each linear layer's GEMM (lib.rs linear_into). elementwise.cu:62, 91, 119:
 * c = val, c = a + b, c = alpha * a over n values (residual adds and gradient scaling of the
 * step, lib.rs add_into / scale). One fp32 operation per value, as the reference. */
void launch_add_bias(const float *input, const float *bias, float *out, uint32_t batch, uint32_t features);
void launch_fill(float *c, float val, uint32_t n);
void launch_add(const float *a, const float *b, float *c, uint32_t n);
void launch_scale(const float *a, float alpha, float *c, uint32_t n);
/* matmul.cu:240: grad_bias[j] = sum over rows of grad_out[row, j] (overwritten). */
void launch_linear_grad_bias(const float *grad_out, float *grad_bias, uint32_t batch, uint32_t out_features);
/* matmul.cu:341: m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2;
 * p = p (1 - lr wd) - lr (m / bc1) / (sqrt(v / bc2) + eps), elementwise over n values. */
void launch_adamw_update(float *parameter, float *first_moment, float *second_moment, const float *gradient,
                         uint32_t n, float lr, float beta1, float beta2, float eps, float weight_decay,
                         float bias_correction1, float bias_correction2);

/* softmax.cu:396 — cross-entropy over a chunk of rows of logits [chunk_rows, cols]: the row's
 * softmax p overwrites logits, grad_logits = (p - one_hot(target)) / total_rows, and
 * *loss += -log(max(p_target, 1e-12)) / total_rows per row (float atomics, as the reference; the
 * engine zeroes *loss before the first chunk). targets: [chunk_rows] token ids.            */
void launch_fused_chunked_logit_ce(float *logits, const uint32_t *targets, float *grad_logits, float *loss,
                                   uint32_t chunk_rows, uint32_t cols, uint32_t total_rows);
/* elementwise.cu:268 — out[p, :] = weight[indices[p], :] for p < seq_len (ids not range-checked,
 * as in the reference). elementwise.cu:291 — grad_weight[indices[p], :] += grad_out[p, :]: the
 * rows of one id are summed in position order by one workgroup (no atomics, reproducible); the
 * caller zeroes grad_weight first, as the reference's wrapper does (lib.rs:1813).             */
void launch_embedding_forward(const uint32_t *indices, const float *weight, float *out, uint32_t seq_len,
                              uint32_t embed_dim);
void launch_embedding_backward(const uint32_t *indices, const float *grad_out, float *grad_weight,
                               uint32_t seq_len, uint32_t embed_dim);

/* Stream variants. Pointers must be 4-byte aligned; 16-byte aligned rows with features % 4 == 0
 * take the vectorised kernels. batch == 0 or n == 0 is a no-op (the bias gradient is then zero), and
 * the pointers of an empty tensor may be NULL. */
int dfgpt2_layernorm_forward(const float *x, const float *gamma, const float *beta, float *out, float *means,
                             float *rstds, uint32_t batch, uint32_t features, hipStream_t stream);
int dfgpt2_layernorm_backward(const float *grad_out, const float *x, const float *gamma, const float *means,
                              const float *rstds, float *grad_x, float *grad_gamma, float *grad_beta,
                              uint32_t batch, uint32_t features, hipStream_t stream);
int dfgpt2_gelu_forward(const float *x, float *out, size_t n, hipStream_t stream);
int dfgpt2_gelu_backward(const float *grad_out, const float *x, float *grad_x, size_t n, hipStream_t stream);
/* launch_add_bias on a stream. */
int dfgpt2_add_bias(const float *input, const float *bias, float *out, uint32_t batch, uint32_t features,
                    hipStream_t stream);
/* accumulate != 0: grad_bias += column sums (else overwritten). */
int dfgpt2_linear_grad_bias(const float *grad_out, float *grad_bias, uint32_t batch, uint32_t out_features,
                            int accumulate, hipStream_t stream);
/* The AdamW update with the step count on the device (a float, as PyTorch keeps it): the kernel
 * takes t = *step + 1 for the bias corrections 1 - beta^t, then *step becomes t. Nothing about the
 * step is read on the host, so a captured graph stays correct on replay. */
int dfgpt2_adamw_update(float *parameter, float *first_moment, float *second_moment, const float *gradient,
                        size_t n, float lr, float beta1, float beta2, float eps, float weight_decay, float *step,
                        hipStream_t stream);

/* The chunked cross-entropy on a stream: as launch_fused_chunked_logit_ce, except that the
 * softmax is not written back (grad_logits may be logits itself, which halves the chunk's write
 * traffic) and each row's loss, -log(max(p_target, 1e-12)) / total_rows, goes to row_loss[row]
 * instead of an atomic sum; dfgpt2_sum then adds the rows in a fixed order. Reference
 * counterpart: softmax.cu:396 as called at static_gpt2.rs:1386-1418.                        */
int dfgpt2_logit_ce_chunk(float *logits, const uint32_t *targets, float *grad_logits, float *row_loss,
                          uint32_t chunk_rows, uint32_t cols, uint32_t total_rows, hipStream_t stream);
/* *out = (accumulate ? *out : 0) + sum of values[0..n) in a fixed order (one workgroup). No
 * reference counterpart: the reference's loss is an atomic sum.                             */
int dfgpt2_sum(const float *values, uint32_t n, float *out, int accumulate, hipStream_t stream);
/* The embedding gather and its gradient on a stream (elementwise.cu:268, 291). Rows whose id is
 * rows_in_table or more are written as zeros (forward) or skipped (backward). The backward
 * sums each id's rows in position order (bitwise reproducible; the reference uses atomics); its
 * cost grows as n_rows^2 (id scans) and with the largest repeat count of one id (summed by one
 * workgroup), so it is meant for sequences of up to a few thousand positions.               */
int dfgpt2_embedding_forward(const uint32_t *indices, const float *table, float *out, uint32_t n_rows,
                             uint32_t dim, uint32_t rows_in_table, hipStream_t stream);
int dfgpt2_embedding_backward(const uint32_t *indices, const float *grad_out, float *grad_table, uint32_t n_rows,
                              uint32_t dim, uint32_t rows_in_table, hipStream_t stream);

/* Fused forms the engine's step uses; no reference counterparts (the reference's step runs these
 * as separate launches: a residual add, then LayerNorm, static_gpt2.rs:1341-1350, 1360 with
 * 1315 / 1364; LayerNorm's backward, then the residual gradient added, 1474-1486, 1543-1555; the
 * linear layer with its bias, then GELU, 1353-1355).
 * dfgpt2_add_layernorm_forward: sum_out = x + y (one fp32 add per value), out = LayerNorm(sum_out)
 * with means / rstds as dfgpt2_layernorm_forward. sum_out and out must not overlap x, y or each
 * other.                                                                                      */
int dfgpt2_add_layernorm_forward(const float *x, const float *y, const float *gamma, const float *beta,
                                 float *sum_out, float *out, float *means, float *rstds, uint32_t batch,
                                 uint32_t features, hipStream_t stream);
/* grad_x = LayerNorm backward of grad_out (+ residual when not NULL); grad_gamma and grad_beta
 * (either may be NULL) are WRITTEN, not added into, so the caller need not zero them. grad_x
 * must not overlap grad_out, x or residual.                                                  */
int dfgpt2_layernorm_backward_residual(const float *grad_out, const float *x, const float *gamma,
                                       const float *means, const float *rstds, const float *residual,
                                       float *grad_x, float *grad_gamma, float *grad_beta, uint32_t batch,
                                       uint32_t features, hipStream_t stream);
/* dfgpt2_layernorm_backward_residual, plus grad_bias[c] = sum over rows of grad_x[r, c] (the
 * bias gradient of the linear layer whose output gradient grad_x is; NULL: not computed), with
 * the rows read once: grad_x and each workgroup's partial column sums in one launch, then a
 * fixed-order sum of the partials. grad_gamma, grad_beta and grad_bias are WRITTEN. The
 * workspace (dfgpt2_layernorm_backward_fused_workspace_bytes, 4-byte aligned) holds the partial
 * sums; nothing in it needs clearing. Reproducible bit for bit; the sums' order differs from the
 * separate calls', so their last bits may too. Reference counterpart: separate launches, the
 * engine's LayerNorm backwards (static_gpt2.rs:1427, 1474, 1543) and the bias gradients of b2
 * and bo that the next linear backwards compute from their results (1451, 1490).            */
size_t dfgpt2_layernorm_backward_fused_workspace_bytes(uint32_t batch, uint32_t features);
int dfgpt2_layernorm_backward_fused(const float *grad_out, const float *x, const float *gamma,
                                    const float *means, const float *rstds, const float *residual,
                                    float *grad_x, float *grad_gamma, float *grad_beta, float *grad_bias,
                                    void *workspace, size_t workspace_bytes, uint32_t batch,
                                    uint32_t features, hipStream_t stream);
/* h[r, c] += bias[c] in place (the GELU input the backward needs), out = gelu(h); [rows, cols];
 * out must not overlap h.                                                                      */
int dfgpt2_bias_gelu_forward(float *h, const float *bias, float *out, uint32_t rows, uint32_t cols,
                             hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* DFGPT2_H */
