//! Raw declarations of every entry point of `include/dfgpt2.h` (the GPT-2 step's non-GEMM kernels
//! in libdfattn). `hipStream_t` is `*mut c_void`. `tests/test_rust_crate.py` checks every
//! declaration here against the header.

use std::os::raw::{c_int, c_void};

#[link(name = "dfattn")]
extern "C" {
    // The reference's launchers (layernorm.cu:97, 187; elementwise.cu:62, 91, 119, 195, 217, 242, 268, 291;
    // matmul.cu:240, 341; softmax.cu:396): null stream, void, errors reported by `darkforest_sync`.
    pub fn launch_layernorm(x: *const f32, gamma: *const f32, beta: *const f32, out: *mut f32,
                            means: *mut f32, rstds: *mut f32, batch: u32, features: u32);
    pub fn launch_layernorm_backward(grad_out: *const f32, x: *const f32, gamma: *const f32,
                                     means: *const f32, rstds: *const f32, grad_x: *mut f32,
                                     grad_gamma: *mut f32, grad_beta: *mut f32, batch: u32, features: u32);
    pub fn launch_gelu(x: *const f32, out: *mut f32, n: u32);
    pub fn launch_gelu_backward(grad_out: *const f32, x: *const f32, grad_x: *mut f32, n: u32);
    pub fn launch_add_bias(input: *const f32, bias: *const f32, out: *mut f32, batch: u32, features: u32);
    pub fn launch_fill(c: *mut f32, val: f32, n: u32);
    pub fn launch_add(a: *const f32, b: *const f32, c: *mut f32, n: u32);
    pub fn launch_scale(a: *const f32, alpha: f32, c: *mut f32, n: u32);
    pub fn launch_linear_grad_bias(grad_out: *const f32, grad_bias: *mut f32, batch: u32, out_features: u32);
    pub fn launch_adamw_update(parameter: *mut f32, first_moment: *mut f32, second_moment: *mut f32,
                               gradient: *const f32, n: u32, lr: f32, beta1: f32, beta2: f32, eps: f32,
                               weight_decay: f32, bias_correction1: f32, bias_correction2: f32);
    pub fn launch_fused_chunked_logit_ce(logits: *mut f32, targets: *const u32, grad_logits: *mut f32,
                                         loss: *mut f32, chunk_rows: u32, cols: u32, total_rows: u32);
    pub fn launch_embedding_forward(indices: *const u32, weight: *const f32, out: *mut f32, seq_len: u32,
                                    embed_dim: u32);
    pub fn launch_embedding_backward(indices: *const u32, grad_out: *const f32, grad_weight: *mut f32,
                                     seq_len: u32, embed_dim: u32);

    // Stream entry points of the engine's step (no reference counterpart): status return.
    pub fn dfgpt2_layernorm_forward(x: *const f32, gamma: *const f32, beta: *const f32, out: *mut f32,
                                    means: *mut f32, rstds: *mut f32, batch: u32, features: u32,
                                    stream: *mut c_void) -> c_int;
    pub fn dfgpt2_layernorm_backward(grad_out: *const f32, x: *const f32, gamma: *const f32,
                                     means: *const f32, rstds: *const f32, grad_x: *mut f32,
                                     grad_gamma: *mut f32, grad_beta: *mut f32, batch: u32, features: u32,
                                     stream: *mut c_void) -> c_int;
    pub fn dfgpt2_gelu_forward(x: *const f32, out: *mut f32, n: usize, stream: *mut c_void) -> c_int;
    pub fn dfgpt2_gelu_backward(grad_out: *const f32, x: *const f32, grad_x: *mut f32, n: usize,
                                stream: *mut c_void) -> c_int;
    pub fn dfgpt2_add_bias(input: *const f32, bias: *const f32, out: *mut f32, batch: u32, features: u32,
                           stream: *mut c_void) -> c_int;
    pub fn dfgpt2_linear_grad_bias(grad_out: *const f32, grad_bias: *mut f32, batch: u32, out_features: u32,
                                   accumulate: c_int, stream: *mut c_void) -> c_int;
    pub fn dfgpt2_adamw_update(parameter: *mut f32, first_moment: *mut f32, second_moment: *mut f32,
                               gradient: *const f32, n: usize, lr: f32, beta1: f32, beta2: f32, eps: f32,
                               weight_decay: f32, step: *mut f32, stream: *mut c_void) -> c_int;
    pub fn dfgpt2_logit_ce_chunk(logits: *mut f32, targets: *const u32, grad_logits: *mut f32,
                                 row_loss: *mut f32, chunk_rows: u32, cols: u32, total_rows: u32,
                                 stream: *mut c_void) -> c_int;
    pub fn dfgpt2_sum(values: *const f32, n: u32, out: *mut f32, accumulate: c_int, stream: *mut c_void) -> c_int;
    pub fn dfgpt2_embedding_forward(indices: *const u32, table: *const f32, out: *mut f32, n_rows: u32,
                                    dim: u32, rows_in_table: u32, stream: *mut c_void) -> c_int;
    pub fn dfgpt2_embedding_backward(indices: *const u32, grad_out: *const f32, grad_table: *mut f32,
                                     n_rows: u32, dim: u32, rows_in_table: u32, stream: *mut c_void) -> c_int;
    pub fn dfgpt2_add_layernorm_forward(x: *const f32, y: *const f32, gamma: *const f32, beta: *const f32,
                                        sum_out: *mut f32, out: *mut f32, means: *mut f32, rstds: *mut f32,
                                        batch: u32, features: u32, stream: *mut c_void) -> c_int;
    pub fn dfgpt2_layernorm_backward_residual(grad_out: *const f32, x: *const f32, gamma: *const f32,
                                              means: *const f32, rstds: *const f32, residual: *const f32,
                                              grad_x: *mut f32, grad_gamma: *mut f32, grad_beta: *mut f32,
                                              batch: u32, features: u32, stream: *mut c_void) -> c_int;
    pub fn dfgpt2_layernorm_backward_fused_workspace_bytes(batch: u32, features: u32) -> usize;
    pub fn dfgpt2_layernorm_backward_fused(grad_out: *const f32, x: *const f32, gamma: *const f32,
                                           means: *const f32, rstds: *const f32, residual: *const f32,
                                           grad_x: *mut f32, grad_gamma: *mut f32, grad_beta: *mut f32,
                                           grad_bias: *mut f32, workspace: *mut c_void,
                                           workspace_bytes: usize, batch: u32, features: u32,
                                           stream: *mut c_void) -> c_int;
    pub fn dfgpt2_bias_gelu_forward(h: *mut f32, bias: *const f32, out: *mut f32, rows: u32, cols: u32,
                                    stream: *mut c_void) -> c_int;
}
