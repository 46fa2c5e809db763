//! Raw declarations of every entry point of `include/dfattn.h` (libdfattn), one `extern "C"` block.
//! Types follow the C header one for one: `const float *` is `*const f32`, `uint32_t` is `u32`,
//! `size_t` is `usize`, `void *stream` (a `hipStream_t`) is `*mut c_void`.
//! `tests/test_rust_crate.py` checks every declaration here against the header.

use std::os::raw::{c_char, c_int, c_void};

/// The opaque attention context of `dfattn_context_create` (`struct dfattn_context` in C).
#[repr(C)]
pub struct DfattnContext {
    _private: [u8; 0],
}

/// Status codes (`enum dfattn_status`).
pub const DFATTN_OK: c_int = 0;
pub const DFATTN_ERR_NULL_POINTER: c_int = -1;
pub const DFATTN_ERR_MISALIGNED: c_int = -2;
pub const DFATTN_ERR_SHAPE: c_int = -3;
pub const DFATTN_ERR_HEAD_DIM: c_int = -4;
pub const DFATTN_ERR_OVERFLOW: c_int = -5;
pub const DFATTN_ERR_WORKSPACE: c_int = -6;
pub const DFATTN_ERR_HIP: c_int = -7;
pub const DFATTN_ERR_FLAGS: c_int = -8;

/// `dfattn_bwd_preprocess` flag: the workspace holds the fp16 copies a `dfattn_fwd_train` left.
pub const DFATTN_BWD_QKV_SAVED: u32 = 1;
/// `dfattn_decode` cache element types.
pub const DFATTN_KV_F32: u32 = 0;
pub const DFATTN_KV_BF16: u32 = 1;
/// Bytes of the static device array `dfattn_bwd_noalloc` uses as its workspace (per GPU).
pub const DFATTN_NOALLOC_SCRATCH_BYTES: usize = 32 << 20;

#[link(name = "dfattn")]
extern "C" {
    // The reference's launchers (attention_fused.cu:223, 233, 361, 518, 617, 762, 1028, 1045, 1075, 1123, 1164, 1192,
    // 1219; matmul.cu:21): null stream, void, errors reported by `darkforest_sync`.
    pub fn launch_fused_attention(q: *const f32, k: *const f32, v: *const f32, out: *mut f32, seq_len: u32,
                                  d_head: u32, scale: f32, causal: u32);
    pub fn launch_fused_mha_forward(q: *const f32, k: *const f32, v: *const f32, out: *mut f32,
                                    n_heads: u32, seq_len: u32, d_head: u32, scale: f32, causal: u32);
    pub fn launch_attention_backward(q: *const f32, k: *const f32, v: *const f32, d_out: *const f32,
                                     d_q: *mut f32, d_k: *mut f32, d_v: *mut f32, probabilities: *mut f32,
                                     seq_len: u32, d_head: u32, scale: f32, causal: u32);
    pub fn launch_fused_mha_backward(q: *const f32, k: *const f32, v: *const f32, d_out: *const f32,
                                     d_q: *mut f32, d_k: *mut f32, d_v: *mut f32, probabilities: *mut f32,
                                     n_heads: u32, seq_len: u32, d_head: u32, scale: f32, causal: u32);
    pub fn launch_fused_mha_decode_kv(q: *const f32, k_cache: *const f32, v_cache: *const f32,
                                      out: *mut f32, n_heads: u32, cur_seq_len: u32, d_head: u32, scale: f32);
    pub fn launch_fused_mha_decode_kv_splitk(q: *const f32, k_cache: *const f32, v_cache: *const f32,
                                             partial_m: *mut f32, partial_l: *mut f32, partial_o: *mut f32,
                                             out: *mut f32, n_heads: u32, cur_seq_len: u32, d_head: u32,
                                             scale: f32, chunk_size: u32);
    pub fn launch_paged_mha_decode_kv(q: *const f32, k_pool: *const f32, v_pool: *const f32,
                                      block_table: *const i32, out: *mut f32, n_heads: u32,
                                      cur_seq_len: u32, d_head: u32, scale: f32, page_size: u32);
    pub fn launch_paged_mha_decode_kv_splitk(q: *const f32, k_pool: *const f32, v_pool: *const f32,
                                             block_table: *const i32, partial_m: *mut f32,
                                             partial_l: *mut f32, partial_o: *mut f32, out: *mut f32,
                                             n_heads: u32, cur_seq_len: u32, d_head: u32, scale: f32,
                                             page_size: u32, chunk_size: u32);
    pub fn launch_paged_mha_decode_kv_bf16(q: *const f32, k_pool: *const u16, v_pool: *const u16,
                                           block_table: *const i32, out: *mut f32, n_heads: u32,
                                           cur_seq_len: u32, d_head: u32, scale: f32, page_size: u32);
    pub fn launch_pos_embed_interpolate(pos_table: *const f32, out: *mut f32, pos: u32,
                                        trained_ctx_len: u32, max_ctx_len: u32, d_model: u32);
    pub fn launch_apply_rope(qk: *mut f32, pos: u32, n_heads: u32, d_head: u32, base_freq: f32);
    pub fn launch_paged_copy_row(src: *const f32, pool: *mut f32, phys_block: i32, page_offset: u32,
                                 page_size: u32, d_model: u32);
    pub fn launch_paged_copy_row_f32_to_bf16(src: *const f32, pool: *mut u16, phys_block: i32,
                                             page_offset: u32, page_size: u32, d_model: u32);
    pub fn darkforest_sync();

    // The fast path (no reference counterpart): explicit stream, status return.
    pub fn dfattn_fwd(q: *const f32, k: *const f32, v: *const f32, o: *mut f32, lse: *mut f32, n_heads: u32,
                      seq_len: u32, d_head: u32, scale: f32, causal: u32, stream: *mut c_void) -> c_int;
    pub fn dfattn_fwd_train(q: *const f32, k: *const f32, v: *const f32, o: *mut f32, lse: *mut f32,
                            workspace: *mut c_void, workspace_bytes: usize, n_heads: u32, seq_len: u32,
                            d_head: u32, scale: f32, causal: u32, stream: *mut c_void) -> c_int;
    pub fn dfattn_bwd_workspace_bytes(n_heads: u32, seq_len: u32, d_head: u32) -> usize;
    pub fn dfattn_bwd(q: *const f32, k: *const f32, v: *const f32, o: *const f32, d_o: *const f32,
                      lse: *const f32, d_q: *mut f32, d_k: *mut f32, d_v: *mut f32, workspace: *mut c_void,
                      workspace_bytes: usize, n_heads: u32, seq_len: u32, d_head: u32, scale: f32,
                      causal: u32, stream: *mut c_void) -> c_int;
    pub fn dfattn_bwd_preprocess(q: *const f32, k: *const f32, v: *const f32, o: *const f32,
                                 d_o: *const f32, lse: *const f32, workspace: *mut c_void,
                                 workspace_bytes: usize, n_heads: u32, seq_len: u32, d_head: u32,
                                 scale: f32, flags: u32, stream: *mut c_void) -> c_int;
    pub fn dfattn_bwd_main(q: *const f32, k: *const f32, v: *const f32, o: *const f32, d_o: *const f32,
                           lse: *const f32, d_q: *mut f32, d_k: *mut f32, d_v: *mut f32,
                           workspace: *mut c_void, workspace_bytes: usize, n_heads: u32, seq_len: u32,
                           d_head: u32, scale: f32, causal: u32, stream: *mut c_void) -> c_int;
    pub fn dfattn_fwd_train_strided(q: *const f32, k: *const f32, v: *const f32, o: *mut f32, lse: *mut f32,
                                    workspace: *mut c_void, workspace_bytes: usize, n_heads: u32,
                                    seq_len: u32, d_head: u32, scale: f32, causal: u32, qkv_row_stride: u32,
                                    stream: *mut c_void) -> c_int;
    pub fn dfattn_bwd_preprocess_strided(q: *const f32, k: *const f32, v: *const f32, o: *const f32,
                                         d_o: *const f32, lse: *const f32, workspace: *mut c_void,
                                         workspace_bytes: usize, n_heads: u32, seq_len: u32, d_head: u32,
                                         scale: f32, flags: u32, qkv_row_stride: u32, stream: *mut c_void) -> c_int;
    pub fn dfattn_bwd_main_strided(lse: *const f32, d_q: *mut f32, d_k: *mut f32, d_v: *mut f32,
                                   workspace: *mut c_void, workspace_bytes: usize, n_heads: u32,
                                   seq_len: u32, d_head: u32, scale: f32, causal: u32, grad_row_stride: u32,
                                   stream: *mut c_void) -> c_int;
    pub fn dfattn_bwd_noalloc(q: *const f32, k: *const f32, v: *const f32, o: *const f32, d_o: *const f32,
                              lse: *const f32, d_q: *mut f32, d_k: *mut f32, d_v: *mut f32, n_heads: u32,
                              seq_len: u32, d_head: u32, scale: f32, causal: u32, stream: *mut c_void) -> c_int;
    pub fn dfattn_decode_workspace_bytes(n_heads: u32, cur_seq_len: u32, d_head: u32) -> usize;
    pub fn dfattn_decode(q: *const f32, k_cache: *const c_void, v_cache: *const c_void,
                         block_table: *const i32, page_size: u32, kv_dtype: u32, out: *mut f32,
                         lse: *mut f32, n_heads: u32, cur_seq_len: u32, d_head: u32, scale: f32,
                         workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void) -> c_int;

    // The AttentionContext mirror (lib.rs:1949-2368) and its host-slice helpers (lib.rs:2371, 2421).
    pub fn dfattn_context_create(n_heads: u32, seq_len: u32, d_head: u32, out: *mut *mut DfattnContext) -> c_int;
    pub fn dfattn_context_destroy(ctx: *mut DfattnContext);
    pub fn dfattn_context_dims(ctx: *const DfattnContext, n_heads: *mut u32, seq_len: *mut u32,
                               d_head: *mut u32, d_model: *mut u32) -> c_int;
    pub fn dfattn_context_lse(ctx: *const DfattnContext) -> *const f32;
    pub fn dfattn_context_set_reuse_forward(ctx: *mut DfattnContext, enable: u32) -> c_int;
    pub fn dfattn_context_forward_device_into(ctx: *mut DfattnContext, q: *const f32, k: *const f32,
                                              v: *const f32, scale: f32, causal: u32, out: *mut f32,
                                              out_elems: usize, stream: *mut c_void) -> c_int;
    pub fn dfattn_context_backward_device_into(ctx: *mut DfattnContext, q: *const f32, k: *const f32,
                                               v: *const f32, d_out: *const f32, scale: f32, causal: u32,
                                               d_q: *mut f32, d_k: *mut f32, d_v: *mut f32,
                                               grad_elems: usize, stream: *mut c_void) -> c_int;
    pub fn dfattn_context_forward_device_into_strided(ctx: *mut DfattnContext, q: *const f32, k: *const f32,
                                                      v: *const f32, scale: f32, causal: u32, out: *mut f32,
                                                      out_elems: usize, qkv_row_stride: u32,
                                                      stream: *mut c_void) -> c_int;
    pub fn dfattn_context_backward_device_into_strided(ctx: *mut DfattnContext, q: *const f32,
                                                       k: *const f32, v: *const f32, d_out: *const f32,
                                                       scale: f32, causal: u32, d_q: *mut f32,
                                                       d_k: *mut f32, d_v: *mut f32, grad_elems: usize,
                                                       qkv_row_stride: u32, grad_row_stride: u32,
                                                       stream: *mut c_void) -> c_int;
    pub fn dfattn_context_forward(ctx: *mut DfattnContext, q: *const f32, k: *const f32, v: *const f32,
                                  len: usize, scale: f32, causal: u32, out: *mut f32) -> c_int;
    pub fn dfattn_context_backward(ctx: *mut DfattnContext, d_out: *const f32, len: usize, scale: f32,
                                   causal: u32, d_q: *mut f32, d_k: *mut f32, d_v: *mut f32) -> c_int;
    pub fn dfattn_fused_attention_forward(q: *const f32, k: *const f32, v: *const f32, len: usize,
                                          seq_len: u32, d_head: u32, scale: f32, causal: u32, out: *mut f32) -> c_int;
    pub fn dfattn_attention_backward(q: *const f32, k: *const f32, v: *const f32, d_out: *const f32,
                                     len: usize, seq_len: u32, d_head: u32, scale: f32, causal: u32,
                                     d_q: *mut f32, d_k: *mut f32, d_v: *mut f32) -> c_int;

    // Status and version.
    pub fn dfattn_status_string(status: c_int) -> *const c_char;
    pub fn dfattn_last_error() -> c_int;
    pub fn dfattn_last_error_message() -> *const c_char;
    pub fn dfattn_clear_error();
    pub fn dfattn_version() -> *const c_char;
}
