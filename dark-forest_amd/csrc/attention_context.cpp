// attention_context.cpp — host-side mirror of the reference's AttentionContext
// (darkforest-cuda/src/lib.rs:1949-2368) and of its host-slice helpers
// fused_attention_forward / attention_backward (lib.rs:2371, 2421), on top of
// the fast-path entry points of include/dfattn.h.
//
// Differences from the reference, all deliberate:
//  * Every buffer the context needs is allocated at construction (logsumexp
//    [H, S] and the backward workspace, O(H*S) and O(H*S*D)); the reference allocates
//    an H*2*S*S probability scratch on the first backward (lib.rs:2019-2027).
//  * backward_device_into recomputes the forward from the current contents of
//    q, k, v (as the reference's does, lib.rs:2240-2293) into context-owned
//    buffers. A caller that keeps a layer's Q, K, V and O untouched between
//    the two calls, as the reference's static engine does
//    (static_gpt2.rs:1329-1336, 1500-1510), may opt in to reusing the last
//    forward_device_into's O, logsumexp and fp16 operand copies instead
//    (dfattn_context_set_reuse_forward); reuse then also needs the same q, k,
//    v pointers, scale and causal flag.
//  * Errors are status codes (dfattn_status) instead of anyhow::Result.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "dfattn.h"
#include "dfattn_status.h"

struct dfattn_context {
  uint32_t n_heads = 0, seq_len = 0, d_head = 0, d_model = 0;
  size_t elems = 0;           // seq_len * d_model
  float *lse = nullptr;       // [n_heads, seq_len], written by every forward
  void *workspace = nullptr;  // dfattn_bwd_workspace_bytes()
  size_t workspace_bytes = 0;
  // Last forward_device_into: its inputs and output (O stays the caller's).
  const float *last_q = nullptr, *last_k = nullptr, *last_v = nullptr;
  const float *last_out = nullptr;
  float last_scale = 0.f;
  uint32_t last_causal = 0;
  uint32_t last_qkv_stride = 0;  // 0: contiguous
  // Opt-in: the backward may reuse the last forward (caller guarantees that
  // q, k, v and that forward's out are unchanged and still allocated).
  bool reuse_forward = false;
  // Context-owned O, allocated on first need (a backward without a matching
  // forward, or the host-slice forward).
  float *own_out = nullptr;
  // Host-slice path buffers (lib.rs:1954-1961), allocated on first use.
  float *q = nullptr, *k = nullptr, *v = nullptr, *d_out = nullptr;
  float *d_q = nullptr, *d_k = nullptr, *d_v = nullptr;
  bool host_forward_done = false;
  std::mutex mu;  // the reference guards its buffers with Mutexes
};

namespace {

int hip_status(hipError_t e) {
  if (e == hipSuccess) return DFATTN_OK;
  return dfattn::record_error(DFATTN_ERR_HIP, std::string("attention context: ") + hipGetErrorString(e));
}

int fail(int status, const char *msg) { return dfattn::record_error(status, msg); }

int ensure(float **p, size_t elems) {
  if (*p != nullptr) return DFATTN_OK;
  return hip_status(hipMalloc(reinterpret_cast<void **>(p), elems * sizeof(float)));
}

// The shape checks of AttentionContext::new_shared (lib.rs:1981-1989).
int check_dims(uint32_t n_heads, uint32_t seq_len, uint32_t d_head) {
  if (d_head == 0 || d_head > 128) return fail(DFATTN_ERR_HEAD_DIM, "d_head must be in the range 1..=128");
  if (n_heads == 0 || seq_len == 0) return fail(DFATTN_ERR_SHAPE, "n_heads and seq_len must be >= 1");
  size_t dm = 0, e = 0, b = 0;
  if (__builtin_mul_overflow((size_t)n_heads, (size_t)d_head, &dm))
    return fail(DFATTN_ERR_OVERFLOW, "d_model overflow");
  if (n_heads > 65535 || seq_len > (1u << 30))  // the attention entry points' limits
    return fail(DFATTN_ERR_OVERFLOW, "attention shape is too large");
  if (__builtin_mul_overflow((size_t)seq_len, dm, &e) || __builtin_mul_overflow(e, sizeof(float), &b))
    return fail(DFATTN_ERR_OVERFLOW, "attention shape is too large");
  return DFATTN_OK;
}

// A row stride of exactly n_heads * d_head is the contiguous layout: 0, so that
// a forward and a backward that name it differently still match for reuse.
uint32_t packed_or(const dfattn_context *c, uint32_t stride) {
  return stride == c->n_heads * c->d_head ? 0 : stride;
}

// The forward also leaves the backward's fp16 copies of Q, K and V in the
// context's workspace (dfattn_fwd_train), which the backward on the same
// q, k, v then reuses. qkv_stride: the row stride of q, k, v (0: contiguous).
int run_forward(dfattn_context *c, const float *q, const float *k, const float *v, float scale,
                uint32_t causal, float *out, uint32_t qkv_stride, void *stream) {
  const int st = qkv_stride == 0
                     ? dfattn_fwd_train(q, k, v, out, c->lse, c->workspace, c->workspace_bytes, c->n_heads,
                                        c->seq_len, c->d_head, scale, causal, stream)
                     : dfattn_fwd_train_strided(q, k, v, out, c->lse, c->workspace, c->workspace_bytes,
                                                c->n_heads, c->seq_len, c->d_head, scale, causal, qkv_stride,
                                                stream);
  if (st == DFATTN_OK) {
    c->last_qkv_stride = qkv_stride;
    c->last_q = q;
    c->last_k = k;
    c->last_v = v;
    c->last_out = out;
    c->last_scale = scale;
    c->last_causal = causal;
  }
  return st;
}

// qkv_stride / grad_stride: the row strides of q, k, v and of d_q, d_k, d_v
// (0: contiguous).
int run_backward(dfattn_context *c, const float *q, const float *k, const float *v,
                 const float *d_out, float scale, uint32_t causal, float *d_q, float *d_k,
                 float *d_v, uint32_t qkv_stride, uint32_t grad_stride, void *stream) {
  const float *o = c->last_out;
  if (!(c->reuse_forward && q == c->last_q && k == c->last_k && v == c->last_v && o != nullptr &&
        scale == c->last_scale && causal == c->last_causal && qkv_stride == c->last_qkv_stride)) {
    int st = ensure(&c->own_out, c->elems);
    if (st != DFATTN_OK) return st;
    st = run_forward(c, q, k, v, scale, causal, c->own_out, qkv_stride, stream);
    if (st != DFATTN_OK) return st;
    o = c->own_out;
  }
  // The forward left the fp16 copies: preprocess reads only o, d_out and
  // lse, so q, k, v pass as they are whatever their stride.
  const int st = dfattn_bwd_preprocess(q, k, v, o, d_out, c->lse, c->workspace, c->workspace_bytes,
                                       c->n_heads, c->seq_len, c->d_head, scale, DFATTN_BWD_QKV_SAVED, stream);
  if (st != DFATTN_OK) return st;
  if (grad_stride != 0)
    return dfattn_bwd_main_strided(c->lse, d_q, d_k, d_v, c->workspace, c->workspace_bytes, c->n_heads,
                                   c->seq_len, c->d_head, scale, causal, grad_stride, stream);
  return dfattn_bwd_main(q, k, v, o, d_out, c->lse, d_q, d_k, d_v, c->workspace, c->workspace_bytes,
                         c->n_heads, c->seq_len, c->d_head, scale, causal, stream);
}

void free_all(dfattn_context *c) {
  float *bufs[] = {c->lse, c->own_out, c->q, c->k, c->v, c->d_out, c->d_q, c->d_k, c->d_v};
  for (float *p : bufs)
    if (p != nullptr) (void)hipFree(p);
  if (c->workspace != nullptr) (void)hipFree(c->workspace);
}

int upload(float *dst, const float *src, size_t elems) {
  return hip_status(hipMemcpy(dst, src, elems * sizeof(float), hipMemcpyHostToDevice));
}

int download(float *dst, const float *src, size_t elems) {
  return hip_status(hipMemcpy(dst, src, elems * sizeof(float), hipMemcpyDeviceToHost));
}

}  // namespace

extern "C" {

int dfattn_context_create(uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
                          dfattn_context **out) {
  if (out == nullptr) return fail(DFATTN_ERR_NULL_POINTER, "null context out-pointer");
  *out = nullptr;
  int st = check_dims(n_heads, seq_len, d_head);
  if (st != DFATTN_OK) return st;
  dfattn_context *c = new (std::nothrow) dfattn_context;
  if (c == nullptr) return fail(DFATTN_ERR_HIP, "out of host memory");
  c->n_heads = n_heads;
  c->seq_len = seq_len;
  c->d_head = d_head;
  c->d_model = n_heads * d_head;
  c->elems = (size_t)seq_len * c->d_model;
  c->workspace_bytes = dfattn_bwd_workspace_bytes(n_heads, seq_len, d_head);
  st = ensure(&c->lse, (size_t)n_heads * seq_len);
  if (st == DFATTN_OK) st = hip_status(hipMalloc(&c->workspace, c->workspace_bytes));
  if (st != DFATTN_OK) {
    free_all(c);
    delete c;
    return st;
  }
  *out = c;
  return DFATTN_OK;
}

void dfattn_context_destroy(dfattn_context *c) {
  if (c == nullptr) return;
  free_all(c);
  delete c;
}

int dfattn_context_dims(const dfattn_context *c, uint32_t *n_heads, uint32_t *seq_len,
                        uint32_t *d_head, uint32_t *d_model) {
  if (c == nullptr) return fail(DFATTN_ERR_NULL_POINTER, "null attention context");
  if (n_heads) *n_heads = c->n_heads;
  if (seq_len) *seq_len = c->seq_len;
  if (d_head) *d_head = c->d_head;
  if (d_model) *d_model = c->d_model;
  return DFATTN_OK;
}

const float *dfattn_context_lse(const dfattn_context *c) { return c ? c->lse : nullptr; }

int dfattn_context_set_reuse_forward(dfattn_context *c, uint32_t enable) {
  if (c == nullptr) return fail(DFATTN_ERR_NULL_POINTER, "null attention context");
  std::lock_guard<std::mutex> lock(c->mu);
  c->reuse_forward = enable != 0;
  return DFATTN_OK;
}

int dfattn_context_forward_device_into(dfattn_context *c, const float *q, const float *k,
                                       const float *v, float scale, uint32_t causal, float *out,
                                       size_t out_elems, void *stream) {
  if (c == nullptr) return fail(DFATTN_ERR_NULL_POINTER, "null attention context");
  if (out_elems != c->elems) return fail(DFATTN_ERR_SHAPE, "attention output shape mismatch");
  std::lock_guard<std::mutex> lock(c->mu);
  return run_forward(c, q, k, v, scale, causal, out, 0, stream);
}

int dfattn_context_forward_device_into_strided(dfattn_context *c, const float *q, const float *k,
                                               const float *v, float scale, uint32_t causal, float *out,
                                               size_t out_elems, uint32_t qkv_row_stride, void *stream) {
  if (c == nullptr) return fail(DFATTN_ERR_NULL_POINTER, "null attention context");
  if (out_elems != c->elems) return fail(DFATTN_ERR_SHAPE, "attention output shape mismatch");
  if (qkv_row_stride == 0) return fail(DFATTN_ERR_SHAPE, "row stride must be >= n_heads*d_head");
  std::lock_guard<std::mutex> lock(c->mu);
  return run_forward(c, q, k, v, scale, causal, out, packed_or(c, qkv_row_stride), stream);
}

int dfattn_context_backward_device_into(dfattn_context *c, const float *q, const float *k,
                                        const float *v, const float *d_out, float scale,
                                        uint32_t causal, float *d_q, float *d_k, float *d_v,
                                        size_t grad_elems, void *stream) {
  if (c == nullptr) return fail(DFATTN_ERR_NULL_POINTER, "null attention context");
  if (grad_elems != c->elems) return fail(DFATTN_ERR_SHAPE, "attention backward output shape mismatch");
  std::lock_guard<std::mutex> lock(c->mu);
  return run_backward(c, q, k, v, d_out, scale, causal, d_q, d_k, d_v, 0, 0, stream);
}

int dfattn_context_backward_device_into_strided(dfattn_context *c, const float *q, const float *k,
                                                const float *v, const float *d_out, float scale,
                                                uint32_t causal, float *d_q, float *d_k, float *d_v,
                                                size_t grad_elems, uint32_t qkv_row_stride,
                                                uint32_t grad_row_stride, void *stream) {
  if (c == nullptr) return fail(DFATTN_ERR_NULL_POINTER, "null attention context");
  if (grad_elems != c->elems) return fail(DFATTN_ERR_SHAPE, "attention backward output shape mismatch");
  if (qkv_row_stride == 0 || grad_row_stride == 0)
    return fail(DFATTN_ERR_SHAPE, "row strides must be >= n_heads*d_head");
  std::lock_guard<std::mutex> lock(c->mu);
  return run_backward(c, q, k, v, d_out, scale, causal, d_q, d_k, d_v, packed_or(c, qkv_row_stride),
                      packed_or(c, grad_row_stride), stream);
}

// lib.rs:2295-2326: upload q, k, v into context buffers, run the single-head
// launcher on [seq_len, d_head], download O. Like the reference, these two
// host-slice methods treat the data as one head of d_head columns.
int dfattn_context_forward(dfattn_context *c, const float *q, const float *k, const float *v,
                           size_t len, float scale, uint32_t causal, float *out) {
  if (c == nullptr || q == nullptr || k == nullptr || v == nullptr || out == nullptr)
    return fail(DFATTN_ERR_NULL_POINTER, "null argument");
  const size_t n = (size_t)c->seq_len * c->d_head;
  if (len != n) return fail(DFATTN_ERR_SHAPE, "q, k, and v must each have shape [seq_len, d_head]");
  std::lock_guard<std::mutex> lock(c->mu);
  int st = DFATTN_OK;
  for (float **p : {&c->q, &c->k, &c->v, &c->own_out})
    if (st == DFATTN_OK) st = ensure(p, c->elems);
  if (st == DFATTN_OK) st = upload(c->q, q, n);
  if (st == DFATTN_OK) st = upload(c->k, k, n);
  if (st == DFATTN_OK) st = upload(c->v, v, n);
  if (st == DFATTN_OK)
    st = dfattn_fwd(c->q, c->k, c->v, c->own_out, c->lse, 1, c->seq_len, c->d_head, scale, causal,
                    nullptr);
  if (st == DFATTN_OK) st = download(out, c->own_out, n);
  c->host_forward_done = st == DFATTN_OK;
  c->last_q = c->last_k = c->last_v = c->last_out = nullptr;  // not a device-path forward
  return st;
}

// lib.rs:2328-2367: the backward of the last host-slice forward's q, k, v.
int dfattn_context_backward(dfattn_context *c, const float *d_out, size_t len, float scale,
                            uint32_t causal, float *d_q, float *d_k, float *d_v) {
  if (c == nullptr || d_out == nullptr || d_q == nullptr || d_k == nullptr || d_v == nullptr)
    return fail(DFATTN_ERR_NULL_POINTER, "null argument");
  const size_t n = (size_t)c->seq_len * c->d_head;
  if (len != n) return fail(DFATTN_ERR_SHAPE, "d_out must have shape [seq_len, d_head]");
  std::lock_guard<std::mutex> lock(c->mu);
  if (!c->host_forward_done)
    return fail(DFATTN_ERR_SHAPE, "backward before any host-slice forward: q, k, v were never uploaded");
  int st = DFATTN_OK;
  for (float **p : {&c->d_out, &c->d_q, &c->d_k, &c->d_v})
    if (st == DFATTN_OK) st = ensure(p, c->elems);
  if (st == DFATTN_OK) st = upload(c->d_out, d_out, n);
  // Recompute O and lse for this scale/causal (the host forward may have used others).
  if (st == DFATTN_OK)
    st = dfattn_fwd(c->q, c->k, c->v, c->own_out, c->lse, 1, c->seq_len, c->d_head, scale, causal,
                    nullptr);
  if (st == DFATTN_OK)
    st = dfattn_bwd(c->q, c->k, c->v, c->own_out, c->d_out, c->lse, c->d_q, c->d_k, c->d_v,
                    c->workspace, c->workspace_bytes, 1, c->seq_len, c->d_head, scale, causal,
                    nullptr);
  if (st == DFATTN_OK) st = download(d_q, c->d_q, n);
  if (st == DFATTN_OK) st = download(d_k, c->d_k, n);
  if (st == DFATTN_OK) st = download(d_v, c->d_v, n);
  return st;
}

// lib.rs:2370-2418: allocate, upload, single-head forward, download.
int dfattn_fused_attention_forward(const float *q, const float *k, const float *v, size_t len,
                                   uint32_t seq_len, uint32_t d_head, float scale, uint32_t causal,
                                   float *out) {
  if (d_head == 0 || d_head > 128) return fail(DFATTN_ERR_HEAD_DIM, "d_head must be in the range 1..=128");
  size_t expected = 0;
  if (__builtin_mul_overflow((size_t)seq_len, (size_t)d_head, &expected))
    return fail(DFATTN_ERR_OVERFLOW, "attention shape is too large");
  if (len != expected) return fail(DFATTN_ERR_SHAPE, "q, k, and v must each have shape [seq_len, d_head]");
  dfattn_context *c = nullptr;
  int st = dfattn_context_create(1, seq_len, d_head, &c);
  if (st == DFATTN_OK) st = dfattn_context_forward(c, q, k, v, len, scale, causal, out);
  dfattn_context_destroy(c);
  return st;
}

// lib.rs:2420-2479: allocate, upload, single-head backward, download.
int dfattn_attention_backward(const float *q, const float *k, const float *v, const float *d_out,
                              size_t len, uint32_t seq_len, uint32_t d_head, float scale,
                              uint32_t causal, float *d_q, float *d_k, float *d_v) {
  if (d_head == 0 || d_head > 128) return fail(DFATTN_ERR_HEAD_DIM, "d_head must be in the range 1..=128");
  size_t expected = 0;
  if (__builtin_mul_overflow((size_t)seq_len, (size_t)d_head, &expected))
    return fail(DFATTN_ERR_OVERFLOW, "attention shape is too large");
  if (len != expected)
    return fail(DFATTN_ERR_SHAPE, "q, k, v, and d_out must each have shape [seq_len, d_head]");
  dfattn_context *c = nullptr;
  int st = dfattn_context_create(1, seq_len, d_head, &c);
  if (st != DFATTN_OK) return st;
  std::vector<float> o(expected);
  st = dfattn_context_forward(c, q, k, v, len, scale, causal, o.data());
  if (st == DFATTN_OK) st = dfattn_context_backward(c, d_out, len, scale, causal, d_q, d_k, d_v);
  dfattn_context_destroy(c);
  return st;
}

}  // extern "C"
