// dfattn_api.hip — the C ABI of include/dfattn.h: argument validation,
// kernel selection, the reference's launcher symbols and the error state.
//
// Kernel selection: d_head == 64 with 16-byte aligned tensors takes the MFMA
// kernels (attn_fwd_d64.hip, attn_bwd_d64.hip); every other valid shape takes
// the exact fp32 kernels in attn_generic.hip. There is no CPU path.
#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>

#include "dfattn.h"
#include "dfattn_internal.h"
#include "dfattn_status.h"

namespace {
std::mutex g_err_mu;
int g_err = DFATTN_OK;  // last error of any entry point (dfattn_last_error)
std::string g_err_msg;
// First error of a reference launcher symbol (void return, no other way to
// report) since the last darkforest_sync, which aborts on it.
int g_pending = DFATTN_OK;
std::string g_pending_msg;

void mark_pending_if_failed(int status) {
  if (status == DFATTN_OK) return;
  std::lock_guard<std::mutex> lock(g_err_mu);
  if (g_pending == DFATTN_OK) {
    g_pending = status;
    g_pending_msg = g_err_msg;
  }
}
}  // namespace

int dfattn::record_error(int status, const std::string &msg) {
  std::lock_guard<std::mutex> lock(g_err_mu);
  g_err = status;
  g_err_msg = msg;
  return status;
}

void dfattn::mark_pending(int status) { mark_pending_if_failed(status); }

namespace {
using dfattn::record_error;

int record_hip(hipError_t err, const char *where) {
  if (err == hipSuccess) return DFATTN_OK;
  return record_error(DFATTN_ERR_HIP, std::string(where) + ": " + hipGetErrorString(err));
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Shape checks shared by every entry point (the reference's are in
// AttentionContext::new_shared, darkforest-cuda/src/lib.rs:1981-1989).
// Launch grids keep one head per row of a 2-D grid, whose second dimension
// holds at most 65535 blocks (the reference's grids, attention_fused.cu:239,
// have the same bound); this also keeps every offset of a 128-row tile of the
// [S, H*64] inputs inside 31 bits.
constexpr uint32_t kMaxHeads = 65535;

int check_shape(const char *fn, uint32_t n_heads, uint32_t seq_len, uint32_t d_head) {
  if (n_heads == 0 || seq_len == 0)
    return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": n_heads and seq_len must be >= 1");
  if (d_head == 0 || d_head > 128)
    return record_error(DFATTN_ERR_HEAD_DIM, std::string(fn) + ": d_head must be in the range 1..=128");
  size_t dm = 0, elems = 0, bytes = 0;
  if (__builtin_mul_overflow((size_t)n_heads, (size_t)d_head, &dm) ||
      __builtin_mul_overflow((size_t)seq_len, dm, &elems) ||
      __builtin_mul_overflow(elems, sizeof(float), &bytes) || seq_len > (1u << 30) ||
      n_heads > kMaxHeads)
    return record_error(DFATTN_ERR_OVERFLOW, std::string(fn) + ": attention shape is too large");
  return DFATTN_OK;
}

int check_ptrs(const char *fn, std::initializer_list<const void *> ptrs) {
  for (const void *p : ptrs) {
    if (p == nullptr)
      return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null tensor pointer");
    if (!aligned(p, alignof(float)))
      return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": tensor pointer not 4-byte aligned");
  }
  return DFATTN_OK;
}

bool fast_path(uint32_t d_head, std::initializer_list<const void *> ptrs) {
  if (d_head != 64) return false;
  for (const void *p : ptrs)
    if (p != nullptr && !aligned(p, 16)) return false;
  return true;
}

int fwd_impl(const float *q, const float *k, const float *v, float *o, float *lse,
             uint32_t n_heads, uint32_t seq_len, uint32_t d_head, float scale, uint32_t causal,
             hipStream_t stream) {
  hipError_t err;
  if (fast_path(d_head, {q, k, v, o, lse}))
    err = dfattn::launch_fwd_d64(q, k, v, o, lse, (int)n_heads, (int)seq_len, scale, causal != 0,
                                 stream);
  else
    err = dfattn::launch_fwd_generic(q, k, v, o, lse, (int)n_heads, (int)seq_len, (int)d_head,
                                     scale, causal != 0, stream);
  return record_hip(err, "attention forward launch");
}

// Legacy backward: the caller's probability scratch (`capacity` floats) holds
// O, lse and the fast path's workspace when it is large enough; otherwise the
// self-contained generic kernel runs.
int legacy_backward(const char *fn, const float *q, const float *k, const float *v,
                    const float *d_out, float *d_q, float *d_k, float *d_v, float *scratch,
                    size_t capacity, uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
                    float scale, uint32_t causal) {
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, d_out, d_q, d_k, d_v});
  if (st != DFATTN_OK) return st;
  const size_t elems = (size_t)seq_len * n_heads * d_head;
  const size_t lse_floats = ((size_t)n_heads * seq_len + 63) / 64 * 64;
  const size_t ws_floats = dfattn::bwd_workspace_bytes_d64((int)n_heads, (int)seq_len) / sizeof(float);
  const bool fits = scratch != nullptr && elems + lse_floats + ws_floats <= capacity;
  hipError_t err;
  if (fits && fast_path(d_head, {q, k, v, d_out, d_q, d_k, d_v, scratch})) {
    float *o_ws = scratch;
    float *lse_ws = scratch + elems;
    float *bwd_ws = lse_ws + lse_floats;
    err = dfattn::launch_fwd_d64(q, k, v, o_ws, lse_ws, (int)n_heads, (int)seq_len, scale,
                                 causal != 0, nullptr);
    if (err == hipSuccess)
      err = dfattn::launch_bwd_d64(q, k, v, o_ws, d_out, lse_ws, d_q, d_k, d_v, bwd_ws,
                                   (int)n_heads, (int)seq_len, scale, causal != 0, nullptr);
  } else {
    err = dfattn::launch_bwd_generic(q, k, v, d_out, d_q, d_k, d_v, (int)n_heads, (int)seq_len,
                                     (int)d_head, scale, causal != 0, nullptr);
  }
  return record_hip(err, fn);
}

// ---- decode --------------------------------------------------------------

// Chunks of the fast decode: enough workgroups to fill the GPU (about 512),
// at least 512 keys each (one 64-key group per wave); up to 1024 keys the
// second launch costs more than one workgroup per head takes.
constexpr uint32_t kDecodeMinChunk = 512;
uint32_t decode_chunks(uint32_t n_heads, uint32_t cur_len) {
  if (cur_len <= 1024) return 1;
  const uint32_t by_len = (cur_len + kDecodeMinChunk - 1) / kDecodeMinChunk;
  const uint32_t by_grid = (512 + n_heads - 1) / n_heads;
  return std::max(1u, std::min(by_len, by_grid));
}
uint32_t decode_chunk_len(uint32_t cur_len, uint32_t n_chunks) {
  const uint32_t c = (cur_len + n_chunks - 1) / n_chunks;
  return (c + 63) / 64 * 64;
}

// Shared validation of every decode entry point; `table` is checked when
// `paged`. cur_len == 0 is valid (nothing is computed, as in the reference).
int check_decode(const char *fn, const float *q, const void *k, const void *v, const int32_t *table,
                 bool paged, uint32_t page_size, bool bf16, const float *out, uint32_t n_heads,
                 uint32_t cur_len, uint32_t d_head) {
  if (n_heads == 0) return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": n_heads must be >= 1");
  if (d_head == 0 || d_head > 128)
    return record_error(DFATTN_ERR_HEAD_DIM, std::string(fn) + ": d_head must be in the range 1..=128");
  if (n_heads > kMaxHeads || cur_len > (1u << 30))
    return record_error(DFATTN_ERR_OVERFLOW, std::string(fn) + ": decode shape is too large");
  if (paged && page_size == 0)
    return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": page_size must be >= 1");
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || (paged && table == nullptr))
    return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null pointer");
  const size_t kv_align = bf16 ? 2 : 4;
  if (!aligned(q, 4) || !aligned(out, 4) || !aligned(k, kv_align) || !aligned(v, kv_align) ||
      (paged && !aligned(table, 4)))
    return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": misaligned pointer");
  return DFATTN_OK;
}

bool decode_fast(uint32_t d_head, bool bf16, const float *q, const void *k, const void *v) {
  const size_t kv_align = bf16 ? 8 : 16;
  return d_head == 64 && aligned(q, 16) && aligned(k, kv_align) && aligned(v, kv_align);
}

// The reference's decode launchers: null stream, errors recorded for
// darkforest_sync. chunk 0 = no split.
int legacy_decode(const char *fn, const float *q, const void *k, const void *v, const int32_t *table,
                  bool paged, uint32_t page_size, bool bf16, float *pm, float *pl, float *po, float *out,
                  uint32_t n_heads, uint32_t cur_len, uint32_t d_head, float scale, uint32_t chunk,
                  bool splitk) {
  int st = check_decode(fn, q, k, v, table, paged, page_size, bf16, out, n_heads, cur_len, d_head);
  if (st != DFATTN_OK) return st;
  if (splitk && chunk == 0) return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": chunk_size must be >= 1");
  if (cur_len == 0) return DFATTN_OK;
  // attention_fused.cu:781-784: no split when the keys fit one chunk.
  const bool split = splitk && cur_len > chunk;
  if (split && (pm == nullptr || pl == nullptr || po == nullptr))
    return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null partial buffer");
  const hipError_t err = dfattn::launch_decode(
      q, k, v, paged ? table : nullptr, (int)page_size, bf16, out, nullptr, (int)n_heads, (int)cur_len,
      (int)d_head, scale, split ? (int)chunk : (int)cur_len, split ? pm : nullptr, split ? pl : nullptr,
      split ? po : nullptr, decode_fast(d_head, bf16, q, k, v), nullptr);
  return record_hip(err, fn);
}

// ---- the elementwise companions (attention_fused.cu:1123-1231) -------------

int pos_embed_impl(const float *table, float *out, uint32_t pos, uint32_t trained, uint32_t max_ctx,
                   uint32_t d_model) {
  const char *fn = "launch_pos_embed_interpolate";
  if (table == nullptr || out == nullptr)
    return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null pointer");
  if (!aligned(table, 4) || !aligned(out, 4))
    return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": misaligned pointer");
  // The reference reads row trained - 1 = 2^32 - 1 of the table then.
  if (trained == 0) return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": trained_ctx_len must be >= 1");
  if (d_model == 0) return DFATTN_OK;
  return record_hip(dfattn::launch_pos_embed_interpolate(table, out, pos, trained, max_ctx, d_model, nullptr), fn);
}

int rope_impl(float *qk, uint32_t pos, uint32_t n_heads, uint32_t d_head, float base) {
  const char *fn = "launch_apply_rope";
  if (qk == nullptr) return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null pointer");
  if (!aligned(qk, 4)) return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": misaligned pointer");
  // The reference's launch (grid n_heads, block d_head / 2) is invalid for these.
  if (n_heads == 0) return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": n_heads must be >= 1");
  if (d_head < 2) return record_error(DFATTN_ERR_HEAD_DIM, std::string(fn) + ": d_head must be >= 2");
  if ((uint64_t)n_heads * d_head > (1ull << 32))
    return record_error(DFATTN_ERR_OVERFLOW, std::string(fn) + ": n_heads * d_head is too large");
  return record_hip(dfattn::launch_apply_rope(qk, pos, n_heads, d_head, base, nullptr), fn);
}

int paged_copy_impl(const char *fn, const float *src, void *pool, bool bf16, int32_t phys_block,
                    uint32_t page_offset, uint32_t page_size, uint32_t d_model) {
  if (src == nullptr || pool == nullptr)
    return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null pointer");
  if (!aligned(src, 4) || !aligned(pool, bf16 ? 2 : 4))
    return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": misaligned pointer");
  // The reference's caller (paged_kv.rs:206-209) always passes a block from
  // the pool's allocator and page_offset = pos % page_size.
  if (phys_block < 0) return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": phys_block must be >= 0");
  if (page_offset >= page_size)
    return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": page_offset must be < page_size");
  if (d_model == 0) return DFATTN_OK;
  return record_hip(
      dfattn::launch_paged_copy_row(src, pool, bf16, phys_block, page_offset, page_size, d_model, nullptr), fn);
}

}  // namespace

extern "C" {

// ---- reference launcher symbols ------------------------------------------

void launch_fused_attention(const float *q, const float *k, const float *v, float *out,
                            uint32_t seq_len, uint32_t d_head, float scale, uint32_t causal) {
  const char *fn = "launch_fused_attention";
  int st = check_shape(fn, 1, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, out});
  if (st == DFATTN_OK) st = fwd_impl(q, k, v, out, nullptr, 1, seq_len, d_head, scale, causal, nullptr);
  mark_pending_if_failed(st);
}

void launch_fused_mha_forward(const float *q, const float *k, const float *v, float *out,
                              uint32_t n_heads, uint32_t seq_len, uint32_t d_head, float scale,
                              uint32_t causal) {
  const char *fn = "launch_fused_mha_forward";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, out});
  if (st == DFATTN_OK)
    st = fwd_impl(q, k, v, out, nullptr, n_heads, seq_len, d_head, scale, causal, nullptr);
  mark_pending_if_failed(st);
}

void launch_attention_backward(const float *q, const float *k, const float *v,
                               const float *d_out, float *d_q, float *d_k, float *d_v,
                               float *probabilities, uint32_t seq_len, uint32_t d_head,
                               float scale, uint32_t causal) {
  // Scratch is [seq_len, seq_len] (lib.rs:2441).
  mark_pending_if_failed(legacy_backward("launch_attention_backward", q, k, v, d_out, d_q, d_k,
                                         d_v, probabilities, (size_t)seq_len * seq_len, 1,
                                         seq_len, d_head, scale, causal));
}

void launch_fused_mha_backward(const float *q, const float *k, const float *v,
                               const float *d_out, float *d_q, float *d_k, float *d_v,
                               float *probabilities, uint32_t n_heads, uint32_t seq_len,
                               uint32_t d_head, float scale, uint32_t causal) {
  // Scratch is [n_heads, 2, seq_len, seq_len] (lib.rs:2023).
  mark_pending_if_failed(legacy_backward("launch_fused_mha_backward", q, k, v, d_out, d_q, d_k,
                                         d_v, probabilities,
                                         (size_t)n_heads * 2 * seq_len * seq_len, n_heads, seq_len,
                                         d_head, scale, causal));
}

void darkforest_sync(void) {
  // A recorded launcher error aborts before any HIP call: nothing was
  // launched for it, so there is no device work to wait for first.
  {
    std::lock_guard<std::mutex> lock(g_err_mu);
    if (g_pending != DFATTN_OK) {
      fprintf(stderr, "[darkforest] attention launch error before sync boundary: %s\n",
              g_pending_msg.c_str());
      abort();
    }
  }
  hipError_t err = hipDeviceSynchronize();
  if (err != hipSuccess) {
    fprintf(stderr, "[darkforest] HIP kernel error at sync boundary: %s\n", hipGetErrorString(err));
    abort();
  }
}

// ---- fast path -------------------------------------------------------------

int dfattn_fwd(const float *q, const float *k, const float *v, float *o, float *lse,
               uint32_t n_heads, uint32_t seq_len, uint32_t d_head, float scale, uint32_t causal,
               void *stream) {
  const char *fn = "dfattn_fwd";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, o});
  if (st == DFATTN_OK && lse != nullptr) st = check_ptrs(fn, {lse});
  if (st != DFATTN_OK) return st;
  return fwd_impl(q, k, v, o, lse, n_heads, seq_len, d_head, scale, causal,
                  static_cast<hipStream_t>(stream));
}

size_t dfattn_bwd_workspace_bytes(uint32_t n_heads, uint32_t seq_len, uint32_t d_head) {
  if (n_heads == 0 || seq_len == 0 || d_head == 0 || d_head > 128 || seq_len > (1u << 30) ||
      n_heads > kMaxHeads)
    return 0;
  return dfattn::bwd_workspace_bytes_d64((int)n_heads, (int)seq_len);
}

namespace {
static int check_workspace(const char *fn, const void *workspace, size_t workspace_bytes,
                           uint32_t n_heads, uint32_t seq_len, uint32_t d_head) {
  const size_t need = dfattn_bwd_workspace_bytes(n_heads, seq_len, d_head);
  if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, alignof(float)))
    return record_error(DFATTN_ERR_WORKSPACE,
                        std::string(fn) + ": workspace must be non-null, 4-byte aligned and hold " +
                            std::to_string(need) + " bytes");
  return DFATTN_OK;
}

// The strided entry points run the d_head = 64 kernels only: 16-byte aligned
// tensors and a row stride that is at least the row's own n_heads * 64
// values, a multiple of 4 floats (16-byte rows) and at most 2^21 (the
// kernels' 32-bit tile offsets).
static int check_strided(const char *fn, uint32_t d_head, uint32_t n_heads, uint32_t stride,
                         std::initializer_list<const void *> ptrs) {
  if (d_head != 64)
    return record_error(DFATTN_ERR_HEAD_DIM, std::string(fn) + ": the strided entry points need d_head 64");
  if (stride < n_heads * d_head || stride % 4 != 0 || stride > (1u << 21))
    return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": row stride must be >= n_heads*d_head, a multiple "
                                                            "of 4 and at most 2^21");
  if (!fast_path(d_head, ptrs))
    return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": tensors must be 16-byte aligned");
  return DFATTN_OK;
}
}  // namespace

int dfattn_bwd(const float *q, const float *k, const float *v, const float *o, const float *d_o,
               const float *lse, float *d_q, float *d_k, float *d_v, void *workspace,
               size_t workspace_bytes, uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
               float scale, uint32_t causal, void *stream) {
  const char *fn = "dfattn_bwd";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, o, d_o, lse, d_q, d_k, d_v});
  if (st == DFATTN_OK) st = check_workspace(fn, workspace, workspace_bytes, n_heads, seq_len, d_head);
  if (st != DFATTN_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  if (fast_path(d_head, {q, k, v, o, d_o, lse, d_q, d_k, d_v}))
    err = dfattn::launch_bwd_d64(q, k, v, o, d_o, lse, d_q, d_k, d_v, workspace, (int)n_heads,
                                 (int)seq_len, scale, causal != 0, s);
  else
    err = dfattn::launch_bwd_generic(q, k, v, d_o, d_q, d_k, d_v, (int)n_heads, (int)seq_len,
                                     (int)d_head, scale, causal != 0, s);
  return record_hip(err, "attention backward launch");
}

int dfattn_fwd_train(const float *q, const float *k, const float *v, float *o, float *lse,
                     void *workspace, size_t workspace_bytes, uint32_t n_heads, uint32_t seq_len,
                     uint32_t d_head, float scale, uint32_t causal, void *stream) {
  const char *fn = "dfattn_fwd_train";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, o, lse});
  if (st == DFATTN_OK) st = check_workspace(fn, workspace, workspace_bytes, n_heads, seq_len, d_head);
  if (st != DFATTN_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Without the fast path there are no copies to write: a backward that
  // takes its fast path has every pointer aligned, so this forward took it too.
  if (!fast_path(d_head, {q, k, v, o, lse})) return fwd_impl(q, k, v, o, lse, n_heads, seq_len, d_head, scale, causal, s);
  return record_hip(dfattn::launch_fwd_d64(q, k, v, o, lse, (int)n_heads, (int)seq_len, scale, causal != 0, s,
                                           workspace),
                    "attention forward launch");
}

// The split backward decides the fast path from q, k, v, o and d_o in both
// phases, so main takes it only when preprocess filled the workspace.
int dfattn_bwd_preprocess(const float *q, const float *k, const float *v, const float *o,
                          const float *d_o, const float *lse, void *workspace, size_t workspace_bytes,
                          uint32_t n_heads, uint32_t seq_len, uint32_t d_head, float scale,
                          uint32_t flags, void *stream) {
  const char *fn = "dfattn_bwd_preprocess";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, o, d_o, lse});
  if (st == DFATTN_OK) st = check_workspace(fn, workspace, workspace_bytes, n_heads, seq_len, d_head);
  if (st != DFATTN_OK) return st;
  // The generic kernel recomputes its row statistics itself: nothing to do.
  if (!fast_path(d_head, {q, k, v, o, d_o})) return DFATTN_OK;
  if ((flags & ~(uint32_t)DFATTN_BWD_QKV_SAVED) != 0)
    return record_error(DFATTN_ERR_FLAGS, std::string(fn) + ": unknown flag bits");
  return record_hip(dfattn::launch_bwd_pre_d64(q, k, v, o, d_o, lse, workspace, (int)n_heads, (int)seq_len,
                                               scale, static_cast<hipStream_t>(stream),
                                               (flags & DFATTN_BWD_QKV_SAVED) != 0),
                    "attention backward preprocess launch");
}

int dfattn_bwd_main(const float *q, const float *k, const float *v, const float *o,
                    const float *d_o, const float *lse, float *d_q, float *d_k, float *d_v,
                    void *workspace, size_t workspace_bytes, uint32_t n_heads, uint32_t seq_len,
                    uint32_t d_head, float scale, uint32_t causal, void *stream) {
  const char *fn = "dfattn_bwd_main";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, o, d_o, lse, d_q, d_k, d_v});
  if (st == DFATTN_OK) st = check_workspace(fn, workspace, workspace_bytes, n_heads, seq_len, d_head);
  if (st != DFATTN_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  if (fast_path(d_head, {q, k, v, o, d_o}) && fast_path(d_head, {lse, d_q, d_k, d_v}))
    err = dfattn::launch_bwd_main_d64(lse, d_q, d_k, d_v, workspace, (int)n_heads, (int)seq_len, scale,
                                      causal != 0, s);
  else
    err = dfattn::launch_bwd_generic(q, k, v, d_o, d_q, d_k, d_v, (int)n_heads, (int)seq_len,
                                     (int)d_head, scale, causal != 0, s);
  return record_hip(err, "attention backward launch");
}

int dfattn_fwd_train_strided(const float *q, const float *k, const float *v, float *o, float *lse,
                             void *workspace, size_t workspace_bytes, uint32_t n_heads, uint32_t seq_len,
                             uint32_t d_head, float scale, uint32_t causal, uint32_t qkv_row_stride,
                             void *stream) {
  const char *fn = "dfattn_fwd_train_strided";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, o, lse});
  if (st == DFATTN_OK) st = check_workspace(fn, workspace, workspace_bytes, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_strided(fn, d_head, n_heads, qkv_row_stride, {q, k, v, o, lse});
  if (st != DFATTN_OK) return st;
  return record_hip(dfattn::launch_fwd_d64(q, k, v, o, lse, (int)n_heads, (int)seq_len, scale, causal != 0,
                                           static_cast<hipStream_t>(stream), workspace, (int)qkv_row_stride),
                    "attention forward launch");
}

int dfattn_bwd_preprocess_strided(const float *q, const float *k, const float *v, const float *o,
                                  const float *d_o, const float *lse, void *workspace, size_t workspace_bytes,
                                  uint32_t n_heads, uint32_t seq_len, uint32_t d_head, float scale, uint32_t flags,
                                  uint32_t qkv_row_stride, void *stream) {
  const char *fn = "dfattn_bwd_preprocess_strided";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, o, d_o, lse});
  if (st == DFATTN_OK) st = check_workspace(fn, workspace, workspace_bytes, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_strided(fn, d_head, n_heads, qkv_row_stride, {q, k, v, o, d_o, lse});
  if (st != DFATTN_OK) return st;
  if ((flags & ~(uint32_t)DFATTN_BWD_QKV_SAVED) != 0)
    return record_error(DFATTN_ERR_FLAGS, std::string(fn) + ": unknown flag bits");
  return record_hip(dfattn::launch_bwd_pre_d64(q, k, v, o, d_o, lse, workspace, (int)n_heads, (int)seq_len,
                                               scale, static_cast<hipStream_t>(stream),
                                               (flags & DFATTN_BWD_QKV_SAVED) != 0, (int)qkv_row_stride),
                    "attention backward preprocess launch");
}

int dfattn_bwd_main_strided(const float *lse, float *d_q, float *d_k, float *d_v, void *workspace,
                            size_t workspace_bytes, uint32_t n_heads, uint32_t seq_len, uint32_t d_head,
                            float scale, uint32_t causal, uint32_t grad_row_stride, void *stream) {
  const char *fn = "dfattn_bwd_main_strided";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {lse, d_q, d_k, d_v});
  if (st == DFATTN_OK) st = check_workspace(fn, workspace, workspace_bytes, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_strided(fn, d_head, n_heads, grad_row_stride, {lse, d_q, d_k, d_v});
  if (st != DFATTN_OK) return st;
  return record_hip(dfattn::launch_bwd_main_d64(lse, d_q, d_k, d_v, workspace, (int)n_heads, (int)seq_len, scale,
                                                causal != 0, static_cast<hipStream_t>(stream),
                                                (int)grad_row_stride),
                    "attention backward launch");
}

}  // extern "C"

// ---- backward without allocation -------------------------------------------
// The backward's workspace in a static device array, for callers that cannot
// allocate (code under graph capture, serving loops, harnesses that forbid
// hipMalloc). Each device holds its own copy of the array from the library's
// load until the process ends; in host code `scratch` only names the symbol,
// its device address comes from hipGetSymbolAddress, once per device.
namespace {
static __device__ __align__(256) unsigned char scratch[DFATTN_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The scratch array's address on the current device (looked up on the first
// call on each device, with that device current). The first lookup makes the
// runtime load this file's code object on the device and place the array: an
// allocation inside the runtime, which a stream capture in global or
// thread-local mode forbids. That first call may itself be under capture, so
// the lookup runs with this thread's capture mode relaxed (and restored after);
// it enqueues nothing on any stream, so nothing enters the captured graph.
int scratch_on_current_device(const char *fn, void **out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return record_hip(err, fn);
  if (dev < 0 || dev >= kMaxDevices)
    return record_error(DFATTN_ERR_HIP, std::string(fn) + ": device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    err = hipThreadExchangeStreamCaptureMode(&mode);
    if (err != hipSuccess) return record_hip(err, fn);
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t restore = hipThreadExchangeStreamCaptureMode(&mode);
    if (err == hipSuccess) err = restore;
    if (err != hipSuccess) return record_hip(err, fn);
    if (p == nullptr) return record_error(DFATTN_ERR_HIP, std::string(fn) + ": scratch symbol has no address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DFATTN_OK;
}
}  // namespace

extern "C" {

int dfattn_bwd_noalloc(const float *q, const float *k, const float *v, const float *o, const float *d_o,
                       const float *lse, float *d_q, float *d_k, float *d_v, uint32_t n_heads,
                       uint32_t seq_len, uint32_t d_head, float scale, uint32_t causal, void *stream) {
  const char *fn = "dfattn_bwd_noalloc";
  int st = check_shape(fn, n_heads, seq_len, d_head);
  if (st == DFATTN_OK) st = check_ptrs(fn, {q, k, v, o, d_o, lse, d_q, d_k, d_v});
  if (st != DFATTN_OK) return st;
  const size_t need = dfattn_bwd_workspace_bytes(n_heads, seq_len, d_head);
  if (need > (size_t)DFATTN_NOALLOC_SCRATCH_BYTES)
    return record_error(DFATTN_ERR_WORKSPACE,
                        std::string(fn) + ": this shape needs " + std::to_string(need) +
                            " bytes of backward workspace, more than the static scratch holds (" +
                            std::to_string((size_t)DFATTN_NOALLOC_SCRATCH_BYTES) + "); use dfattn_bwd");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err;
  if (fast_path(d_head, {q, k, v, o, d_o, lse, d_q, d_k, d_v})) {
    void *ws = nullptr;
    st = scratch_on_current_device(fn, &ws);
    if (st != DFATTN_OK) return st;
    // Preprocess overwrites every workspace value the main kernel reads, so
    // nothing has to be cleared between calls.
    err = dfattn::launch_bwd_d64(q, k, v, o, d_o, lse, d_q, d_k, d_v, ws, (int)n_heads, (int)seq_len, scale,
                                 causal != 0, s);
  } else {
    err = dfattn::launch_bwd_generic(q, k, v, d_o, d_q, d_k, d_v, (int)n_heads, (int)seq_len, (int)d_head,
                                     scale, causal != 0, s);
  }
  return record_hip(err, "attention backward launch");
}

// ---- decode ----------------------------------------------------------------

void launch_fused_mha_decode_kv(const float *q, const float *k_cache, const float *v_cache, float *out,
                                uint32_t n_heads, uint32_t cur_seq_len, uint32_t d_head, float scale) {
  mark_pending_if_failed(legacy_decode("launch_fused_mha_decode_kv", q, k_cache, v_cache, nullptr, false, 1,
                                       false, nullptr, nullptr, nullptr, out, n_heads, cur_seq_len, d_head,
                                       scale, 0, false));
}

void launch_fused_mha_decode_kv_splitk(const float *q, const float *k_cache, const float *v_cache,
                                       float *partial_m, float *partial_l, float *partial_o, float *out,
                                       uint32_t n_heads, uint32_t cur_seq_len, uint32_t d_head, float scale,
                                       uint32_t chunk_size) {
  mark_pending_if_failed(legacy_decode("launch_fused_mha_decode_kv_splitk", q, k_cache, v_cache, nullptr,
                                       false, 1, false, partial_m, partial_l, partial_o, out, n_heads,
                                       cur_seq_len, d_head, scale, chunk_size, true));
}

void launch_paged_mha_decode_kv(const float *q, const float *k_pool, const float *v_pool,
                                const int32_t *block_table, float *out, uint32_t n_heads,
                                uint32_t cur_seq_len, uint32_t d_head, float scale, uint32_t page_size) {
  mark_pending_if_failed(legacy_decode("launch_paged_mha_decode_kv", q, k_pool, v_pool, block_table, true,
                                       page_size, false, nullptr, nullptr, nullptr, out, n_heads, cur_seq_len,
                                       d_head, scale, 0, false));
}

void launch_paged_mha_decode_kv_splitk(const float *q, const float *k_pool, const float *v_pool,
                                       const int32_t *block_table, float *partial_m, float *partial_l,
                                       float *partial_o, float *out, uint32_t n_heads, uint32_t cur_seq_len,
                                       uint32_t d_head, float scale, uint32_t page_size,
                                       uint32_t chunk_size) {
  mark_pending_if_failed(legacy_decode("launch_paged_mha_decode_kv_splitk", q, k_pool, v_pool, block_table,
                                       true, page_size, false, partial_m, partial_l, partial_o, out, n_heads,
                                       cur_seq_len, d_head, scale, chunk_size, true));
}

void launch_paged_mha_decode_kv_bf16(const float *q, const uint16_t *k_pool, const uint16_t *v_pool,
                                     const int32_t *block_table, float *out, uint32_t n_heads,
                                     uint32_t cur_seq_len, uint32_t d_head, float scale, uint32_t page_size) {
  mark_pending_if_failed(legacy_decode("launch_paged_mha_decode_kv_bf16", q, k_pool, v_pool, block_table,
                                       true, page_size, true, nullptr, nullptr, nullptr, out, n_heads,
                                       cur_seq_len, d_head, scale, 0, false));
}

void launch_pos_embed_interpolate(const float *pos_table, float *out, uint32_t pos, uint32_t trained_ctx_len,
                                  uint32_t max_ctx_len, uint32_t d_model) {
  mark_pending_if_failed(pos_embed_impl(pos_table, out, pos, trained_ctx_len, max_ctx_len, d_model));
}

void launch_apply_rope(float *qk, uint32_t pos, uint32_t n_heads, uint32_t d_head, float base_freq) {
  mark_pending_if_failed(rope_impl(qk, pos, n_heads, d_head, base_freq));
}

void launch_paged_copy_row(const float *src, float *pool, int32_t phys_block, uint32_t page_offset,
                           uint32_t page_size, uint32_t d_model) {
  mark_pending_if_failed(
      paged_copy_impl("launch_paged_copy_row", src, pool, false, phys_block, page_offset, page_size, d_model));
}

void launch_paged_copy_row_f32_to_bf16(const float *src, uint16_t *pool, int32_t phys_block, uint32_t page_offset,
                                       uint32_t page_size, uint32_t d_model) {
  mark_pending_if_failed(paged_copy_impl("launch_paged_copy_row_f32_to_bf16", src, pool, true, phys_block,
                                         page_offset, page_size, d_model));
}

size_t dfattn_decode_workspace_bytes(uint32_t n_heads, uint32_t cur_seq_len, uint32_t d_head) {
  if (n_heads == 0 || cur_seq_len == 0 || d_head == 0 || d_head > 128 || n_heads > kMaxHeads ||
      cur_seq_len > (1u << 30))
    return 0;
  const uint32_t n_chunks = decode_chunks(n_heads, cur_seq_len);
  if (n_chunks == 1) return 0;
  return (size_t)n_heads * n_chunks * (d_head + 2) * sizeof(float);
}

int dfattn_decode(const float *q, const void *k_cache, const void *v_cache, const int32_t *block_table,
                  uint32_t page_size, uint32_t kv_dtype, float *out, float *lse, uint32_t n_heads,
                  uint32_t cur_seq_len, uint32_t d_head, float scale, void *workspace, size_t workspace_bytes,
                  void *stream) {
  const char *fn = "dfattn_decode";
  if (kv_dtype != DFATTN_KV_F32 && kv_dtype != DFATTN_KV_BF16)
    return record_error(DFATTN_ERR_FLAGS, std::string(fn) + ": unknown kv_dtype");
  const bool bf16 = kv_dtype == DFATTN_KV_BF16, paged = block_table != nullptr;
  int st = check_decode(fn, q, k_cache, v_cache, block_table, paged, paged ? page_size : 1, bf16, out, n_heads,
                        cur_seq_len, d_head);
  if (st != DFATTN_OK) return st;
  if (lse != nullptr && !aligned(lse, 4))
    return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": misaligned pointer");
  if (cur_seq_len == 0) return DFATTN_OK;
  const size_t need = dfattn_decode_workspace_bytes(n_heads, cur_seq_len, d_head);
  if (workspace != nullptr && (workspace_bytes < need || !aligned(workspace, 4)))
    return record_error(DFATTN_ERR_WORKSPACE, std::string(fn) + ": workspace too small or misaligned");
  // Without a workspace one workgroup per head walks all keys.
  const uint32_t n_chunks = workspace != nullptr ? decode_chunks(n_heads, cur_seq_len) : 1;
  float *pm = nullptr, *pl = nullptr, *po = nullptr;
  uint32_t chunk = cur_seq_len;
  if (n_chunks > 1) {
    chunk = decode_chunk_len(cur_seq_len, n_chunks);
    const uint32_t used = (cur_seq_len + chunk - 1) / chunk;
    pm = static_cast<float *>(workspace);
    pl = pm + (size_t)n_heads * used;
    po = pl + (size_t)n_heads * used;
  }
  const hipError_t err = dfattn::launch_decode(
      q, k_cache, v_cache, block_table, (int)(paged ? page_size : 1), bf16, out, lse, (int)n_heads,
      (int)cur_seq_len, (int)d_head, scale, (int)chunk, pm, pl, po,
      decode_fast(d_head, bf16, q, k_cache, v_cache) && (lse == nullptr || aligned(lse, 4)),
      static_cast<hipStream_t>(stream));
  return record_hip(err, "decode launch");
}

const char *dfattn_status_string(int status) {
  switch (status) {
    case DFATTN_OK: return "ok";
    case DFATTN_ERR_NULL_POINTER: return "null pointer";
    case DFATTN_ERR_MISALIGNED: return "misaligned pointer";
    case DFATTN_ERR_SHAPE: return "invalid shape";
    case DFATTN_ERR_HEAD_DIM: return "d_head out of range";
    case DFATTN_ERR_OVERFLOW: return "shape overflow";
    case DFATTN_ERR_WORKSPACE: return "workspace too small";
    case DFATTN_ERR_HIP: return "HIP error";
    case DFATTN_ERR_FLAGS: return "unknown flags";
    default: return "unknown status";
  }
}

int dfattn_last_error(void) {
  std::lock_guard<std::mutex> lock(g_err_mu);
  return g_err;
}

const char *dfattn_last_error_message(void) {
  static thread_local std::string copy;
  std::lock_guard<std::mutex> lock(g_err_mu);
  copy = g_err_msg;
  return copy.c_str();
}

void dfattn_clear_error(void) {
  std::lock_guard<std::mutex> lock(g_err_mu);
  g_err = DFATTN_OK;
  g_err_msg.clear();
  g_pending = DFATTN_OK;
  g_pending_msg.clear();
}

const char *dfattn_version(void) { return "dfattn 0.1.0 (gfx950, MFMA f16 / fp32 accumulate)"; }

}  // extern "C"
