// gpt2_loss_embed.hip — the GPT-2 step's token embedding (forward and
// backward) and its chunked, fused logit cross-entropy on gfx950.
//
// They replace the reference engine's launchers of the same names
// (darkforest-cuda/kernels/elementwise.cu:268, 291; softmax.cu:396), which
// the engine's step calls at static_gpt2.rs:1292-1305 (embedding lookups),
// 1386-1418 (the loss over chunks of at most 512 rows) and 1559-1574
// (embedding gradients).
//
//  * Cross-entropy: one workgroup per row of logits. The row (50257 values
//    for GPT-2) is read once into registers (98 values per thread), its max
//    and sum of exponentials are merged in a fixed order, and the gradient
//    (softmax - one_hot) / total_rows is written from the registers (rows
//    too long for that: an online max and sum per thread, then a second
//    read for the gradient). The
//    stream entry point writes each row's loss to its own slot (summed in a
//    fixed order afterwards), so a step's loss is reproducible bit for bit;
//    the reference's launcher adds the rows' losses with float atomics, and
//    so does its counterpart here.
//  * Embedding forward: a gather of table rows, one wave per row, float4.
//  * Embedding backward: grad_table[idx[p]] += grad_out[p] with every row
//    summed in position order by the workgroup of the first position that
//    holds its token id (a ballot scan finds the others), so no two
//    workgroups write one table row and there are no atomics; the reference
//    adds with one float atomic per value.
#include "dfattn_internal.h"
#include "dfattn_status.h"
#include "dfgpt2.h"

#include <climits>
#include <initializer_list>
#include <string>

namespace dfattn {
namespace {

constexpr int kCeThreads = 512;

// Online (max, sum of exp(x - max)) of a stream of values, in log2 units.
struct MaxSum {
  float m, s;
};
__device__ __forceinline__ MaxSum ms_add(MaxSum a, float x) {
  if (x > a.m) {
    a.s = a.s * exp2f((a.m - x) * kLog2e) + 1.f;
    a.m = x;
  } else if (x > -INFINITY) {
    a.s += exp2f((x - a.m) * kLog2e);
  }
  return a;
}
__device__ __forceinline__ MaxSum ms_merge(MaxSum a, MaxSum b) {
  if (b.m > a.m) {
    const MaxSum t = a;
    a = b;
    b = t;
  }
  if (b.m == -INFINITY) return a;
  a.s += b.s * exp2f((b.m - a.m) * kLog2e);
  return a;
}

// One row of `cols` logits per workgroup. WRITE_PROBS (the reference
// launcher's contract): the logits row is overwritten with the softmax;
// ROW_LOSS: the row's loss goes to row_loss[row], else it is added to *loss
// with an atomic. grad may alias logits when !WRITE_PROBS.
template <bool WRITE_PROBS, bool ROW_LOSS>
__global__ __launch_bounds__(kCeThreads) void ce_row_kernel(float *logits, const uint32_t *__restrict__ targets,
                                                            float *grad, float *__restrict__ row_loss,
                                                            float *__restrict__ loss, int cols, float inv_total) {
  __shared__ float red_m[kCeThreads / 64], red_s[kCeThreads / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float *x = logits + (size_t)row * cols;
  float *gx = grad + (size_t)row * cols;
  MaxSum acc = {-INFINITY, 0.f};
  for (int i = tid; i < cols; i += kCeThreads) acc = ms_add(acc, x[i]);
  // Fixed-order merge: lanes by xor butterfly, then the waves in order.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    MaxSum o;
    o.m = __shfl_xor(acc.m, off, 64);
    o.s = __shfl_xor(acc.s, off, 64);
    acc = (lane & off) ? ms_merge(o, acc) : ms_merge(acc, o);
  }
  if (lane == 0) {
    red_m[wave] = acc.m;
    red_s[wave] = acc.s;
  }
  __syncthreads();
  MaxSum tot = {red_m[0], red_s[0]};
#pragma unroll
  for (int w = 1; w < kCeThreads / 64; ++w) tot = ms_merge(tot, MaxSum{red_m[w], red_s[w]});
  const float inv_sum = 1.f / tot.s;
  const uint32_t target = targets[row];
  // The target's logit, read before the row is overwritten below.
  const float xt = target < (uint32_t)cols ? x[target] : -INFINITY;
  __syncthreads();
  for (int i = tid; i < cols; i += kCeThreads) {
    const float p = exp2f((x[i] - tot.m) * kLog2e) * inv_sum;
    if (WRITE_PROBS) x[i] = p;
    gx[i] = (p - ((uint32_t)i == target ? 1.f : 0.f)) * inv_total;
  }
  if (tid == 0) {
    // The target's probability from the same formula the gradient used (a
    // target outside the row gives probability 0, clamped as below).
    const float pt = exp2f((xt - tot.m) * kLog2e) * inv_sum;
    const float l = -logf(fmaxf(pt, 1e-12f)) * inv_total;  // softmax.cu:377 clamps at 1e-12
    if (ROW_LOSS)
      row_loss[row] = l;
    else
      atomicAdd(loss, l);
  }
}

// The same contract with the row held in registers, K values per thread
// (cols <= K * kCeThreads): one read of the row, its maximum, then the sum of
// exponentials about it (both merged in a fixed order: lanes by butterfly,
// then the waves in order), with the exponentials kept in registers for the
// gradient's write. One read and one write of the row instead of two reads
// and a write.
template <bool WRITE_PROBS, bool ROW_LOSS, int K>
__global__ __launch_bounds__(kCeThreads) void ce_row_reg_kernel(float *logits, const uint32_t *__restrict__ targets,
                                                                float *grad, float *__restrict__ row_loss,
                                                                float *__restrict__ loss, int cols, float inv_total) {
  __shared__ float red[kCeThreads / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float *x = logits + (size_t)row * cols;
  float *gx = grad + (size_t)row * cols;
  const uint32_t target = targets[row];
  // The target's logit, read before any thread overwrites the row.
  const float xt = (tid == 0 && target < (uint32_t)cols) ? x[target] : -INFINITY;
  // Buffer accesses bounded by the row (the lane's byte offset in the vector
  // offset, which the hardware checks: loads past the row read 0, stores
  // there are dropped), so the row needs no 64-bit address per value.
  const auto rx = buffer_rsrc(x, (unsigned)cols * 4u);
  const auto rg = buffer_rsrc(gx, (unsigned)cols * 4u);
  float v[K];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < K; ++k)
    v[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, (tid + k * kCeThreads) * 4, 0, 0));
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (tid + k * kCeThreads >= cols) v[k] = -INFINITY;
    mx = fmaxf(mx, v[k]);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kCeThreads / 64; ++w) m = fmaxf(m, red[w]);
  __syncthreads();  // red is reused for the sums
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    v[k] = exp2f((v[k] - m) * kLog2e);  // 0 past the row's end
    s += v[k];
  }
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  float tot = red[0];
#pragma unroll
  for (int w = 1; w < kCeThreads / 64; ++w) tot += red[w];
  const float inv_sum = 1.f / tot;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = tid + k * kCeThreads;
    const float p = v[k] * inv_sum;
    if (WRITE_PROBS) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, p), rx, i * 4, 0, 0);
    const float gv = (p - ((uint32_t)i == target ? 1.f : 0.f)) * inv_total;
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, gv), rg, i * 4, 0, 0);
  }
  if (tid == 0) {
    const float pt = exp2f((xt - m) * kLog2e) * inv_sum;
    const float l = -logf(fmaxf(pt, 1e-12f)) * inv_total;  // softmax.cu:377 clamps at 1e-12
    if (ROW_LOSS)
      row_loss[row] = l;
    else
      atomicAdd(loss, l);
  }
}

// One launch of the cross-entropy over `rows` rows: the register-resident
// kernel when a row fits (cols <= 100 * kCeThreads, GPT-2's 50257 among
// them), else the two-read one.
template <bool WRITE_PROBS, bool ROW_LOSS>
void launch_ce(float *logits, const uint32_t *targets, float *grad, float *row_loss, float *loss, uint32_t rows,
               uint32_t cols, float inv_total, hipStream_t stream) {
  const dim3 grid(rows), block(kCeThreads);
  const int c = (int)cols;
  if (cols <= 1u * kCeThreads)
    hipLaunchKernelGGL((ce_row_reg_kernel<WRITE_PROBS, ROW_LOSS, 1>), grid, block, 0, stream, logits, targets, grad,
                       row_loss, loss, c, inv_total);
  else if (cols <= 8u * kCeThreads)
    hipLaunchKernelGGL((ce_row_reg_kernel<WRITE_PROBS, ROW_LOSS, 8>), grid, block, 0, stream, logits, targets, grad,
                       row_loss, loss, c, inv_total);
  else if (cols <= 32u * kCeThreads)
    hipLaunchKernelGGL((ce_row_reg_kernel<WRITE_PROBS, ROW_LOSS, 32>), grid, block, 0, stream, logits, targets, grad,
                       row_loss, loss, c, inv_total);
  else if (cols <= 100u * kCeThreads)
    hipLaunchKernelGGL((ce_row_reg_kernel<WRITE_PROBS, ROW_LOSS, 100>), grid, block, 0, stream, logits, targets,
                       grad, row_loss, loss, c, inv_total);
  else
    hipLaunchKernelGGL((ce_row_kernel<WRITE_PROBS, ROW_LOSS>), grid, block, 0, stream, logits, targets, grad, row_loss,
                       loss, c, inv_total);
}

// Sum of n values in a fixed order (one workgroup): the step's loss from the
// rows' slots.
__global__ __launch_bounds__(256) void sum_kernel(const float *__restrict__ v, int n, float *__restrict__ out,
                                                  int accumulate) {
  __shared__ float part[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float a = 0.f;
  for (int i = tid; i < n; i += 256) a += v[i];
  a = wave_sum(a);
  if (lane == 0) part[wave] = a;
  __syncthreads();
  if (tid == 0) {
    const float s = (part[0] + part[1]) + (part[2] + part[3]);
    *out = accumulate ? *out + s : s;
  }
}

// Rows of the table by token id: one wave per output row; rows with an id at
// or past `rows_in_table` are written as zeros (the reference reads past the
// table there). VEC: dim % 4 == 0 and 16-byte aligned tensors.
template <bool VEC>
__global__ __launch_bounds__(256) void embed_fwd_kernel(const uint32_t *__restrict__ idx,
                                                        const float *__restrict__ table, float *__restrict__ out,
                                                        int n_rows, int dim, uint32_t rows_in_table) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= n_rows) return;
  const uint32_t id = idx[row];
  const bool ok = id < rows_in_table;
  const float *src = table + (size_t)(ok ? id : 0) * dim;
  float *dst = out + (size_t)row * dim;
  if (VEC) {
    for (int c = lane; c < dim / 4; c += 64) {
      const float4 vv = ok ? reinterpret_cast<const float4 *>(src)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
      reinterpret_cast<float4 *>(dst)[c] = vv;
    }
  } else {
    for (int c = lane; c < dim; c += 64) dst[c] = ok ? src[c] : 0.f;
  }
}

// grad_table[idx[p]] += the sum of grad_out[q] over the positions q holding
// that id, in a fixed order. Workgroup p owns the id if no earlier position
// holds it: its four waves scan the earlier ids, wave w the 64-position blocks
// b = w (mod 4), and the workgroup leaves if any wave finds one. In the owner,
// wave w sums the matching rows q >= p of its blocks in increasing q
// (kRowsInFlight rows loaded ahead of the adds), and wave 0 adds
// ((s0 + s1) + s2) + s3 to the table row: bitwise reproducible (the
// reference's launcher adds with atomics, in no fixed order). Lane l holds
// columns 4l + 256j, j < kColChunks (dim <= 1024 per pass, looping above).
// Ids at or past rows_in_table are skipped. VEC: dim % 4 == 0 and 16-byte
// aligned grad_out and grad_table.
// Cost: the scans read about n^2/2 ids in all, 256 per step of a workgroup
// (L2 hits); an id repeated r times costs its owner about
// r / (4 * kRowsInFlight) load latencies. Meant for the GPT-2 step's
// sequences (up to a few thousand positions).
constexpr int kRowsInFlight = 8;
constexpr int kColChunks = 4;

template <bool VEC>
__global__ __launch_bounds__(256) void embed_bwd_kernel(const uint32_t *__restrict__ idx,
                                                        const float *__restrict__ grad_out,
                                                        float *__restrict__ grad_table, int n_rows, int dim,
                                                        uint32_t rows_in_table) {
  __shared__ float4 part[4][kColChunks][64];
  const int p = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t id = idx[p];
  if (id >= rows_in_table) return;  // the same for the whole workgroup
  bool found = false;
  for (int base = w * 64; base < p && !found; base += 256) {
    const int q = base + lane;
    found = __any(q < p && idx[q] == id);
  }
  if (__syncthreads_or(found)) return;

  auto load4 = [&](const float *row, int c) {
    if (VEC) return c < dim ? *reinterpret_cast<const float4 *>(row + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    float4 r = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c + j < dim) (&r.x)[j] = row[c + j];
    return r;
  };
  const int b0 = p >> 6;
  const int first = b0 + (((w - b0) % 4) + 4) % 4;  // this wave's first block at or after p's
  for (int c0 = 0; c0 < dim; c0 += 256 * kColChunks) {
    float4 acc[kColChunks];
#pragma unroll
    for (int k = 0; k < kColChunks; ++k) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int b = first; b * 64 < n_rows; b += 4) {
      const int q = b * 64 + lane;
      unsigned long long hits = __ballot(q >= p && q < n_rows && idx[q] == id);
      while (hits) {
        int rows[kRowsInFlight], n = 0;
        for (; hits && n < kRowsInFlight; ++n) {
          rows[n] = b * 64 + __builtin_ctzll(hits);
          hits &= hits - 1;
        }
        float4 r[kRowsInFlight][kColChunks];
#pragma unroll
        for (int j = 0; j < kRowsInFlight; ++j)
#pragma unroll
          for (int k = 0; k < kColChunks; ++k)
            if (j < n) r[j][k] = load4(grad_out + (size_t)rows[j] * dim, c0 + 256 * k + 4 * lane);
#pragma unroll
        for (int j = 0; j < kRowsInFlight; ++j)
#pragma unroll
          for (int k = 0; k < kColChunks; ++k)
            if (j < n) {
              acc[k].x += r[j][k].x;
              acc[k].y += r[j][k].y;
              acc[k].z += r[j][k].z;
              acc[k].w += r[j][k].w;
            }
      }
    }
#pragma unroll
    for (int k = 0; k < kColChunks; ++k) part[w][k][lane] = acc[k];
    __syncthreads();
    if (w == 0) {
      float *dst = grad_table + (size_t)id * dim;
#pragma unroll
      for (int k = 0; k < kColChunks; ++k) {
        const int c = c0 + 256 * k + 4 * lane;
        float4 t = part[0][k][lane];
#pragma unroll
        for (int v = 1; v < 4; ++v) {
          const float4 u = part[v][k][lane];
          t.x += u.x;
          t.y += u.y;
          t.z += u.z;
          t.w += u.w;
        }
        if (VEC) {
          if (c < dim) {
            float4 d = *reinterpret_cast<float4 *>(dst + c);
            d.x += t.x;
            d.y += t.y;
            d.z += t.z;
            d.w += t.w;
            *reinterpret_cast<float4 *>(dst + c) = d;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (c + j < dim) dst[c + j] += (&t.x)[j];
        }
      }
    }
    __syncthreads();  // part is written again by the next pass
  }
}

// ------------------------------------------------------------------- host
bool al(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int launched(const char *fn) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return DFATTN_OK;
  return record_error(DFATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(err));
}

int need(const char *fn, std::initializer_list<const void *> ptrs) {
  for (const void *p : ptrs)
    if (p == nullptr) return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null pointer");
  for (const void *p : ptrs)
    if (!al(p, 4)) return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": pointer not 4-byte aligned");
  return DFATTN_OK;
}

int dims_ok(const char *fn, uint32_t rows, uint32_t cols) {
  if (cols == 0) return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": row length must be >= 1");
  size_t n = 0;
  if (rows > (uint32_t)INT_MAX || cols > (uint32_t)INT_MAX || __builtin_mul_overflow((size_t)rows, (size_t)cols, &n))
    return record_error(DFATTN_ERR_OVERFLOW, std::string(fn) + ": shape is too large");
  return DFATTN_OK;
}

}  // namespace
}  // namespace dfattn

using namespace dfattn;

extern "C" int dfgpt2_logit_ce_chunk(float *logits, const uint32_t *targets, float *grad_logits, float *row_loss,
                                     uint32_t chunk_rows, uint32_t cols, uint32_t total_rows, hipStream_t stream) {
  const char *fn = "dfgpt2_logit_ce_chunk";
  if (chunk_rows == 0) return DFATTN_OK;
  if (int st = need(fn, {logits, targets, grad_logits, row_loss}); st != DFATTN_OK) return st;
  if (int st = dims_ok(fn, chunk_rows, cols); st != DFATTN_OK) return st;
  if (total_rows == 0) return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": total_rows must be >= 1");
  launch_ce<false, true>(logits, targets, grad_logits, row_loss, nullptr, chunk_rows, cols, 1.f / (float)total_rows,
                         stream);
  return launched(fn);
}

extern "C" int dfgpt2_sum(const float *values, uint32_t n, float *out, int accumulate, hipStream_t stream) {
  const char *fn = "dfgpt2_sum";
  if (int st = need(fn, {out}); st != DFATTN_OK) return st;
  if (n > 0)
    if (int st = need(fn, {values}); st != DFATTN_OK) return st;
  if (n > (uint32_t)INT_MAX) return record_error(DFATTN_ERR_OVERFLOW, std::string(fn) + ": n is too large");
  hipLaunchKernelGGL(sum_kernel, dim3(1), dim3(256), 0, stream, values, (int)n, out, accumulate ? 1 : 0);
  return launched(fn);
}

extern "C" int dfgpt2_embedding_forward(const uint32_t *indices, const float *table, float *out, uint32_t n_rows,
                                        uint32_t dim, uint32_t rows_in_table, hipStream_t stream) {
  const char *fn = "dfgpt2_embedding_forward";
  if (n_rows == 0) return DFATTN_OK;
  if (int st = need(fn, {indices, table, out}); st != DFATTN_OK) return st;
  if (int st = dims_ok(fn, n_rows, dim); st != DFATTN_OK) return st;
  const dim3 grid((n_rows + 3) / 4);
  if (dim % 4 == 0 && al(table, 16) && al(out, 16))
    hipLaunchKernelGGL(embed_fwd_kernel<true>, grid, dim3(256), 0, stream, indices, table, out, (int)n_rows,
                       (int)dim, rows_in_table);
  else
    hipLaunchKernelGGL(embed_fwd_kernel<false>, grid, dim3(256), 0, stream, indices, table, out, (int)n_rows,
                       (int)dim, rows_in_table);
  return launched(fn);
}

extern "C" int dfgpt2_embedding_backward(const uint32_t *indices, const float *grad_out, float *grad_table,
                                         uint32_t n_rows, uint32_t dim, uint32_t rows_in_table, hipStream_t stream) {
  const char *fn = "dfgpt2_embedding_backward";
  if (n_rows == 0) return DFATTN_OK;
  if (int st = need(fn, {indices, grad_out, grad_table}); st != DFATTN_OK) return st;
  if (int st = dims_ok(fn, n_rows, dim); st != DFATTN_OK) return st;
  if (dim % 4 == 0 && al(grad_out, 16) && al(grad_table, 16))
    hipLaunchKernelGGL(embed_bwd_kernel<true>, dim3(n_rows), dim3(256), 0, stream, indices, grad_out, grad_table,
                       (int)n_rows, (int)dim, rows_in_table);
  else
    hipLaunchKernelGGL(embed_bwd_kernel<false>, dim3(n_rows), dim3(256), 0, stream, indices, grad_out, grad_table,
                       (int)n_rows, (int)dim, rows_in_table);
  return launched(fn);
}

// ------------------------------------------------- the reference's symbols
// softmax.cu:396: logits overwritten with the softmax, grad_logits =
// (softmax - one_hot) / total_rows, *loss += sum of -log(p_target) /
// total_rows (float atomics, as the reference).
extern "C" void launch_fused_chunked_logit_ce(float *logits, const uint32_t *targets, float *grad_logits,
                                              float *loss, uint32_t chunk_rows, uint32_t cols,
                                              uint32_t total_rows) {
  const char *fn = "launch_fused_chunked_logit_ce";
  int st = DFATTN_OK;
  if (chunk_rows > 0) {
    st = need(fn, {logits, targets, grad_logits, loss});
    if (st == DFATTN_OK) st = dims_ok(fn, chunk_rows, cols);
    if (st == DFATTN_OK && total_rows == 0)
      st = record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": total_rows must be >= 1");
    if (st == DFATTN_OK) {
      launch_ce<true, false>(logits, targets, grad_logits, nullptr, loss, chunk_rows, cols, 1.f / (float)total_rows,
                             nullptr);
      st = launched(fn);
    }
  }
  mark_pending(st);
}

// elementwise.cu:268: out[p] = weight[indices[p]] (ids are not range-checked:
// the launcher, like the reference's, has no table size).
extern "C" void launch_embedding_forward(const uint32_t *indices, const float *weight, float *out, uint32_t seq_len,
                                         uint32_t embed_dim) {
  mark_pending(dfgpt2_embedding_forward(indices, weight, out, seq_len, embed_dim, UINT32_MAX, nullptr));
}

// elementwise.cu:291: grad_weight[indices[p]] += grad_out[p] (the caller
// zeroes grad_weight, as the reference's DeviceTensor wrapper does).
extern "C" void launch_embedding_backward(const uint32_t *indices, const float *grad_out, float *grad_weight,
                                          uint32_t seq_len, uint32_t embed_dim) {
  mark_pending(dfgpt2_embedding_backward(indices, grad_out, grad_weight, seq_len, embed_dim, UINT32_MAX, nullptr));
}
