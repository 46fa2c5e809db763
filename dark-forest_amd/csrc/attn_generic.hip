// attn_generic.hip — fp32 attention kernels for any d_head in 1..=128.
//
// The MFMA kernels cover d_head = 64 (GPT-2's head size and every config this
// library is measured on). These kernels keep the reference's full argument
// range (AttentionContext accepts 1 <= d_head <= 128, darkforest-cuda/src/lib.rs:1981)
// and are exact fp32: one wave per (query row, head); lanes take 64 keys at a
// time for the scores and the d columns for the accumulations. Unlike the
// reference kernels (attention_fused.cu:111-112, 417-420) they are correct for
// 64 < d_head <= 128 as well.
#include "dfattn_internal.h"

namespace dfattn {
namespace {

constexpr int kMaxD = 128;

__global__ __launch_bounds__(256) void fill_zero_kernel(float *__restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0.f;
}

// One online-softmax pass over the visible keys of one row. On return
// o0/o1 hold the unnormalised output for columns lane and lane + 64, m the
// running max and l the sum of exp(s - m).
__device__ void row_forward(const float *qrow_lds, const float *__restrict__ K,
                            const float *__restrict__ V, size_t ld, size_t hoff, int D,
                            int kmax, float scale, int lane, float &m, float &l, float &o0,
                            float &o1) {
  m = -INFINITY;
  l = 0.f;
  o0 = o1 = 0.f;
  for (int j0 = 0; j0 < kmax; j0 += 64) {
    const int key = j0 + lane;
    float s = -INFINITY;
    if (key < kmax) {
      const float *krow = K + (size_t)key * ld + hoff;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot += qrow_lds[d] * krow[d];
      s = dot * scale;
    }
    const float m_new = fmaxf(m, wave_max(s));
    const float alpha = (m == -INFINITY) ? 0.f : expf(m - m_new);
    const float p = (key < kmax) ? expf(s - m_new) : 0.f;
    l = l * alpha + wave_sum(p);
    o0 *= alpha;
    o1 *= alpha;
    const int n = min(64, kmax - j0);
    for (int jj = 0; jj < n; ++jj) {
      const float pj = __shfl(p, jj, 64);
      const float *vrow = V + (size_t)(j0 + jj) * ld + hoff;
      if (lane < D) o0 += pj * vrow[lane];
      if (lane + 64 < D) o1 += pj * vrow[lane + 64];
    }
    m = m_new;
  }
}

__global__ __launch_bounds__(256) void fwd_generic_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    float *__restrict__ O, float *__restrict__ LSE, int H, int S, int D, float scale,
    int causal) {
  __shared__ float qs[4][kMaxD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave, head = blockIdx.y;
  const size_t ld = (size_t)H * D, hoff = (size_t)head * D;
  for (int d = lane; d < D; d += 64) qs[wave][d] = row < S ? Q[(size_t)row * ld + hoff + d] : 0.f;
  __syncthreads();
  if (row >= S) return;
  const int kmax = causal ? row + 1 : S;
  float m, l, o0, o1;
  row_forward(qs[wave], K, V, ld, hoff, D, kmax, scale, lane, m, l, o0, o1);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float *orow = O + (size_t)row * ld + hoff;
  if (lane < D) orow[lane] = o0 * inv;
  if (lane + 64 < D) orow[lane + 64] = o1 * inv;
  if (LSE != nullptr && lane == 0)
    LSE[(size_t)head * S + row] = l > 0.f ? m + logf(l) : -INFINITY;
}

// Backward of one row: recompute (m, l, o) to get lse and Delta = dO . O,
// then P = exp(s - lse), dS = P (dP - Delta); dQ stays in registers, dK and
// dV are accumulated with fp32 atomics (the reference's scheme,
// attention_fused.cu:483-507). dK and dV must be zero on entry.
__global__ __launch_bounds__(256) void bwd_generic_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    const float *__restrict__ dO, float *__restrict__ dQ, float *__restrict__ dK,
    float *__restrict__ dV, int H, int S, int D, float scale, int causal) {
  __shared__ float qs[4][kMaxD];
  __shared__ float gs[4][kMaxD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave, head = blockIdx.y;
  const size_t ld = (size_t)H * D, hoff = (size_t)head * D;
  for (int d = lane; d < D; d += 64) {
    qs[wave][d] = row < S ? Q[(size_t)row * ld + hoff + d] : 0.f;
    gs[wave][d] = row < S ? dO[(size_t)row * ld + hoff + d] : 0.f;
  }
  __syncthreads();
  if (row >= S) return;
  const int kmax = causal ? row + 1 : S;
  float m, l, o0, o1;
  row_forward(qs[wave], K, V, ld, hoff, D, kmax, scale, lane, m, l, o0, o1);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const float lse = l > 0.f ? m + logf(l) : INFINITY;
  float part = 0.f;
  if (lane < D) part += gs[wave][lane] * o0 * inv;
  if (lane + 64 < D) part += gs[wave][lane + 64] * o1 * inv;
  const float delta = wave_sum(part);

  float dq0 = 0.f, dq1 = 0.f;
  const float q0 = lane < D ? qs[wave][lane] : 0.f, q1 = lane + 64 < D ? qs[wave][lane + 64] : 0.f;
  const float g0 = lane < D ? gs[wave][lane] : 0.f, g1 = lane + 64 < D ? gs[wave][lane + 64] : 0.f;
  for (int j0 = 0; j0 < kmax; j0 += 64) {
    const int key = j0 + lane;
    float p = 0.f, dsc = 0.f;
    if (key < kmax) {
      const float *krow = K + (size_t)key * ld + hoff;
      const float *vrow = V + (size_t)key * ld + hoff;
      float dot = 0.f, dp = 0.f;
      for (int d = 0; d < D; ++d) {
        dot += qs[wave][d] * krow[d];
        dp += gs[wave][d] * vrow[d];
      }
      p = expf(dot * scale - lse);
      dsc = p * (dp - delta);
    }
    const int n = min(64, kmax - j0);
    for (int jj = 0; jj < n; ++jj) {
      const float pj = __shfl(p, jj, 64), dsj = __shfl(dsc, jj, 64);
      const size_t base = (size_t)(j0 + jj) * ld + hoff;
      if (lane < D) {
        dq0 += dsj * K[base + lane];
        unsafeAtomicAdd(dK + base + lane, scale * dsj * q0);
        unsafeAtomicAdd(dV + base + lane, pj * g0);
      }
      if (lane + 64 < D) {
        dq1 += dsj * K[base + lane + 64];
        unsafeAtomicAdd(dK + base + lane + 64, scale * dsj * q1);
        unsafeAtomicAdd(dV + base + lane + 64, pj * g1);
      }
    }
  }
  float *dqrow = dQ + (size_t)row * ld + hoff;
  if (lane < D) dqrow[lane] = scale * dq0;
  if (lane + 64 < D) dqrow[lane + 64] = scale * dq1;
}

hipError_t fill_zero(float *p, size_t n, hipStream_t stream) {
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)std::max<size_t>(blocks, 1)), dim3(256), 0,
                     stream, p, n);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd_generic(const float *q, const float *k, const float *v, float *o,
                              float *lse, int n_heads, int seq_len, int d_head, float scale,
                              bool causal, hipStream_t stream) {
  const dim3 grid((seq_len + 3) / 4, n_heads);
  hipLaunchKernelGGL(fwd_generic_kernel, grid, dim3(256), 0, stream, q, k, v, o, lse, n_heads,
                     seq_len, d_head, scale, causal ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_bwd_generic(const float *q, const float *k, const float *v, const float *d_o,
                              float *d_q, float *d_k, float *d_v, int n_heads, int seq_len,
                              int d_head, float scale, bool causal, hipStream_t stream) {
  const size_t n = (size_t)seq_len * n_heads * d_head;
  hipError_t err = fill_zero(d_k, n, stream);
  if (err == hipSuccess) err = fill_zero(d_v, n, stream);
  if (err != hipSuccess) return err;
  const dim3 grid((seq_len + 3) / 4, n_heads);
  hipLaunchKernelGGL(bwd_generic_kernel, grid, dim3(256), 0, stream, q, k, v, d_o, d_q, d_k, d_v,
                     n_heads, seq_len, d_head, scale, causal ? 1 : 0);
  return hipGetLastError();
}

}  // namespace dfattn
