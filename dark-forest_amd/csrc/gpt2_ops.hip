// gpt2_ops.hip — the GPT-2 training step's non-attention kernels on gfx950:
// LayerNorm forward and backward, tanh GELU forward and backward, the bias
// gradient of a linear layer and the AdamW update.
//
// They replace the reference engine's launchers of the same names
// (darkforest-cuda/kernels/layernorm.cu:97, 187; elementwise.cu:195, 217;
// matmul.cu:240, 341), which the engine's step calls around its attention
// (darkforest-core/src/engine/static_gpt2.rs:1315-1364, 1427-1543, 1661).
// All of them are memory-bound (a few bytes per flop): rows are read as
// float4 by wave64 lanes, LayerNorm keeps a row in registers (one wave per
// row), and the column reductions (bias and LayerNorm parameter gradients)
// give each workgroup 16 columns and a fixed summation order instead of the
// reference's floating-point atomics, so every result is reproducible bit
// for bit (AdamW's sign-sensitive update of a near-zero gradient depends on
// that).
#include "dfattn_internal.h"
#include "dfattn_status.h"
#include "dfgpt2.h"

#include <climits>
#include <initializer_list>
#include <string>

namespace dfattn {
namespace {

constexpr float kLnEps = 1e-5f;  // layernorm.cu:14
// tanh GELU constants: sqrt(2/pi) and the cubic coefficient (elementwise.cu:181-182).
constexpr float kGeluK0 = 0.7978845608028654f;
constexpr float kGeluK1 = 0.044715f;

__device__ __forceinline__ float4 splat4(float a) { return make_float4(a, a, a, a); }
__device__ __forceinline__ float hsum4(float4 v) { return (v.x + v.y) + (v.z + v.w); }

// ------------------------------------------------------------ LayerNorm forward
// One wave per row, V float4 per lane held in registers (features <= 256 V,
// features % 4 == 0, 16-byte aligned rows); four rows per 256-thread
// workgroup. The mean, then the variance about it, as layernorm.cu:41-75.
// With y: the row normalised is x + y (one fp32 add per value, a residual
// connection), also stored to sum_out.
template <int V>
__global__ __launch_bounds__(256) void ln_fwd_vec_kernel(const float *__restrict__ x, const float *__restrict__ y,
                                                         const float *__restrict__ gamma,
                                                         const float *__restrict__ beta, float *__restrict__ sum_out,
                                                         float *__restrict__ out, float *__restrict__ means,
                                                         float *__restrict__ rstds, int batch, int features) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= batch) return;
  const int nv = features >> 2;
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)row * features);
  const float4 *yr = reinterpret_cast<const float4 *>(y + (size_t)row * features);
  float4 v[V];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < nv ? xr[c] : splat4(0.f);
    if (y != nullptr && c < nv) {
      const float4 yv = yr[c];
      v[i] = make_float4(v[i].x + yv.x, v[i].y + yv.y, v[i].z + yv.z, v[i].w + yv.w);
    }
    s += hsum4(v[i]);
  }
  if (sum_out != nullptr) {
    float4 *sr = reinterpret_cast<float4 *>(sum_out + (size_t)row * features);
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (lane + 64 * i < nv) sr[lane + 64 * i] = v[i];
  }
  const float mean = wave_sum(s) / (float)features;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    if (lane + 64 * i < nv) {
      const float4 d = make_float4(v[i].x - mean, v[i].y - mean, v[i].z - mean, v[i].w - mean);
      q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
    }
  }
  const float rstd = 1.f / sqrtf(wave_sum(q) / (float)features + kLnEps);
  if (lane == 0) {
    if (means) means[row] = mean;
    if (rstds) rstds[row] = rstd;
  }
  float4 *orow = reinterpret_cast<float4 *>(out + (size_t)row * features);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = lane + 64 * i;
    if (c < nv) {
      const float4 g = gamma ? reinterpret_cast<const float4 *>(gamma)[c] : splat4(1.f);
      const float4 b = beta ? reinterpret_cast<const float4 *>(beta)[c] : splat4(0.f);
      orow[c] = make_float4((v[i].x - mean) * rstd * g.x + b.x, (v[i].y - mean) * rstd * g.y + b.y,
                            (v[i].z - mean) * rstd * g.z + b.z, (v[i].w - mean) * rstd * g.w + b.w);
    }
  }
}

// Any width and 4-byte alignment: one wave per row, three passes over the
// row (it stays in the caches between them).
__global__ __launch_bounds__(256) void ln_fwd_generic_kernel(const float *__restrict__ x, const float *__restrict__ y,
                                                             const float *__restrict__ gamma,
                                                             const float *__restrict__ beta, float *__restrict__ sum_out,
                                                             float *__restrict__ out, float *__restrict__ means,
                                                             float *__restrict__ rstds, int batch, int features) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= batch) return;
  const float *xr = x + (size_t)row * features;
  const float *yr = y + (size_t)row * features;
  auto val = [&](int c) { return y != nullptr ? xr[c] + yr[c] : xr[c]; };
  float s = 0.f;
  for (int c = lane; c < features; c += 64) s += val(c);
  const float mean = wave_sum(s) / (float)features;
  float q = 0.f;
  for (int c = lane; c < features; c += 64) {
    const float d = val(c) - mean;
    q += d * d;
  }
  const float rstd = 1.f / sqrtf(wave_sum(q) / (float)features + kLnEps);
  if (lane == 0) {
    if (means) means[row] = mean;
    if (rstds) rstds[row] = rstd;
  }
  float *orow = out + (size_t)row * features;
  for (int c = lane; c < features; c += 64) {
    const float v = val(c);
    if (sum_out != nullptr) sum_out[(size_t)row * features + c] = v;
    orow[c] = (v - mean) * rstd * (gamma ? gamma[c] : 1.f) + (beta ? beta[c] : 0.f);
  }
}

// ------------------------------------------------------ LayerNorm backward, dx
// grad_x = rstd / F * (F ds - sum(ds) - x_hat sum(ds x_hat)), ds = grad_out *
// gamma (layernorm.cu:126-178). One wave per row, row in registers.
// With residual: grad_x = that + residual (a residual connection's gradient
// added in the same pass, one fp32 add per value).
template <int V>
__global__ __launch_bounds__(256) void ln_bwd_dx_vec_kernel(const float *__restrict__ dout, const float *__restrict__ x,
                                                            const float *__restrict__ gamma,
                                                            const float *__restrict__ means,
                                                            const float *__restrict__ rstds,
                                                            const float *__restrict__ residual, float *__restrict__ grad_x,
                                                            int batch, int features) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= batch) return;
  const int nv = features >> 2;
  const float mean = means[row], rstd = rstds[row];
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)row * features);
  const float4 *dr = reinterpret_cast<const float4 *>(dout + (size_t)row * features);
  float4 xh[V], ds[V];
  float sds = 0.f, sdsx = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = lane + 64 * i;
    xh[i] = ds[i] = splat4(0.f);
    if (c < nv) {
      const float4 xv = xr[c], dv = dr[c];
      const float4 g = gamma ? reinterpret_cast<const float4 *>(gamma)[c] : splat4(1.f);
      xh[i] = make_float4((xv.x - mean) * rstd, (xv.y - mean) * rstd, (xv.z - mean) * rstd, (xv.w - mean) * rstd);
      ds[i] = make_float4(dv.x * g.x, dv.y * g.y, dv.z * g.z, dv.w * g.w);
      sds += hsum4(ds[i]);
      sdsx += (ds[i].x * xh[i].x + ds[i].y * xh[i].y) + (ds[i].z * xh[i].z + ds[i].w * xh[i].w);
    }
  }
  const float sum_ds = wave_sum(sds), sum_dsx = wave_sum(sdsx);
  const float f = (float)features, k = rstd / f;
  float4 *gr = reinterpret_cast<float4 *>(grad_x + (size_t)row * features);
  const float4 *rr = reinterpret_cast<const float4 *>(residual + (size_t)row * features);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = lane + 64 * i;
    if (c < nv) {
      float4 o = make_float4(k * (f * ds[i].x - sum_ds - xh[i].x * sum_dsx), k * (f * ds[i].y - sum_ds - xh[i].y * sum_dsx),
                             k * (f * ds[i].z - sum_ds - xh[i].z * sum_dsx), k * (f * ds[i].w - sum_ds - xh[i].w * sum_dsx));
      if (residual != nullptr) {
        const float4 r = rr[c];
        o = make_float4(o.x + r.x, o.y + r.y, o.z + r.z, o.w + r.w);
      }
      gr[c] = o;
    }
  }
}

__global__ __launch_bounds__(256) void ln_bwd_dx_generic_kernel(const float *__restrict__ dout,
                                                                const float *__restrict__ x,
                                                                const float *__restrict__ gamma,
                                                                const float *__restrict__ means,
                                                                const float *__restrict__ rstds,
                                                                const float *__restrict__ residual,
                                                                float *__restrict__ grad_x, int batch, int features) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= batch) return;
  const float mean = means[row], rstd = rstds[row];
  const float *xr = x + (size_t)row * features, *dr = dout + (size_t)row * features;
  float sds = 0.f, sdsx = 0.f;
  for (int c = lane; c < features; c += 64) {
    const float xh = (xr[c] - mean) * rstd, ds = dr[c] * (gamma ? gamma[c] : 1.f);
    sds += ds;
    sdsx += ds * xh;
  }
  const float sum_ds = wave_sum(sds), sum_dsx = wave_sum(sdsx);
  const float f = (float)features, k = rstd / f;
  float *gr = grad_x + (size_t)row * features;
  for (int c = lane; c < features; c += 64) {
    const float xh = (xr[c] - mean) * rstd, ds = dr[c] * (gamma ? gamma[c] : 1.f);
    const float o = k * (f * ds - sum_ds - xh * sum_dsx);
    gr[c] = residual != nullptr ? o + residual[(size_t)row * features + c] : o;
  }
}

// ------------------------------------ LayerNorm backward with its column sums
// ln_bwd_dx_vec_kernel's grad_x (the same arithmetic, so the same values),
// plus each workgroup's partial column sums of grad_out * x_hat and grad_out
// (the parameter gradients' terms) and, when `planes` is 3, of grad_x itself
// (the bias gradient of the linear layer whose output gradient grad_x is):
// per lane over its row, then the four rows added in wave order through LDS,
// into partial[blockIdx.x][plane][features]. colsum_partials_kernel adds the
// workgroups' partials in order. The rows are read once for all of it.
template <int V>
__global__ __launch_bounds__(256) void ln_bwd_fused_kernel(const float *__restrict__ dout, const float *__restrict__ x,
                                                           const float *__restrict__ gamma,
                                                           const float *__restrict__ means,
                                                           const float *__restrict__ rstds,
                                                           const float *__restrict__ residual,
                                                           float *__restrict__ grad_x, float *__restrict__ partial,
                                                           int planes, int batch, int features) {
  __shared__ __attribute__((aligned(16))) float part[4][3][V * 256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + wave;
  const bool ok = row < batch;
  const int nv = features >> 2;
  const float mean = ok ? means[row] : 0.f, rstd = ok ? rstds[row] : 0.f;
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)row * features);
  const float4 *dr = reinterpret_cast<const float4 *>(dout + (size_t)row * features);
  float4 xh[V], ds[V], dv[V];
  float sds = 0.f, sdsx = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = lane + 64 * i;
    xh[i] = ds[i] = dv[i] = splat4(0.f);
    if (ok && c < nv) {
      const float4 xv = xr[c];
      dv[i] = dr[c];
      const float4 g = gamma ? reinterpret_cast<const float4 *>(gamma)[c] : splat4(1.f);
      xh[i] = make_float4((xv.x - mean) * rstd, (xv.y - mean) * rstd, (xv.z - mean) * rstd, (xv.w - mean) * rstd);
      ds[i] = make_float4(dv[i].x * g.x, dv[i].y * g.y, dv[i].z * g.z, dv[i].w * g.w);
      sds += hsum4(ds[i]);
      sdsx += (ds[i].x * xh[i].x + ds[i].y * xh[i].y) + (ds[i].z * xh[i].z + ds[i].w * xh[i].w);
    }
  }
  const float sum_ds = wave_sum(sds), sum_dsx = wave_sum(sdsx);
  const float f = (float)features, k = rstd / f;
  float4 *gr = reinterpret_cast<float4 *>(grad_x + (size_t)row * features);
  const float4 *rr = reinterpret_cast<const float4 *>(residual + (size_t)row * features);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int c = lane + 64 * i;
    float4 o = splat4(0.f);
    if (ok && c < nv) {
      o = make_float4(k * (f * ds[i].x - sum_ds - xh[i].x * sum_dsx), k * (f * ds[i].y - sum_ds - xh[i].y * sum_dsx),
                      k * (f * ds[i].z - sum_ds - xh[i].z * sum_dsx), k * (f * ds[i].w - sum_ds - xh[i].w * sum_dsx));
      if (residual != nullptr) {
        const float4 r = rr[c];
        o = make_float4(o.x + r.x, o.y + r.y, o.z + r.z, o.w + r.w);
      }
      gr[c] = o;
    }
    if (c < nv) {
      *reinterpret_cast<float4 *>(&part[wave][0][4 * c]) =
          make_float4(dv[i].x * xh[i].x, dv[i].y * xh[i].y, dv[i].z * xh[i].z, dv[i].w * xh[i].w);
      *reinterpret_cast<float4 *>(&part[wave][1][4 * c]) = dv[i];
      *reinterpret_cast<float4 *>(&part[wave][2][4 * c]) = o;
    }
  }
  __syncthreads();
  float *dst = partial + (size_t)blockIdx.x * planes * features;
  for (int j = threadIdx.x; j < planes * features; j += 256) {
    const int plane = j / features, c = j - plane * features;
    dst[j] = ((part[0][plane][c] + part[1][plane][c]) + part[2][plane][c]) + part[3][plane][c];
  }
}

// out_p[c] = sum over the n_parts workgroups' partial[w][p][c] (p < planes,
// out_p NULL: not written): 16 slices of consecutive workgroups, each added
// in order, then the slices in order; 16 columns of one plane per workgroup.
__global__ __launch_bounds__(256) void colsum_partials_kernel(const float *__restrict__ partial, int n_parts,
                                                              int planes, int features, float *__restrict__ out0,
                                                              float *__restrict__ out1, float *__restrict__ out2) {
  __shared__ float acc[16][17];
  const int t = threadIdx.x, col16 = t & 15, slice = t >> 4;
  const int j = blockIdx.x * 16 + col16;  // flattened plane * features + c
  const int per = (n_parts + 15) / 16;
  const int w0 = slice * per, w1 = min(n_parts, w0 + per);
  const size_t stride = (size_t)planes * features;
  // Up to 16 independent loads in flight per thread, then added in order.
  float s = 0.f;
  if (j < planes * features)
    for (int wb = w0; wb < w1; wb += 16) {
      float v[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) v[k] = wb + k < w1 ? partial[(size_t)(wb + k) * stride + j] : 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) s += v[k];
    }
  acc[slice][col16] = s;
  __syncthreads();
  if (t < 16 && j < planes * features) {
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < 16; ++q) tot += acc[q][t];
    const int plane = j / features, c = j - plane * features;
    float *o = plane == 0 ? out0 : (plane == 1 ? out1 : out2);
    if (o != nullptr) o[c] = tot;
  }
}

// ------------------------------------------------------------- column sums
// Sums over the rows of a [rows, cols] row-major matrix g, kColStrip = 16
// columns per workgroup of 1024 threads (48 workgroups at 768 columns): lane
// l of wave w reads columns 4(l%4) .. +3 (float4) of rows r = 16w + l/4 +
// 256k (k = 0, 1, ...) and adds them in increasing k; the 256 row slots are
// then added through LDS in two fixed stages (contiguous groups of slots,
// then the groups in order), so every sum has one order and is reproducible.
// LN (the LayerNorm parameter gradients): out0 receives the sums of
// g * x_hat, x_hat = (x - means[r]) * rstds[r], and out1 those of g;
// otherwise out0 receives the sums of g (the bias gradient). accumulate:
// out += sums, else out = sums. cols % 4 == 0 and 16-byte aligned rows.
constexpr int kColStrip = 16;
constexpr int kRowSlots = 256;  // 16 waves x 16 rows per load
template <bool LN>
__global__ __launch_bounds__(1024) void colsum_vec_kernel(const float *__restrict__ g, const float *__restrict__ x,
                                                          const float *__restrict__ means,
                                                          const float *__restrict__ rstds, float *__restrict__ out0,
                                                          float *__restrict__ out1, int rows, int cols,
                                                          int accumulate) {
  constexpr int kPlanes = LN ? 2 : 1;
  constexpr int kGroups = 64 / kPlanes;            // stage-1 groups per plane and column
  constexpr int kPerGroup = kRowSlots / kGroups;  // slots per group
  __shared__ __attribute__((aligned(16))) float part[kPlanes][kRowSlots][kColStrip];
  __shared__ float grp[kPlanes][kGroups][kColStrip];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int slot = 16 * w + (lane >> 2);
  const int c4 = lane & 3;
  const int col = blockIdx.x * kColStrip + 4 * c4;
  float4 a0 = splat4(0.f), a1 = splat4(0.f);
  if (col < cols) {
#pragma unroll 4
    for (int r = slot; r < rows; r += kRowSlots) {
      const float4 gv = *reinterpret_cast<const float4 *>(g + (size_t)r * cols + col);
      if constexpr (LN) {
        const float4 xv = *reinterpret_cast<const float4 *>(x + (size_t)r * cols + col);
        const float mu = means[r], rs = rstds[r];
        a0.x += gv.x * ((xv.x - mu) * rs);
        a0.y += gv.y * ((xv.y - mu) * rs);
        a0.z += gv.z * ((xv.z - mu) * rs);
        a0.w += gv.w * ((xv.w - mu) * rs);
        a1.x += gv.x;
        a1.y += gv.y;
        a1.z += gv.z;
        a1.w += gv.w;
      } else {
        a0.x += gv.x;
        a0.y += gv.y;
        a0.z += gv.z;
        a0.w += gv.w;
      }
    }
  }
  *reinterpret_cast<float4 *>(&part[0][slot][4 * c4]) = a0;
  if constexpr (LN) *reinterpret_cast<float4 *>(&part[kPlanes - 1][slot][4 * c4]) = a1;
  __syncthreads();
  {
    // Stage 1: thread t adds slots kPerGroup*j .. +kPerGroup-1 of column t%16 (j = group).
    const int c = tid % kColStrip, j = (tid / kColStrip) % kGroups, plane = tid / (kColStrip * kGroups);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kPerGroup; ++k) s += part[plane][kPerGroup * j + k][c];
    grp[plane][j][c] = s;
  }
  __syncthreads();
  if (tid < kPlanes * kColStrip) {
    const int plane = tid / kColStrip, t = tid % kColStrip;
    const int c = blockIdx.x * kColStrip + t;
    float *o = plane ? out1 : out0;
    if (c < cols && o != nullptr) {
      float s = 0.f;
      for (int j = 0; j < kGroups; ++j) s += grp[plane][j][t];
      o[c] = accumulate ? o[c] + s : s;
    }
  }
}

// Any width and 4-byte alignment: one thread per column, rows in order.
template <bool LN>
__global__ __launch_bounds__(256) void colsum_generic_kernel(const float *__restrict__ g, const float *__restrict__ x,
                                                             const float *__restrict__ means,
                                                             const float *__restrict__ rstds, float *__restrict__ out0,
                                                             float *__restrict__ out1, int rows, int cols,
                                                             int accumulate) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  float s0 = 0.f, s1 = 0.f;
  for (int r = 0; r < rows; ++r) {
    const float gv = g[(size_t)r * cols + c];
    if constexpr (LN) {
      s0 += gv * ((x[(size_t)r * cols + c] - means[r]) * rstds[r]);
      s1 += gv;
    } else {
      s0 += gv;
    }
  }
  if (out0) out0[c] = accumulate ? out0[c] + s0 : s0;
  if constexpr (LN) {
    if (out1) out1[c] = accumulate ? out1[c] + s1 : s1;
  }
}

// ------------------------------------------------------------------- GELU
__device__ __forceinline__ float gelu_f(float v) {
  return 0.5f * v * (1.f + tanhf(kGeluK0 * (v + kGeluK1 * v * v * v)));
}
__device__ __forceinline__ float gelu_grad(float go, float v) {
  const float t = tanhf(kGeluK0 * (v + kGeluK1 * v * v * v));
  const float d_inner = kGeluK0 * (1.f + 3.f * kGeluK1 * v * v);
  return go * (0.5f * (1.f + t) + 0.5f * v * (1.f - t * t) * d_inner);
}

// out = gelu(x) (BWD: out = go * gelu'(x)); grid-stride over float4 groups
// when every pointer is 16-byte aligned, the n % 4 tail by the first threads.
template <bool BWD>
__global__ __launch_bounds__(256) void gelu_kernel(const float *__restrict__ go, const float *__restrict__ x,
                                                   float *__restrict__ out, size_t n, int vec) {
  const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, stride = (size_t)gridDim.x * 256;
  size_t done = 0;
  if (vec) {
    const size_t n4 = n / 4;
    for (size_t i = tid; i < n4; i += stride) {
      const float4 v = reinterpret_cast<const float4 *>(x)[i];
      float4 r;
      if constexpr (BWD) {
        const float4 gv = reinterpret_cast<const float4 *>(go)[i];
        r = make_float4(gelu_grad(gv.x, v.x), gelu_grad(gv.y, v.y), gelu_grad(gv.z, v.z), gelu_grad(gv.w, v.w));
      } else {
        r = make_float4(gelu_f(v.x), gelu_f(v.y), gelu_f(v.z), gelu_f(v.w));
      }
      reinterpret_cast<float4 *>(out)[i] = r;
    }
    done = n4 * 4;
  }
  for (size_t i = done + tid; i < n; i += stride) {
    if constexpr (BWD)
      out[i] = gelu_grad(go[i], x[i]);
    else
      out[i] = gelu_f(x[i]);
  }
}

// The reference step's plain elementwise launchers (elementwise.cu:48-124,
// 229-250), one fp32 operation per value: OP 0 c = a + b, 1 c = alpha * a,
// 2 c = alpha, 3 c = a + b[column] (b a bias over rows of `cols` values).
// Grid-stride over float4 groups when `vec` (every pointer 16-byte aligned
// and, for the bias, cols % 4 == 0), value by value otherwise; c may be a.
template <int OP>
__global__ __launch_bounds__(256) void ew_kernel(const float *a, const float *__restrict__ b, float *c, float alpha,
                                                 size_t n, int cols, int vec) {
  const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, stride = (size_t)gridDim.x * 256;
  auto op = [&](float x, float y) {
    if constexpr (OP == 0 || OP == 3) return x + y;
    else if constexpr (OP == 1) return alpha * x;
    else return alpha;
  };
  size_t done = 0;
  if (vec) {
    const size_t n4 = n / 4;
    const size_t c4 = (size_t)cols / 4;
    for (size_t i = tid; i < n4; i += stride) {
      const float4 x = OP == 2 ? splat4(0.f) : reinterpret_cast<const float4 *>(a)[i];
      const float4 y = OP == 0   ? reinterpret_cast<const float4 *>(b)[i]
                       : OP == 3 ? reinterpret_cast<const float4 *>(b)[i % c4]
                                 : splat4(0.f);
      reinterpret_cast<float4 *>(c)[i] = make_float4(op(x.x, y.x), op(x.y, y.y), op(x.z, y.z), op(x.w, y.w));
    }
    done = n4 * 4;
  }
  for (size_t i = done + tid; i < n; i += stride) {
    const float x = OP == 2 ? 0.f : a[i];
    const float y = OP == 0 ? b[i] : (OP == 3 ? b[i % (size_t)cols] : 0.f);
    c[i] = op(x, y);
  }
}

// h = h + bias (bias broadcast over rows of `cols` values, written back: the
// backward's GELU input) and out = gelu(h), in one pass over [rows, cols].
// vec: cols % 4 == 0 and 16-byte aligned tensors.
__global__ __launch_bounds__(256) void bias_gelu_kernel(float *__restrict__ h, const float *__restrict__ bias,
                                                        float *__restrict__ out, size_t n, int cols, int vec) {
  const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, stride = (size_t)gridDim.x * 256;
  if (vec) {
    const size_t n4 = n / 4;
    const int c4 = cols / 4;
    for (size_t i = tid; i < n4; i += stride) {
      float4 v = reinterpret_cast<const float4 *>(h)[i];
      const float4 b = reinterpret_cast<const float4 *>(bias)[i % c4];
      v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
      reinterpret_cast<float4 *>(h)[i] = v;
      reinterpret_cast<float4 *>(out)[i] = make_float4(gelu_f(v.x), gelu_f(v.y), gelu_f(v.z), gelu_f(v.w));
    }
    return;
  }
  for (size_t i = tid; i < n; i += stride) {
    const float v = h[i] + bias[i % cols];
    h[i] = v;
    out[i] = gelu_f(v);
  }
}

// ------------------------------------------------------------------ AdamW
// matmul.cu:285-339: m = b1 m + (1-b1) g, v = b2 v + (1-b2) g^2,
// p = p (1 - lr wd) - lr m_hat / (sqrt(v_hat) + eps).
__device__ __forceinline__ void adamw1(float &p, float &m, float &v, float g, float lr, float b1, float b2,
                                       float eps, float decay, float bc1, float bc2) {
  m = b1 * m + (1.f - b1) * g;
  v = b2 * v + (1.f - b2) * (g * g);
  p = p * decay - lr * (m / bc1) / (sqrtf(v / bc2) + eps);
}

// step != nullptr: the bias corrections come from t = *step + 1 on the device.
// vec: each thread updates float4 groups i and i + 256 of its workgroup's 512
// (every load of both issued before the arithmetic), the n % 4 tail by the
// first workgroup; otherwise one value per thread.
constexpr int kAdamGroups = 2;
// Each value is read and written once per step: streaming (nontemporal)
// accesses, which do not keep the 2 GB the update moves in the caches.
typedef float stream4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 stream_load4(const float *base, size_t i) {
  return __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const stream4_t *>(base) + i));
}
__device__ __forceinline__ void stream_store4(float *base, size_t i, float4 x) {
  __builtin_nontemporal_store(__builtin_bit_cast(stream4_t, x), reinterpret_cast<stream4_t *>(base) + i);
}
__global__ __launch_bounds__(256) void adamw_kernel(float *__restrict__ p, float *__restrict__ m,
                                                    float *__restrict__ v, const float *__restrict__ g, size_t n,
                                                    float lr, float b1, float b2, float eps, float wd, float bc1,
                                                    float bc2, const float *__restrict__ step, int vec) {
  if (step != nullptr) {
    const float t = *step + 1.f;
    bc1 = 1.f - powf(b1, t);
    bc2 = 1.f - powf(b2, t);
  }
  const float decay = 1.f - lr * wd;
  if (!vec) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) adamw1(p[i], m[i], v[i], g[i], lr, b1, b2, eps, decay, bc1, bc2);
    return;
  }
  const size_t n4 = n / 4;
  const size_t base = (size_t)blockIdx.x * (256 * kAdamGroups) + threadIdx.x;
  float4 pp[kAdamGroups], mm[kAdamGroups], vv[kAdamGroups], gg[kAdamGroups];
#pragma unroll
  for (int k = 0; k < kAdamGroups; ++k) {
    const size_t i = base + 256 * k;
    if (i < n4) {
      pp[k] = stream_load4(p, i);
      mm[k] = stream_load4(m, i);
      vv[k] = stream_load4(v, i);
      gg[k] = stream_load4(g, i);
    }
  }
#pragma unroll
  for (int k = 0; k < kAdamGroups; ++k) {
    const size_t i = base + 256 * k;
    if (i < n4) {
      adamw1(pp[k].x, mm[k].x, vv[k].x, gg[k].x, lr, b1, b2, eps, decay, bc1, bc2);
      adamw1(pp[k].y, mm[k].y, vv[k].y, gg[k].y, lr, b1, b2, eps, decay, bc1, bc2);
      adamw1(pp[k].z, mm[k].z, vv[k].z, gg[k].z, lr, b1, b2, eps, decay, bc1, bc2);
      adamw1(pp[k].w, mm[k].w, vv[k].w, gg[k].w, lr, b1, b2, eps, decay, bc1, bc2);
      stream_store4(p, i, pp[k]);
      stream_store4(m, i, mm[k]);
      stream_store4(v, i, vv[k]);
    }
  }
  if (blockIdx.x == 0) {
    const size_t i = n4 * 4 + threadIdx.x;
    if (i < n) adamw1(p[i], m[i], v[i], g[i], lr, b1, b2, eps, decay, bc1, bc2);
  }
}

// Workgroups of the AdamW kernel over n values.
unsigned adamw_blocks(size_t n, int vec) {
  const size_t per = vec ? (size_t)256 * kAdamGroups * 4 : 256;
  const size_t b = (n + per - 1) / per;
  return (unsigned)(b < 1 ? 1 : b);
}

__global__ void step_advance_kernel(float *step) {
  if (threadIdx.x == 0) *step += 1.f;
}

// ------------------------------------------------------------------- host
bool al(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int launched(const char *fn) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return DFATTN_OK;
  return record_error(DFATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(err));
}

int check_ptrs(const char *fn, std::initializer_list<const void *> required,
               std::initializer_list<const void *> optional) {
  for (const void *p : required)
    if (p == nullptr) return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null pointer");
  for (const void *p : required)
    if (!al(p, 4)) return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": pointer not 4-byte aligned");
  for (const void *p : optional)
    if (p != nullptr && !al(p, 4))
      return record_error(DFATTN_ERR_MISALIGNED, std::string(fn) + ": pointer not 4-byte aligned");
  return DFATTN_OK;
}

int check_dims(const char *fn, uint32_t rows, uint32_t cols) {
  if (cols == 0) return record_error(DFATTN_ERR_SHAPE, std::string(fn) + ": features must be >= 1");
  if (rows > (uint32_t)INT_MAX || cols > (uint32_t)INT_MAX)
    return record_error(DFATTN_ERR_OVERFLOW, std::string(fn) + ": shape is too large");
  return DFATTN_OK;
}

// Grid of a grid-stride elementwise kernel: 256 threads, four values each.
unsigned elementwise_blocks(size_t n) {
  const size_t b = (n / 4 + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 4096 ? 4096 : b));
}

template <int V>
void launch_ln_fwd_v(const float *x, const float *y, const float *gamma, const float *beta, float *sum_out, float *out,
                     float *means, float *rstds, int batch, int features, hipStream_t stream) {
  hipLaunchKernelGGL(ln_fwd_vec_kernel<V>, dim3((batch + 3) / 4), dim3(256), 0, stream, x, y, gamma, beta, sum_out,
                     out, means, rstds, batch, features);
}

template <int V>
void launch_ln_dx_v(const float *dout, const float *x, const float *gamma, const float *means, const float *rstds,
                    const float *residual, float *grad_x, int batch, int features, hipStream_t stream) {
  hipLaunchKernelGGL(ln_bwd_dx_vec_kernel<V>, dim3((batch + 3) / 4), dim3(256), 0, stream, dout, x, gamma, means,
                     rstds, residual, grad_x, batch, features);
}

// LayerNorm forward of x (+ y, stored to sum_out) on the register-resident
// path when it applies, else the generic one.
void ln_forward(const float *x, const float *y, const float *gamma, const float *beta, float *sum_out, float *out,
                float *means, float *rstds, int b, int f, hipStream_t stream);
// LayerNorm backward's grad_x (+ residual).
void ln_backward_dx(const float *dout, const float *x, const float *gamma, const float *means, const float *rstds,
                    const float *residual, float *grad_x, int b, int f, hipStream_t stream);

// The register-resident row path: features % 4 == 0, at most 1024, 16-byte
// aligned tensors.
bool ln_vec(uint32_t features, std::initializer_list<const void *> ptrs) {
  if (features % 4 != 0 || features > 1024) return false;
  for (const void *p : ptrs)
    if (p != nullptr && !al(p, 16)) return false;
  return true;
}

void ln_forward(const float *x, const float *y, const float *gamma, const float *beta, float *sum_out, float *out,
                float *means, float *rstds, int b, int f, hipStream_t stream) {
  if (ln_vec((uint32_t)f, {x, y, out, sum_out, gamma, beta})) {
    switch ((f / 4 + 63) / 64) {
      case 1: launch_ln_fwd_v<1>(x, y, gamma, beta, sum_out, out, means, rstds, b, f, stream); break;
      case 2: launch_ln_fwd_v<2>(x, y, gamma, beta, sum_out, out, means, rstds, b, f, stream); break;
      case 3: launch_ln_fwd_v<3>(x, y, gamma, beta, sum_out, out, means, rstds, b, f, stream); break;
      default: launch_ln_fwd_v<4>(x, y, gamma, beta, sum_out, out, means, rstds, b, f, stream); break;
    }
  } else {
    hipLaunchKernelGGL(ln_fwd_generic_kernel, dim3((b + 3) / 4), dim3(256), 0, stream, x, y, gamma, beta, sum_out, out,
                       means, rstds, b, f);
  }
}

void ln_backward_dx(const float *dout, const float *x, const float *gamma, const float *means, const float *rstds,
                    const float *residual, float *grad_x, int b, int f, hipStream_t stream) {
  if (ln_vec((uint32_t)f, {dout, x, gamma, residual, grad_x})) {
    switch ((f / 4 + 63) / 64) {
      case 1: launch_ln_dx_v<1>(dout, x, gamma, means, rstds, residual, grad_x, b, f, stream); break;
      case 2: launch_ln_dx_v<2>(dout, x, gamma, means, rstds, residual, grad_x, b, f, stream); break;
      case 3: launch_ln_dx_v<3>(dout, x, gamma, means, rstds, residual, grad_x, b, f, stream); break;
      default: launch_ln_dx_v<4>(dout, x, gamma, means, rstds, residual, grad_x, b, f, stream); break;
    }
  } else {
    hipLaunchKernelGGL(ln_bwd_dx_generic_kernel, dim3((b + 3) / 4), dim3(256), 0, stream, dout, x, gamma, means, rstds,
                       residual, grad_x, b, f);
  }
}

template <bool LN>
void launch_colsum(const float *g, const float *x, const float *means, const float *rstds, float *out0, float *out1,
                   int rows, int cols, int accumulate, bool vec, hipStream_t stream) {
  if (vec)
    hipLaunchKernelGGL(colsum_vec_kernel<LN>, dim3((cols + kColStrip - 1) / kColStrip), dim3(1024), 0, stream, g, x,
                       means, rstds, out0, out1, rows, cols, accumulate);
  else
    hipLaunchKernelGGL(colsum_generic_kernel<LN>, dim3((cols + 255) / 256), dim3(256), 0, stream, g, x, means,
                       rstds, out0, out1, rows, cols, accumulate);
}

}  // namespace
}  // namespace dfattn

using namespace dfattn;

extern "C" int dfgpt2_layernorm_forward(const float *x, const float *gamma, const float *beta, float *out,
                                        float *means, float *rstds, uint32_t batch, uint32_t features,
                                        hipStream_t stream) {
  const char *fn = "dfgpt2_layernorm_forward";
  if (int st = check_dims(fn, batch, features); st != DFATTN_OK) return st;
  if (batch == 0) return DFATTN_OK;  // no rows: nothing to read or write
  if (int st = check_ptrs(fn, {x, out}, {gamma, beta, means, rstds}); st != DFATTN_OK) return st;
  ln_forward(x, nullptr, gamma, beta, nullptr, out, means, rstds, (int)batch, (int)features, stream);
  return launched(fn);
}

extern "C" int dfgpt2_add_layernorm_forward(const float *x, const float *y, const float *gamma, const float *beta,
                                            float *sum_out, float *out, float *means, float *rstds, uint32_t batch,
                                            uint32_t features, hipStream_t stream) {
  const char *fn = "dfgpt2_add_layernorm_forward";
  if (int st = check_dims(fn, batch, features); st != DFATTN_OK) return st;
  if (batch == 0) return DFATTN_OK;
  if (int st = check_ptrs(fn, {x, y, sum_out, out}, {gamma, beta, means, rstds}); st != DFATTN_OK) return st;
  ln_forward(x, y, gamma, beta, sum_out, out, means, rstds, (int)batch, (int)features, stream);
  return launched(fn);
}

// grad_x, then the parameter gradients (added into grad_gamma / grad_beta, or
// written when !accumulate) by the fixed-order column sums.
static int ln_backward(const char *fn, const float *grad_out, const float *x, const float *gamma, const float *means,
                       const float *rstds, const float *residual, float *grad_x, float *grad_gamma, float *grad_beta,
                       int accumulate, uint32_t batch, uint32_t features, hipStream_t stream) {
  const int b = (int)batch, f = (int)features;
  ln_backward_dx(grad_out, x, gamma, means, rstds, residual, grad_x, b, f, stream);
  if (int st = launched(fn); st != DFATTN_OK) return st;
  if (grad_gamma == nullptr && grad_beta == nullptr) return DFATTN_OK;
  const bool vec = f % 4 == 0 && al(grad_out, 16) && al(x, 16);
  launch_colsum<true>(grad_out, x, means, rstds, grad_gamma, grad_beta, b, f, accumulate, vec, stream);
  return launched(fn);
}

extern "C" int dfgpt2_layernorm_backward(const float *grad_out, const float *x, const float *gamma,
                                         const float *means, const float *rstds, float *grad_x, float *grad_gamma,
                                         float *grad_beta, uint32_t batch, uint32_t features, hipStream_t stream) {
  const char *fn = "dfgpt2_layernorm_backward";
  if (int st = check_dims(fn, batch, features); st != DFATTN_OK) return st;
  if (batch == 0) return DFATTN_OK;  // no rows: grad_x is empty and nothing is added
  if (int st = check_ptrs(fn, {grad_out, x, means, rstds, grad_x}, {gamma, grad_gamma, grad_beta}); st != DFATTN_OK)
    return st;
  return ln_backward(fn, grad_out, x, gamma, means, rstds, nullptr, grad_x, grad_gamma, grad_beta, 1, batch, features,
                     stream);
}

extern "C" int dfgpt2_layernorm_backward_residual(const float *grad_out, const float *x, const float *gamma,
                                                  const float *means, const float *rstds, const float *residual,
                                                  float *grad_x, float *grad_gamma, float *grad_beta, uint32_t batch,
                                                  uint32_t features, hipStream_t stream) {
  const char *fn = "dfgpt2_layernorm_backward_residual";
  if (int st = check_dims(fn, batch, features); st != DFATTN_OK) return st;
  if (batch == 0) return DFATTN_OK;
  if (int st = check_ptrs(fn, {grad_out, x, means, rstds, grad_x}, {gamma, residual, grad_gamma, grad_beta});
      st != DFATTN_OK)
    return st;
  return ln_backward(fn, grad_out, x, gamma, means, rstds, residual, grad_x, grad_gamma, grad_beta, 0, batch, features,
                     stream);
}

extern "C" size_t dfgpt2_layernorm_backward_fused_workspace_bytes(uint32_t batch, uint32_t features) {
  return (size_t)((batch + 3) / 4) * 3 * features * sizeof(float);
}

template <int V>
void launch_ln_fused_v(const float *dout, const float *x, const float *gamma, const float *means, const float *rstds,
                       const float *residual, float *grad_x, float *partial, int planes, int batch, int features,
                       hipStream_t stream) {
  hipLaunchKernelGGL(ln_bwd_fused_kernel<V>, dim3((batch + 3) / 4), dim3(256), 0, stream, dout, x, gamma, means,
                     rstds, residual, grad_x, partial, planes, batch, features);
}

extern "C" int dfgpt2_layernorm_backward_fused(const float *grad_out, const float *x, const float *gamma,
                                               const float *means, const float *rstds, const float *residual,
                                               float *grad_x, float *grad_gamma, float *grad_beta, float *grad_bias,
                                               void *workspace, size_t workspace_bytes, uint32_t batch,
                                               uint32_t features, hipStream_t stream) {
  const char *fn = "dfgpt2_layernorm_backward_fused";
  if (int st = check_dims(fn, batch, features); st != DFATTN_OK) return st;
  if (batch == 0) return DFATTN_OK;
  if (int st = check_ptrs(fn, {grad_out, x, means, rstds, grad_x}, {gamma, residual, grad_gamma, grad_beta, grad_bias});
      st != DFATTN_OK)
    return st;
  const int b = (int)batch, f = (int)features;
  const bool sums = grad_gamma != nullptr || grad_beta != nullptr || grad_bias != nullptr;
  if (!sums || !ln_vec(features, {grad_out, x, gamma, residual, grad_x})) {
    // Any width and alignment: the separate launches, the same results contract.
    ln_backward_dx(grad_out, x, gamma, means, rstds, residual, grad_x, b, f, stream);
    if (int st = launched(fn); st != DFATTN_OK || !sums) return st;
    if (grad_gamma != nullptr || grad_beta != nullptr)
      launch_colsum<true>(grad_out, x, means, rstds, grad_gamma, grad_beta, b, f, 0,
                          f % 4 == 0 && al(grad_out, 16) && al(x, 16), stream);
    if (grad_bias != nullptr)
      launch_colsum<false>(grad_x, nullptr, nullptr, nullptr, grad_bias, nullptr, b, f, 0,
                           f % 4 == 0 && al(grad_x, 16), stream);
    return launched(fn);
  }
  const int planes = grad_bias != nullptr ? 3 : 2;
  const size_t need = (size_t)((batch + 3) / 4) * planes * features * sizeof(float);
  if (workspace == nullptr || workspace_bytes < need || !al(workspace, 4))
    return record_error(DFATTN_ERR_WORKSPACE, std::string(fn) + ": workspace must be non-null, 4-byte aligned and hold " +
                                                  std::to_string(need) + " bytes");
  float *partial = static_cast<float *>(workspace);
  switch ((f / 4 + 63) / 64) {
    case 1: launch_ln_fused_v<1>(grad_out, x, gamma, means, rstds, residual, grad_x, partial, planes, b, f, stream); break;
    case 2: launch_ln_fused_v<2>(grad_out, x, gamma, means, rstds, residual, grad_x, partial, planes, b, f, stream); break;
    case 3: launch_ln_fused_v<3>(grad_out, x, gamma, means, rstds, residual, grad_x, partial, planes, b, f, stream); break;
    default: launch_ln_fused_v<4>(grad_out, x, gamma, means, rstds, residual, grad_x, partial, planes, b, f, stream); break;
  }
  if (int st = launched(fn); st != DFATTN_OK) return st;
  hipLaunchKernelGGL(colsum_partials_kernel, dim3((planes * f + 15) / 16), dim3(256), 0, stream, partial,
                     (b + 3) / 4, planes, f, grad_gamma, grad_beta, grad_bias);
  return launched(fn);
}

namespace dfattn {
namespace {
template <int OP>
void launch_ew(const float *a, const float *b, float *c, float alpha, size_t n, int cols, bool vec,
               hipStream_t stream) {
  hipLaunchKernelGGL(ew_kernel<OP>, dim3(elementwise_blocks(n)), dim3(256), 0, stream, a, b, c, alpha, n, cols,
                     vec ? 1 : 0);
}
}  // namespace
}  // namespace dfattn

extern "C" int dfgpt2_add_bias(const float *input, const float *bias, float *out, uint32_t batch, uint32_t features,
                               hipStream_t stream) {
  const char *fn = "dfgpt2_add_bias";
  if (int st = check_dims(fn, batch, features); st != DFATTN_OK) return st;
  if (batch == 0) return DFATTN_OK;
  if (int st = check_ptrs(fn, {input, bias, out}, {}); st != DFATTN_OK) return st;
  const size_t n = (size_t)batch * features;
  launch_ew<3>(input, bias, out, 0.f, n, (int)features, features % 4 == 0 && al(input, 16) && al(bias, 16) && al(out, 16),
               stream);
  return launched(fn);
}

extern "C" int dfgpt2_gelu_forward(const float *x, float *out, size_t n, hipStream_t stream) {
  const char *fn = "dfgpt2_gelu_forward";
  if (n == 0) return DFATTN_OK;
  if (int st = check_ptrs(fn, {x, out}, {}); st != DFATTN_OK) return st;
  hipLaunchKernelGGL(gelu_kernel<false>, dim3(elementwise_blocks(n)), dim3(256), 0, stream, nullptr, x, out, n,
                     (al(x, 16) && al(out, 16)) ? 1 : 0);
  return launched(fn);
}

extern "C" int dfgpt2_gelu_backward(const float *grad_out, const float *x, float *grad_x, size_t n,
                                    hipStream_t stream) {
  const char *fn = "dfgpt2_gelu_backward";
  if (n == 0) return DFATTN_OK;
  if (int st = check_ptrs(fn, {grad_out, x, grad_x}, {}); st != DFATTN_OK) return st;
  hipLaunchKernelGGL(gelu_kernel<true>, dim3(elementwise_blocks(n)), dim3(256), 0, stream, grad_out, x, grad_x, n,
                     (al(grad_out, 16) && al(x, 16) && al(grad_x, 16)) ? 1 : 0);
  return launched(fn);
}

extern "C" int dfgpt2_bias_gelu_forward(float *h, const float *bias, float *out, uint32_t rows, uint32_t cols,
                                        hipStream_t stream) {
  const char *fn = "dfgpt2_bias_gelu_forward";
  if (int st = check_dims(fn, rows, cols); st != DFATTN_OK) return st;
  if (rows == 0) return DFATTN_OK;
  if (int st = check_ptrs(fn, {h, bias, out}, {}); st != DFATTN_OK) return st;
  const size_t n = (size_t)rows * cols;
  const int vec = (cols % 4 == 0 && al(h, 16) && al(bias, 16) && al(out, 16)) ? 1 : 0;
  hipLaunchKernelGGL(bias_gelu_kernel, dim3(elementwise_blocks(n)), dim3(256), 0, stream, h, bias, out, n, (int)cols,
                     vec);
  return launched(fn);
}

extern "C" int dfgpt2_linear_grad_bias(const float *grad_out, float *grad_bias, uint32_t batch,
                                       uint32_t out_features, int accumulate, hipStream_t stream) {
  const char *fn = "dfgpt2_linear_grad_bias";
  // No rows: grad_out may be empty (NULL) and the sums are zero.
  if (int st = check_ptrs(fn, {grad_bias}, {grad_out}); st != DFATTN_OK) return st;
  if (batch > 0 && grad_out == nullptr) return record_error(DFATTN_ERR_NULL_POINTER, std::string(fn) + ": null pointer");
  if (int st = check_dims(fn, batch, out_features); st != DFATTN_OK) return st;
  const bool vec = out_features % 4 == 0 && al(grad_out, 16);
  launch_colsum<false>(grad_out, nullptr, nullptr, nullptr, grad_bias, nullptr, (int)batch, (int)out_features,
                       accumulate ? 1 : 0, vec, stream);
  return launched(fn);
}

extern "C" int dfgpt2_adamw_update(float *parameter, float *first_moment, float *second_moment,
                                   const float *gradient, size_t n, float lr, float beta1, float beta2, float eps,
                                   float weight_decay, float *step, hipStream_t stream) {
  const char *fn = "dfgpt2_adamw_update";
  if (int st = check_ptrs(fn, {parameter, first_moment, second_moment, gradient, step}, {}); st != DFATTN_OK)
    return st;
  const int vec = (al(parameter, 16) && al(first_moment, 16) && al(second_moment, 16) && al(gradient, 16)) ? 1 : 0;
  if (n > 0) {
    hipLaunchKernelGGL(adamw_kernel, dim3(adamw_blocks(n, vec)), dim3(256), 0, stream, parameter, first_moment,
                       second_moment, gradient, n, lr, beta1, beta2, eps, weight_decay, 1.f, 1.f, step, vec);
    if (int st = launched(fn); st != DFATTN_OK) return st;
  }
  hipLaunchKernelGGL(step_advance_kernel, dim3(1), dim3(64), 0, stream, step);
  return launched(fn);
}

// ------------------------------------------------- the reference's symbols
extern "C" void launch_layernorm(const float *x, const float *gamma, const float *beta, float *out, float *means,
                                 float *rstds, uint32_t batch, uint32_t features) {
  mark_pending(dfgpt2_layernorm_forward(x, gamma, beta, out, means, rstds, batch, features, nullptr));
}

extern "C" void launch_layernorm_backward(const float *grad_out, const float *x, const float *gamma,
                                          const float *means, const float *rstds, float *grad_x, float *grad_gamma,
                                          float *grad_beta, uint32_t batch, uint32_t features) {
  mark_pending(dfgpt2_layernorm_backward(grad_out, x, gamma, means, rstds, grad_x, grad_gamma, grad_beta, batch,
                                         features, nullptr));
}

// elementwise.cu:242 (null stream; out may be input).
extern "C" void launch_add_bias(const float *input, const float *bias, float *out, uint32_t batch,
                                uint32_t features) {
  mark_pending(dfgpt2_add_bias(input, bias, out, batch, features, nullptr));
}

// elementwise.cu:62, 91, 119: fill, add and scale of n values (null stream).
extern "C" void launch_fill(float *c, float val, uint32_t n) {
  int st = DFATTN_OK;
  if (n > 0) {
    st = check_ptrs("launch_fill", {c}, {});
    if (st == DFATTN_OK) {
      launch_ew<2>(nullptr, nullptr, c, val, n, 1, al(c, 16), nullptr);
      st = launched("launch_fill");
    }
  }
  mark_pending(st);
}

extern "C" void launch_add(const float *a, const float *b, float *c, uint32_t n) {
  int st = DFATTN_OK;
  if (n > 0) {
    st = check_ptrs("launch_add", {a, b, c}, {});
    if (st == DFATTN_OK) {
      launch_ew<0>(a, b, c, 0.f, n, 1, al(a, 16) && al(b, 16) && al(c, 16), nullptr);
      st = launched("launch_add");
    }
  }
  mark_pending(st);
}

extern "C" void launch_scale(const float *a, float alpha, float *c, uint32_t n) {
  int st = DFATTN_OK;
  if (n > 0) {
    st = check_ptrs("launch_scale", {a, c}, {});
    if (st == DFATTN_OK) {
      launch_ew<1>(a, nullptr, c, alpha, n, 1, al(a, 16) && al(c, 16), nullptr);
      st = launched("launch_scale");
    }
  }
  mark_pending(st);
}

extern "C" void launch_gelu(const float *x, float *out, uint32_t n) {
  mark_pending(dfgpt2_gelu_forward(x, out, n, nullptr));
}

extern "C" void launch_gelu_backward(const float *grad_out, const float *x, float *grad_x, uint32_t n) {
  mark_pending(dfgpt2_gelu_backward(grad_out, x, grad_x, n, nullptr));
}

extern "C" void launch_linear_grad_bias(const float *grad_out, float *grad_bias, uint32_t batch,
                                        uint32_t out_features) {
  mark_pending(dfgpt2_linear_grad_bias(grad_out, grad_bias, batch, out_features, 0, nullptr));
}

extern "C" void launch_adamw_update(float *parameter, float *first_moment, float *second_moment,
                                    const float *gradient, uint32_t n, float lr, float beta1, float beta2, float eps,
                                    float weight_decay, float bias_correction1, float bias_correction2) {
  const char *fn = "launch_adamw_update";
  int st = check_ptrs(fn, {parameter, first_moment, second_moment, gradient}, {});
  if (st == DFATTN_OK && n > 0) {
    const int vec = (al(parameter, 16) && al(first_moment, 16) && al(second_moment, 16) && al(gradient, 16)) ? 1 : 0;
    hipLaunchKernelGGL(adamw_kernel, dim3(adamw_blocks(n, vec)), dim3(256), 0, nullptr, parameter, first_moment,
                       second_moment, gradient, (size_t)n, lr, beta1, beta2, eps, weight_decay, bias_correction1,
                       bias_correction2, nullptr, vec);
    st = launched(fn);
  }
  mark_pending(st);
}
