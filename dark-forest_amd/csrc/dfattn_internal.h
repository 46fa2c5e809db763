// dfattn_internal.h — shared device helpers and the internal launch API of
// the gfx950 attention kernels. Not installed; the public ABI is
// include/dfattn.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dfattn {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// D = 64 fast path: one 32x32x16 fp16 MFMA (fp32 accumulate). Operand
// convention used by every kernel here: for A (M x K) lane l holds row
// m = l % 32 and the 8 contraction slots k = 8*(l/32) + j, j = 0..7; for B
// (K x N) lane l holds column n = l % 32 and the same 8 slots. The result C
// (32 x 32, 16 fp32 per lane) has column n = l % 32 and row
// m = 8*(r/4) + 4*(l/32) + r%4 in register r. Which physical k the
// hardware assigns to a slot does not matter as long as A and B agree, and
// they always do because both are built with the same slot -> k map.
__device__ __forceinline__ f32x16 mfma32x32x16(half8_t a, half8_t b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);  // v_exp_f32; exp2(-inf) = 0
}

__device__ __forceinline__ half4_t to_half4(float4 v) {
  half4_t h;
  h[0] = (half_t)v.x;
  h[1] = (half_t)v.y;
  h[2] = (half_t)v.z;
  h[3] = (half_t)v.w;
  return h;
}

__device__ __forceinline__ float4 scale4(float4 v, float s) {
  return make_float4(v.x * s, v.y * s, v.z * s, v.w * s);
}

__device__ __forceinline__ float4 load4_or_zero(const float *p, bool ok) {
  return ok ? *reinterpret_cast<const float4 *>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// ---- internal launch API (host side, all asynchronous on `stream`) -------

// Forward, D = 64, MFMA. q/k/v/o 16-byte aligned. lse may be null.
hipError_t launch_fwd_d64(const float *q, const float *k, const float *v, float *o,
                          float *lse, int n_heads, int seq_len, float scale, bool causal,
                          hipStream_t stream);

// Backward, D = 64, MFMA. Needs bwd_workspace_bytes_d64() of workspace.
size_t bwd_workspace_bytes_d64(int n_heads, int seq_len);
hipError_t launch_bwd_d64(const float *q, const float *k, const float *v, const float *o,
                          const float *d_o, const float *lse, float *d_q, float *d_k,
                          float *d_v, void *workspace, int n_heads, int seq_len, float scale,
                          bool causal, hipStream_t stream);
// The two phases of launch_bwd_d64: Delta/dO-range/dQ:=0, then the main kernel.
hipError_t launch_bwd_pre_d64(const float *o, const float *d_o, float *d_q, void *workspace,
                              int n_heads, int seq_len, hipStream_t stream);
hipError_t launch_bwd_main_d64(const float *q, const float *k, const float *v, const float *d_o,
                               const float *lse, float *d_q, float *d_k, float *d_v,
                               const void *workspace, int n_heads, int seq_len, float scale,
                               bool causal, hipStream_t stream);

// Generic fp32 kernels for any d_head in 1..=128 and any 4-byte alignment.
// The backward recomputes everything it needs per row and uses no workspace.
hipError_t launch_fwd_generic(const float *q, const float *k, const float *v, float *o,
                              float *lse, int n_heads, int seq_len, int d_head, float scale,
                              bool causal, hipStream_t stream);
hipError_t launch_bwd_generic(const float *q, const float *k, const float *v,
                              const float *d_o, float *d_q, float *d_k, float *d_v,
                              int n_heads, int seq_len, int d_head, float scale, bool causal,
                              hipStream_t stream);

}  // namespace dfattn
