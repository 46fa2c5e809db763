// attn_aux.hip — the elementwise kernels that share the reference's attention
// object file (attention_fused.cu:1098-1231), so that this library replaces
// that object as a unit: position-embedding interpolation, rotary position
// embedding of one row, and the paged KV pool's row writes (fp32 and bf16).
//
// All are one row of d_model (or H*d_head) values: memory-latency bound,
// one thread per value (per pair for RoPE), 256 threads per workgroup.
// Products and sums are not contracted into FMAs, so interpolation and the
// bf16 rounding are bit-exact against a plain fp32 restatement; RoPE
// differs from one only through powf, cosf and sinf.
#include "dfattn_internal.h"

#include <hip/hip_runtime.h>

namespace dfattn {
namespace {

constexpr int kAuxThreads = 256;

// attention_fused.cu:1098-1121. Inside the trained range the row is copied;
// otherwise position pos*(trained-1)/(max-1) is interpolated linearly between
// rows p0 = floor and min(p0+1, trained-1). Where the reference would read
// past the table (p0 >= trained, i.e. pos beyond max_ctx_len - 1) the last
// row is returned instead; every in-range position gives the reference's
// arithmetic unchanged.
__global__ __launch_bounds__(kAuxThreads) void pos_embed_interpolate_kernel(const float *__restrict__ table,
                                                                            float *__restrict__ out, unsigned pos,
                                                                            unsigned trained, unsigned max_ctx,
                                                                            unsigned d_model) {
#pragma clang fp contract(off)
  const unsigned idx = blockIdx.x * kAuxThreads + threadIdx.x;
  if (idx >= d_model) return;
  if (pos < trained && max_ctx <= trained) {
    out[idx] = table[(size_t)pos * d_model + idx];
  } else {
    const float scale = (float)(trained - 1) / (float)(max_ctx - 1);
    const float p_scaled = (float)pos * scale;
    unsigned p0 = (unsigned)p_scaled;
    float alpha = p_scaled - (float)p0;
    if (p0 >= trained) p0 = trained - 1, alpha = 0.0f;
    const unsigned p1 = p0 + 1 < trained ? p0 + 1 : trained - 1;
    const float v0 = table[(size_t)p0 * d_model + idx];
    const float v1 = table[(size_t)p1 * d_model + idx];
    out[idx] = (1.0f - alpha) * v0 + alpha * v1;
  }
}

// attention_fused.cu:1136-1158: pair (2i, 2i+1) of every head rotated by
// pos * base^(-2i/d_head), in place; thread = (head, pair).
__global__ __launch_bounds__(kAuxThreads) void apply_rope_kernel(float *__restrict__ qk, unsigned pos,
                                                                 unsigned n_heads, unsigned d_head, float base) {
#pragma clang fp contract(off)
  const unsigned pairs = d_head / 2;
  const size_t t = (size_t)blockIdx.x * kAuxThreads + threadIdx.x;
  if (t >= (size_t)n_heads * pairs) return;
  const unsigned h = (unsigned)(t / pairs), i = (unsigned)(t % pairs);
  const float theta = powf(base, -2.0f * (float)i / (float)d_head);
  const float angle = (float)pos * theta;
  const float c = cosf(angle), s = sinf(angle);
  const size_t i0 = (size_t)h * d_head + 2 * i;
  const float x0 = qk[i0], x1 = qk[i0 + 1];
  qk[i0] = x0 * c - x1 * s;
  qk[i0 + 1] = x0 * s + x1 * c;
}

// fp32 -> bf16 bits, round to nearest even (NaN stays a quiet NaN).
__device__ __forceinline__ unsigned short f32_to_bf16_rne(float f) {
  const unsigned u = __builtin_bit_cast(unsigned, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);
  return (unsigned short)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// attention_fused.cu:1179-1231: row `page_offset` of physical block
// `phys_block` of a [blocks * page_size, d_model] pool := src.
template <bool BF16>
__global__ __launch_bounds__(kAuxThreads) void paged_copy_row_kernel(const float *__restrict__ src, void *pool,
                                                                     int phys_block, unsigned page_offset,
                                                                     unsigned page_size, unsigned d_model) {
  const unsigned idx = blockIdx.x * kAuxThreads + threadIdx.x;
  if (idx >= d_model) return;
  const size_t dst = ((size_t)phys_block * page_size + page_offset) * d_model + idx;
  if constexpr (BF16)
    reinterpret_cast<unsigned short *>(pool)[dst] = f32_to_bf16_rne(src[idx]);
  else
    reinterpret_cast<float *>(pool)[dst] = src[idx];
}

unsigned blocks_for(size_t n) { return (unsigned)((n + kAuxThreads - 1) / kAuxThreads); }

}  // namespace

hipError_t launch_pos_embed_interpolate(const float *table, float *out, unsigned pos, unsigned trained,
                                        unsigned max_ctx, unsigned d_model, hipStream_t stream) {
  hipLaunchKernelGGL(pos_embed_interpolate_kernel, dim3(blocks_for(d_model)), dim3(kAuxThreads), 0, stream, table,
                     out, pos, trained, max_ctx, d_model);
  return hipGetLastError();
}

hipError_t launch_apply_rope(float *qk, unsigned pos, unsigned n_heads, unsigned d_head, float base,
                             hipStream_t stream) {
  const size_t n = (size_t)n_heads * (d_head / 2);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(apply_rope_kernel, dim3(blocks_for(n)), dim3(kAuxThreads), 0, stream, qk, pos, n_heads, d_head,
                     base);
  return hipGetLastError();
}

hipError_t launch_paged_copy_row(const float *src, void *pool, bool bf16, int phys_block, unsigned page_offset,
                                 unsigned page_size, unsigned d_model, hipStream_t stream) {
  if (bf16)
    hipLaunchKernelGGL(paged_copy_row_kernel<true>, dim3(blocks_for(d_model)), dim3(kAuxThreads), 0, stream, src,
                       pool, phys_block, page_offset, page_size, d_model);
  else
    hipLaunchKernelGGL(paged_copy_row_kernel<false>, dim3(blocks_for(d_model)), dim3(kAuxThreads), 0, stream, src,
                       pool, phys_block, page_offset, page_size, d_model);
  return hipGetLastError();
}

}  // namespace dfattn
