// attn_decode.hip — single-query attention against a KV cache (autoregressive
// decode), gfx950.
//
// Reference: attention_fused.cu:551-615 (kernel_fused_mha_decode_kv), 622-745
// (split-K kernel and its reduction), 800-1090 (paged pools, fp32 and bf16).
// Per head h and cached keys t = 0 .. L-1 (row t of the cache, or of the pool
// through the block table): out = softmax_t(scale * q.k_t) . v_t, computed as
// an online softmax; nothing is written when L is 0.
//
// The work is split over the key range: workgroup (h, c) takes keys
// [c*chunk, min(L, (c+1)*chunk)) and either writes the normalised output
// (one chunk) or the chunk's partial (m, l, unnormalised o) in the reference's
// split-K layout (m, l: [H, n_chunks]; o: [H, n_chunks, D]), which
// decode_reduce_kernel merges with the logsumexp identity.
//
// decode_d64_kernel (D = 64, the GPT-2 shape; fp32 or bf16 cache, contiguous
// or paged): 8 waves; each wave takes 64-key groups. Its loads are coalesced
// rows: lane l reads 4 values (16 bytes fp32, 8 bytes bf16) of row
// 4j + l/16 of the group at column 4*(l%16), for j = 0..15, K and V alike.
// The score of a row is reduced over its 16 lanes, gathered through LDS so
// that lane r holds key r for the softmax, and P goes back through LDS to
// the V lanes. decode_generic_kernel handles every other D (1..128): one wave
// per workgroup, lanes over d, one key at a time.
#include "dfattn_internal.h"

#include <hip/hip_runtime.h>

namespace dfattn {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kDecWaves = 8;
constexpr int kDecThreads = 64 * kDecWaves;

struct DecodeArgs {
  const float *q;            // [H*D]
  const void *k, *v;         // rows of H*D values (fp32, or bf16 bit patterns)
  const int32_t *table;      // logical page -> physical block; null: contiguous cache
  int page_size;
  int H, L, D;
  float scale;
  int chunk, n_chunks;
  float *out, *lse;                  // n_chunks == 1
  float *part_m, *part_l, *part_o;   // n_chunks > 1
};

__device__ __forceinline__ size_t cache_row(const DecodeArgs &a, int t) {
  if (a.table == nullptr) return (size_t)t;
  return (size_t)a.table[t / a.page_size] * (size_t)a.page_size + (size_t)(t % a.page_size);
}

__device__ __forceinline__ float bf16_bits_to_float(unsigned short b) {
  return __builtin_bit_cast(float, (unsigned)b << 16);
}

// 4 consecutive values of a cache row: the raw bits (fp32: the floats; bf16:
// four bf16 in the low 8 bytes), loaded without conversion so that every
// load of a group is issued before the first wait, and widened later. A
// call reads each cache row once, and a long cache is larger than the
// caches: the loads are nontemporal (streaming), which measured 10-11 %
// faster at 131072 rows than cached loads.
typedef unsigned raw2_t __attribute__((ext_vector_type(2)));
typedef unsigned raw4_t __attribute__((ext_vector_type(4)));
template <bool BF16>
__device__ __forceinline__ uint4 load4_raw(const void *base, size_t elem) {
  if constexpr (BF16) {
    const raw2_t u = __builtin_nontemporal_load(
        reinterpret_cast<const raw2_t *>(reinterpret_cast<const unsigned short *>(base) + elem));
    return make_uint4(u.x, u.y, 0u, 0u);
  } else {
    const raw4_t u =
        __builtin_nontemporal_load(reinterpret_cast<const raw4_t *>(reinterpret_cast<const float *>(base) + elem));
    return make_uint4(u.x, u.y, u.z, u.w);
  }
}
template <bool BF16>
__device__ __forceinline__ float4 widen4(uint4 r) {
  if constexpr (BF16)
    return make_float4(__builtin_bit_cast(float, r.x << 16), __builtin_bit_cast(float, r.x & 0xffff0000u),
                       __builtin_bit_cast(float, r.y << 16), __builtin_bit_cast(float, r.y & 0xffff0000u));
  else
    return __builtin_bit_cast(float4, r);
}

// Sum over each row of 16 lanes, in every lane of the row: DPP rotations
// within the row (row_ror:8, 4, 2, 1), full-rate VALU instead of LDS-pipe
// permutes.
__device__ __forceinline__ float row16_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x122, 0xf, 0xf, false));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x121, 0xf, 0xf, false));
  return x;
}

template <bool BF16>
__device__ __forceinline__ float load1(const void *base, size_t elem) {
  if constexpr (BF16)
    return bf16_bits_to_float(reinterpret_cast<const unsigned short *>(base)[elem]);
  else
    return reinterpret_cast<const float *>(base)[elem];
}

// Writes one chunk's (m, l, o) — m and the scores in the log2 domain — as the
// normalised output and logsumexp (one chunk) or as the chunk's partial in the
// reference's layout (m converted to the natural-log domain).
__device__ __forceinline__ void write_chunk(const DecodeArgs &a, int h, int c, int d, float m2, float l,
                                            float o) {
  if (a.n_chunks == 1) {
    a.out[(size_t)h * a.D + d] = l > 0.f ? o / l : 0.f;
    if (d == 0 && a.lse) a.lse[h] = l > 0.f ? (m2 + __builtin_log2f(l)) * kLn2 : -INFINITY;
  } else {
    const size_t slot = (size_t)h * a.n_chunks + c;
    a.part_o[slot * a.D + d] = o;
    if (d == 0) {
      a.part_m[slot] = m2 * kLn2;
      a.part_l[slot] = l;
    }
  }
}

template <bool BF16, bool PAGED>
__global__ __launch_bounds__(kDecThreads) void decode_d64_kernel(DecodeArgs a) {
  __shared__ float s_lds[kDecWaves][64];   // scores, then P, of the wave's group
  __shared__ unsigned row_lds[kDecWaves][64];  // paged: the group's physical rows
  __shared__ float m_lds[kDecWaves], l_lds[kDecWaves];
  __shared__ float o_lds[kDecWaves][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane >> 4, dq = lane & 15;  // row 4j + sub of a group, columns 4*dq .. +3
  const int h = blockIdx.x / a.n_chunks, c = blockIdx.x % a.n_chunks;
  const int t0 = c * a.chunk, t1 = min(a.L, t0 + a.chunk);
  const size_t dm = (size_t)a.H * 64;
  const size_t col = (size_t)h * 64 + 4 * dq;
  const float4 q4 = *reinterpret_cast<const float4 *>(a.q + col);
  const float c2 = a.scale * kLog2e;

  float m = -INFINITY, l = 0.f;
  float4 o4 = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int g0 = t0 + 64 * wave; g0 < t1; g0 += 64 * kDecWaves) {
    // This wave's group: keys g0 .. g0+63 (those below t1). Paged: lane r
    // looks up the physical row of key g0 + r once, for every lane.
    if constexpr (PAGED) {
      const int t = min(g0 + lane, t1 - 1);
      row_lds[wave][lane] = (unsigned)cache_row(a, t);
      __builtin_amdgcn_wave_barrier();
    }
    // Rows past t1 read row t1-1 instead (their P is 0), so every load is
    // unconditional.
    uint4 kr[16], vr[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int t = min(g0 + 4 * j + sub, t1 - 1);
      const size_t row = PAGED ? (size_t)row_lds[wave][min(4 * j + sub, t1 - 1 - g0)] : (size_t)t;
      const size_t e = row * dm + col;
      kr[j] = load4_raw<BF16>(a.k, e);
      vr[j] = load4_raw<BF16>(a.v, e);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float4 k4 = widen4<BF16>(kr[j]);
      const float s = row16_sum(q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w);
      if (dq == 0) s_lds[wave][4 * j + sub] = s;
    }
    __builtin_amdgcn_wave_barrier();
    // Online softmax over the group, lane r = key g0 + r.
    const bool valid = g0 + lane < t1;
    const float s2 = valid ? s_lds[wave][lane] * c2 : -INFINITY;
    const float m_new = fmaxf(m, wave_max(s2));
    const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - m_new);
    const float p = valid ? __builtin_amdgcn_exp2f(s2 - m_new) : 0.f;
    l = l * alpha + p;
    m = m_new;
    __builtin_amdgcn_wave_barrier();
    s_lds[wave][lane] = p;
    __builtin_amdgcn_wave_barrier();
    o4.x *= alpha;
    o4.y *= alpha;
    o4.z *= alpha;
    o4.w *= alpha;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float pj = s_lds[wave][4 * j + sub];
      const float4 v4 = widen4<BF16>(vr[j]);
      o4.x += pj * v4.x;
      o4.y += pj * v4.y;
      o4.z += pj * v4.z;
      o4.w += pj * v4.w;
    }
    __builtin_amdgcn_wave_barrier();
  }
  // The wave's (m, l, o): l summed over lanes, o over the four row groups.
  l = wave_sum(l);
#pragma unroll
  for (int off = 16; off < 64; off <<= 1) {
    o4.x += __shfl_xor(o4.x, off, 64);
    o4.y += __shfl_xor(o4.y, off, 64);
    o4.z += __shfl_xor(o4.z, off, 64);
    o4.w += __shfl_xor(o4.w, off, 64);
  }
  if (lane == 0) {
    m_lds[wave] = m;
    l_lds[wave] = l;
  }
  if (sub == 0) *reinterpret_cast<float4 *>(&o_lds[wave][4 * dq]) = o4;
  __syncthreads();
  if (wave == 0) {
    // Merge the waves (a wave with no keys has m = -inf and weight 0).
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) mm = fmaxf(mm, m_lds[w]);
    float ll = 0.f, oo = 0.f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const float f = m_lds[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_lds[w] - mm);
      ll += f * l_lds[w];
      oo += f * o_lds[w][lane];
    }
    write_chunk(a, h, c, lane, mm, ll, oo);
  }
}

// Any D in 1..128: one wave per workgroup, lane d holds columns d and d+64,
// keys one at a time (the reference's order of work, wave64 wide).
template <bool BF16>
__global__ __launch_bounds__(64) void decode_generic_kernel(DecodeArgs a) {
  const int lane = threadIdx.x;
  const int h = blockIdx.x / a.n_chunks, c = blockIdx.x % a.n_chunks;
  const int t0 = c * a.chunk, t1 = min(a.L, t0 + a.chunk);
  const int D = a.D;
  const size_t dm = (size_t)a.H * D, hoff = (size_t)h * D;
  const bool in0 = lane < D, in1 = lane + 64 < D;
  const float q0 = in0 ? a.q[hoff + lane] : 0.f, q1 = in1 ? a.q[hoff + lane + 64] : 0.f;
  const float c2 = a.scale * kLog2e;
  float m = -INFINITY, l = 0.f, o0 = 0.f, o1 = 0.f;
  for (int t = t0; t < t1; ++t) {
    const size_t base = cache_row(a, t) * dm + hoff;
    float s = 0.f;
    if (in0) s += q0 * load1<BF16>(a.k, base + lane);
    if (in1) s += q1 * load1<BF16>(a.k, base + lane + 64);
    s = wave_sum(s) * c2;
    const float m_new = fmaxf(m, s);
    const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - m_new);
    const float p = __builtin_amdgcn_exp2f(s - m_new);
    l = l * alpha + p;
    m = m_new;
    o0 = o0 * alpha + (in0 ? p * load1<BF16>(a.v, base + lane) : 0.f);
    o1 = o1 * alpha + (in1 ? p * load1<BF16>(a.v, base + lane + 64) : 0.f);
  }
  if (in0) write_chunk(a, h, c, lane, m, l, o0);
  if (in1) write_chunk(a, h, c, lane + 64, m, l, o1);
}

// Merges the split-K partials of one head (attention_fused.cu:712-757):
// m = max_c m_c, l = sum_c l_c exp(m_c - m), out = sum_c exp(m_c - m) o_c / l.
// Chunks whose m_c is not above -FLT_MAX hold no key and are skipped. 512
// threads per head: the chunks are strided over the threads (and, for o,
// over 8 groups of 64 columns), so the partial loads are independent of each
// other instead of one chained loop.
constexpr int kRedThreads = 512;
__device__ __forceinline__ float block_reduce(float v, float *scratch, bool is_max) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = is_max ? wave_max(v) : wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
#pragma unroll
  for (int w = 1; w < kRedThreads / 64; ++w) r = is_max ? fmaxf(r, scratch[w]) : r + scratch[w];
  return r;
}

__global__ __launch_bounds__(kRedThreads) void decode_reduce_kernel(const float *__restrict__ part_m,
                                                                    const float *__restrict__ part_l,
                                                                    const float *__restrict__ part_o,
                                                                    float *__restrict__ out, float *__restrict__ lse,
                                                                    int n_chunks, int D) {
  __shared__ float scratch[kRedThreads / 64];
  __shared__ float w_lds[kRedThreads];
  __shared__ float acc_lds[kRedThreads / 64][128];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, grp = tid >> 6;
  constexpr int kGroups = kRedThreads / 64;
  constexpr int kPre = 8;  // o values a lane loads before the weights are known
  const float *pm = part_m + (size_t)h * n_chunks;
  const float *pl = part_l + (size_t)h * n_chunks;
  const float *po = part_o + (size_t)h * n_chunks * D;
  constexpr float kNoKey = -3.402823466e38f;  // -FLT_MAX, the reference's empty-chunk mark
  // Every load of the first kRedThreads chunks is issued at once: thread c
  // takes chunk c's (m, l); lane d of group g takes o[c][d] of chunks
  // c = g + 8i, i < kPre.
  const bool mine = tid < n_chunks;
  const float m_c = mine ? pm[tid] : -INFINITY, l_c = mine ? pl[tid] : 0.f;
  float o0[kPre], o1[kPre];
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const int cc = grp + kGroups * i;
    o0[i] = cc < n_chunks && lane < D ? po[(size_t)cc * D + lane] : 0.f;
    o1[i] = cc < n_chunks && lane + 64 < D ? po[(size_t)cc * D + lane + 64] : 0.f;
  }
  float mm = m_c;
  for (int cc = tid + kRedThreads; cc < n_chunks; cc += kRedThreads) mm = fmaxf(mm, pm[cc]);
  mm = block_reduce(mm, scratch, true);
  const float w_c = m_c > kNoKey ? __expf(m_c - mm) : 0.f;
  w_lds[tid] = w_c;
  float ll = w_c * l_c;
  for (int cc = tid + kRedThreads; cc < n_chunks; cc += kRedThreads)
    if (pm[cc] > kNoKey) ll += pl[cc] * __expf(pm[cc] - mm);
  ll = block_reduce(ll, scratch, false);  // (its barriers also publish w_lds)
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const int cc = grp + kGroups * i;
    if (cc < kRedThreads) {
      a0 += w_lds[cc] * o0[i];
      a1 += w_lds[cc] * o1[i];
    }
  }
  for (int cc = grp + kGroups * kPre; cc < n_chunks; cc += kGroups) {
    const float m2 = pm[cc];
    const float w = cc < kRedThreads ? w_lds[cc] : (m2 > kNoKey ? __expf(m2 - mm) : 0.f);
    if (lane < D) a0 += w * po[(size_t)cc * D + lane];
    if (lane + 64 < D) a1 += w * po[(size_t)cc * D + lane + 64];
  }
  acc_lds[grp][lane] = a0;
  acc_lds[grp][lane + 64] = a1;
  __syncthreads();
  if (grp == 0) {
    const float inv = ll > 0.f ? 1.f / ll : 0.f;
    for (int d = lane; d < D; d += 64) {
      float o = 0.f;
#pragma unroll
      for (int g = 0; g < kGroups; ++g) o += acc_lds[g][d];
      out[(size_t)h * D + d] = o * inv;
    }
    if (lane == 0 && lse) lse[h] = ll > 0.f ? mm + __logf(ll) : -INFINITY;
  }
}

}  // namespace

hipError_t launch_decode(const float *q, const void *k, const void *v, const int32_t *block_table,
                         int page_size, bool bf16, float *out, float *lse, int n_heads, int cur_len,
                         int d_head, float scale, int chunk, float *part_m, float *part_l, float *part_o,
                         bool fast, hipStream_t stream) {
  DecodeArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.table = block_table;
  a.page_size = page_size > 0 ? page_size : 1;
  a.H = n_heads;
  a.L = cur_len;
  a.D = d_head;
  a.scale = scale;
  a.chunk = chunk >= cur_len || part_m == nullptr ? cur_len : chunk;
  a.n_chunks = (cur_len + a.chunk - 1) / a.chunk;
  a.out = out;
  a.lse = lse;
  a.part_m = part_m;
  a.part_l = part_l;
  a.part_o = part_o;
  const unsigned grid = (unsigned)(n_heads * a.n_chunks);
  if (fast && d_head == 64) {
    const bool paged = block_table != nullptr;
    if (bf16 && paged)
      hipLaunchKernelGGL((decode_d64_kernel<true, true>), dim3(grid), dim3(kDecThreads), 0, stream, a);
    else if (bf16)
      hipLaunchKernelGGL((decode_d64_kernel<true, false>), dim3(grid), dim3(kDecThreads), 0, stream, a);
    else if (paged)
      hipLaunchKernelGGL((decode_d64_kernel<false, true>), dim3(grid), dim3(kDecThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((decode_d64_kernel<false, false>), dim3(grid), dim3(kDecThreads), 0, stream, a);
  } else {
    if (bf16)
      hipLaunchKernelGGL(decode_generic_kernel<true>, dim3(grid), dim3(64), 0, stream, a);
    else
      hipLaunchKernelGGL(decode_generic_kernel<false>, dim3(grid), dim3(64), 0, stream, a);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || a.n_chunks == 1) return err;
  hipLaunchKernelGGL(decode_reduce_kernel, dim3((unsigned)n_heads), dim3(kRedThreads), 0, stream, part_m, part_l,
                     part_o, out, lse, a.n_chunks, d_head);
  return hipGetLastError();
}

}  // namespace dfattn
