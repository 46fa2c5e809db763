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
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
// Word 3 of a raw buffer descriptor (gfx9 family: 32-bit data format, no
// swizzle); loads past num_records return zeros.
constexpr int kBufferFlags = 0x00020000;

// Direct-to-LDS fetch: 16 bytes per lane from the buffer (descriptor in
// scalar registers, see sgpr_rsrc) at byte offset voff into LDS at
// lds_addr + 16 * lane (lds_addr uniform across the wave). The data bypasses
// the registers; the wave's vmcnt counts the fetch until it has landed in
// LDS. The instruction is issued through asm so that the compiler does not
// see an LDS write: it would otherwise wait for every fetch in flight before
// the next LDS read it cannot prove disjoint (the transposing reads), which
// defeats the prefetch. The caller synchronises with lds_fetch_barrier; the
// compiler's own vmcnt waits for its loads can only over-count these.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 sgpr_rsrc(const void *p, unsigned nrec) {
  const unsigned long long addr = reinterpret_cast<unsigned long long>(p);
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane((int)(unsigned)addr);
  r.y = __builtin_amdgcn_readfirstlane((int)((unsigned)(addr >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane((int)nrec);
  r.w = kBufferFlags;
  return r;
}
// LDS address of p as a wave-uniform 32-bit value (the caller guarantees
// uniformity across the wave; readfirstlane puts it in a scalar register).
__device__ __forceinline__ unsigned lds_addr32(const unsigned char *p) {
  return __builtin_amdgcn_readfirstlane(
      (unsigned)reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) unsigned char *)p));
}
// M0 is reserved to the compiler, which warns that it is not restored after
// the asm; these kernels use M0 for nothing else.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_fetch16(i32x4 rsrc, unsigned lds_addr, int voff) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(voff), "s"(lds_addr), "s"(rsrc)
               : "memory", "m0");
}
// The same for 4 bytes per lane (LDS at lds_addr + 4 * lane).
__device__ __forceinline__ void lds_fetch4(i32x4 rsrc, unsigned lds_addr, int voff) {
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dword %0, %2, 0 offen lds" ::"v"(voff), "s"(lds_addr), "s"(rsrc)
               : "memory", "m0");
}
#pragma clang diagnostic pop
// Workgroup barrier after this wave's LDS writes and all but its N most
// recent vector-memory operations have completed: with direct-to-LDS
// fetches in flight, N of them (the prefetches of later tiles) may stay
// outstanding across the barrier. The compiler's own barrier waits for
// every vector-memory operation.
template <int N>
__device__ __forceinline__ void lds_fetch_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Raw buffer descriptor over nrec bytes from p. The kernels build descriptors
// only from workgroup-uniform values; readfirstlane states that, which keeps
// the descriptor in scalar registers (a clamp the compiler lowers to a vector
// med3 would otherwise move it to vector registers and wrap every load in a
// loop over the lanes' distinct descriptors).
__device__ __forceinline__ auto buffer_rsrc(const void *p, unsigned nrec) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, __builtin_amdgcn_readfirstlane(nrec),
                                           kBufferFlags);
}
// min(max(x, 0), HI) of a wave-uniform x, on the scalar unit: the compiler
// lowers the clamp to a vector med3 followed by readfirstlane otherwise.
template <int HI>
__device__ __forceinline__ int uniform_clamp0(int x) {
  int r;
  asm("s_max_i32 %0, %1, 0\n\ts_min_i32 %0, %0, %2" : "=&s"(r) : "s"(x), "n"(HI) : "scc");
  return r;
}
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

// fp16(fp32(v * s)): the product is rounded to fp32 first, then to fp16. The
// forward and both backward paths round c2 * Q through this one function, so
// the backward recomputes exactly the forward's scores; the empty asm keeps
// the compiler from fusing the product into a single-rounding mixed-precision
// FMA in some call sites and not in others.
__device__ __forceinline__ half4_t round_scaled4(float4 v, float s) {
  float4 p = scale4(v, s);
  asm volatile("" : "+v"(p.x), "+v"(p.y), "+v"(p.z), "+v"(p.w));
  return to_half4(p);
}

// fp16(p - fp16(p)) for p = fp32(v * s): what round_scaled4 rounds away
// (the difference is exact in fp32).
__device__ __forceinline__ half4_t scaled_residue4(float4 v, float s) {
  float4 p = scale4(v, s);
  asm volatile("" : "+v"(p.x), "+v"(p.y), "+v"(p.z), "+v"(p.w));
  const half4_t h = to_half4(p);
  return to_half4(make_float4(p.x - (float)h[0], p.y - (float)h[1], p.z - (float)h[2], p.w - (float)h[3]));
}

__device__ __forceinline__ float4 load4_or_zero(const float *p, bool ok) {
  return ok ? *reinterpret_cast<const float4 *>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Max / sum over the lane pair (l, l ^ 32), the two halves of one MFMA
// result column, with one v_permlane32_swap (no LDS round trip).
__device__ __forceinline__ float pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// acc + the 8 halves of h, each widened to fp32 and added in order by
// v_fma_mix_f32 (h * 1.0 + acc). A v_dot2 with ones would take two halves
// per instruction, but it occupies the SIMD's matrix pipe (an MFMA of the
// other wave on the SIMD stalls behind it); the mixed-precision fma issues
// beside the MFMAs.
__device__ __forceinline__ float sum8_f16(half8_t h, float acc) {
  const u32x4_t u = __builtin_bit_cast(u32x4_t, h);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(u[i]));
    asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(acc) : "v"(u[i]));
  }
  return acc;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// ---- fp16 tiles in LDS -----------------------------------------------------
// Every K, V, Q and dO tile the MFMA kernels stage is [rows][64] fp16 with a
// 128-byte row stride and an XOR swizzle of its 16-byte granules: granule g of
// row r sits at granule g ^ swz(r), swz(r) = 4*((r/2)%2) + (r/4)%4. The LDS
// has 64 banks of 4 bytes, so rows r and r+1 fill one 256-byte bank line.
// The three access patterns of the kernels are conflict-free:
//  * row reads (ds_read_b128, 16 lanes per pass): 16 consecutive rows from a
//    multiple of 16, one granule each — even rows take 8 distinct granules
//    and so do odd rows;
//  * transposed reads (ds_read_b64_tr_b16, 32 lanes per pass): 4 consecutive
//    rows from a multiple of 4, four adjacent granules each — rows r and r+2
//    differ in bit 2 of the swizzle, which moves an aligned group of four
//    granules to the other group;
//  * stores (8 bytes per lane, 32 lanes per pass): two full rows.
__device__ __forceinline__ int tile_swz(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }

// Offset in halves of element (r, col), col a multiple of 4.
__device__ __forceinline__ int tile_off(int r, int col) {
  return r * 64 + ((((col >> 3) ^ tile_swz(r)) << 3) | (col & 7));
}

// 8 halves of row r, columns 8*g .. 8*g+7.
__device__ __forceinline__ half8_t tile_row8(const half_t *tile, int r, int g) {
  return *reinterpret_cast<const half8_t *>(tile + r * 64 + ((g ^ tile_swz(r)) << 3));
}

__device__ __forceinline__ void tile_store4(half_t *tile, int r, int col, float4 v) {
  *reinterpret_cast<half4_t *>(tile + tile_off(r, col)) = to_half4(v);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) half_t lds_half_t;

// ds_read_b64_tr_b16: within each group of 16 lanes, result lane i, slot j is
// element i%4 of the 8 bytes that lane 4*j + i/4 addresses. With lane r of
// the group addressing (row0 + r/4, col0 + 4*(r%4)), lane i receives column
// col0 + i of rows row0 .. row0+3 — four consecutive rows of one column.
__device__ __forceinline__ half4_t tile_tr4(const half_t *tile, int row0, int col0, int lane) {
  const int r = lane & 15;
  const lds_half_t *base = (const lds_half_t *)tile;
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(base + tile_off(row0 + (r >> 2), col0 + 4 * (r & 3))));
  return __builtin_bit_cast(half4_t, v);
}

// Offset (in halves) that tile_tr4 reads for this lane, and the read itself
// at a precomputed offset: loops keep the offsets in registers and add only
// the stage base.
__device__ __forceinline__ int tile_tr4_off(int row0, int col0, int lane) {
  const int r = lane & 15;
  return tile_off(row0 + (r >> 2), col0 + 4 * (r & 3));
}
__device__ __forceinline__ half4_t tile_tr4_at(const half_t *tile, int off) {
  const lds_half_t *base = (const lds_half_t *)tile;
  return __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(base + off)));
}

// MFMA operand (A or B) holding, for the lane's column n = 32*blk + lane%32 of
// the tile's transpose, the 8 k-slots j -> tile rows 16*ks + 8*(j/4) + 4*hh +
// j%4 (hh = lane/32): the row order of a 32x32 MFMA result's registers, so the
// operand pairs with P or dS converted straight from accumulator registers.
__device__ __forceinline__ half8_t tile_tr8(const half_t *tile, int ks, int blk, int lane) {
  const int hh = lane >> 5, col0 = 32 * blk + 16 * ((lane >> 4) & 1);
  const half4_t lo = tile_tr4(tile, 16 * ks + 4 * hh, col0, lane);
  const half4_t hi = tile_tr4(tile, 16 * ks + 8 + 4 * hh, col0, lane);
  return half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Accumulator registers (16 floats, rows 8*(r/4) + 4*hh + r%4) of two
// consecutive 32-row blocks, as the 8 fp16 k-slots of step ks (rows
// 16*ks + 8*(j/4) + 4*hh + j%4) — the pairing tile_tr8 reads.
__device__ __forceinline__ half8_t acc_to_slots(const f32x16 &blk, int half_sel) {
  const int b = 8 * half_sel;
  half8_t h;
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = (half_t)blk[b + j];
  return h;
}

// ---- internal launch API (host side, all asynchronous on `stream`) -------

// Forward, D = 64, MFMA. q/k/v/o 16-byte aligned. lse may be null. With a
// backward workspace (bwd_workspace_bytes_d64 bytes), the forward also
// writes the backward's fp16 copies of c2*Q, K and V into it (see
// launch_bwd_pre_d64's qkv_saved). ldi: the row stride of q, k and v in
// floats (0: n_heads * 64, contiguous); o is always contiguous.
hipError_t launch_fwd_d64(const float *q, const float *k, const float *v, float *o,
                          float *lse, int n_heads, int seq_len, float scale, bool causal,
                          hipStream_t stream, void *bwd_workspace = nullptr, int ldi = 0);

// Backward, D = 64, MFMA. Needs bwd_workspace_bytes_d64() of workspace.
size_t bwd_workspace_bytes_d64(int n_heads, int seq_len);
// Where the fp16 copies of c2*Q, K and V sit in a backward workspace, and
// the residues fp16(x - fp16(x)) of each head's rows 0-63 of c2*Q and K (two
// [64][64] fp16 tiles per head from *qlo, `qlo_head_stride` halves apart).
void bwd_ws_qkv_copies(void *workspace, int n_heads, int seq_len, half_t **q16, half_t **k16, half_t **v16,
                       half_t **qlo, int *qlo_head_stride);
hipError_t launch_bwd_d64(const float *q, const float *k, const float *v, const float *o,
                          const float *d_o, const float *lse, float *d_q, float *d_k,
                          float *d_v, void *workspace, int n_heads, int seq_len, float scale,
                          bool causal, hipStream_t stream);
// The two phases of launch_bwd_d64: the workspace (Delta, the dO range and
// the fp16 operand copies), then the main kernel, which reads only the
// workspace, lse and its outputs.
// qkv_saved: the workspace already holds the copies of c2*Q, K and V that a
// launch_fwd_d64 with this workspace wrote for the same q, k, v and scale;
// only dO is converted.
// ldi: the row stride of q, k and v (read only without qkv_saved); ldg: the
// row stride of d_q, d_k and d_v (0: n_heads * 64, contiguous).
hipError_t launch_bwd_pre_d64(const float *q, const float *k, const float *v, const float *o,
                              const float *d_o, const float *lse, void *workspace, int n_heads, int seq_len,
                              float scale, hipStream_t stream, bool qkv_saved = false, int ldi = 0);
hipError_t launch_bwd_main_d64(const float *lse, float *d_q, float *d_k, float *d_v, const void *workspace,
                               int n_heads, int seq_len, float scale, bool causal, hipStream_t stream,
                               int ldg = 0);

// Generic fp32 kernels for any d_head in 1..=128 and any 4-byte alignment.
// The backward recomputes everything it needs per row and uses no workspace.
hipError_t launch_fwd_generic(const float *q, const float *k, const float *v, float *o,
                              float *lse, int n_heads, int seq_len, int d_head, float scale,
                              bool causal, hipStream_t stream);
hipError_t launch_bwd_generic(const float *q, const float *k, const float *v,
                              const float *d_o, float *d_q, float *d_k, float *d_v,
                              int n_heads, int seq_len, int d_head, float scale, bool causal,
                              hipStream_t stream);

// Single-query decode against a KV cache (attn_decode.hip). k, v: fp32 rows
// of n_heads*d_head, or bf16 bit patterns (bf16); block_table null for a
// contiguous cache. chunk >= cur_len or null partials: one workgroup per
// head writes out (and lse if not null) directly; otherwise the key range is
// split into ceil(cur_len / chunk) chunks whose partials (part_m, part_l:
// [n_heads, n_chunks], part_o: [n_heads, n_chunks, d_head]) a second kernel
// merges. fast: d_head == 64 with 16-byte aligned q and 8-byte aligned
// cache rows may take the coalesced kernel. cur_len >= 1.
hipError_t launch_decode(const float *q, const void *k, const void *v, const int32_t *block_table,
                         int page_size, bool bf16, float *out, float *lse, int n_heads, int cur_len,
                         int d_head, float scale, int chunk, float *part_m, float *part_l, float *part_o,
                         bool fast, hipStream_t stream);

// Elementwise companions of the decode path (attn_aux.hip). trained >= 1.
hipError_t launch_pos_embed_interpolate(const float *table, float *out, unsigned pos, unsigned trained,
                                        unsigned max_ctx, unsigned d_model, hipStream_t stream);
// In place on qk [n_heads * d_head]; an odd d_head leaves its last value alone.
hipError_t launch_apply_rope(float *qk, unsigned pos, unsigned n_heads, unsigned d_head, float base,
                             hipStream_t stream);
// pool row (phys_block * page_size + page_offset) := src [d_model], as fp32 or
// as bf16 bit patterns rounded to nearest even.
hipError_t launch_paged_copy_row(const float *src, void *pool, bool bf16, int phys_block, unsigned page_offset,
                                 unsigned page_size, unsigned d_model, hipStream_t stream);

}  // namespace dfattn
