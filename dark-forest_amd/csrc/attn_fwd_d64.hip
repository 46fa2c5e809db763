// attn_fwd_d64.hip — fused causal attention forward for d_head = 64 on gfx950.
//
// Replaces kernel_fused_mha_fwd_tiled (darkforest-cuda/kernels/attention_fused.cu:41-159),
// which walks keys one at a time per query row with a warp-shuffle dot
// product. Here a workgroup of 8 waves owns BM = 128 query rows of one head
// and streams the keys in tiles of BN = 64 through LDS. Waves w and w+4 own
// the same 32 query rows and split every key tile (keys 0-31 and 32-63), each
// keeping its own running max, sum and output; the pair merges through LDS at
// the end. Two waves per SIMD on the same rows let one wave's softmax overlap
// the other's matrix products. Both products run on MFMA (32x32x16 f16, fp32
// accumulate):
//
//   S^T (keys x queries) = K (keys x d) . Q^T (d x queries)
//   O^T (d x queries)   += V^T (d x keys) . P^T (keys x queries)
//
// Computing the transposed products puts one query row in one lane (the MFMA
// result's column), so the online-softmax row max and row sum are per-lane
// register reductions plus one exchange between the two lane halves, and the
// probabilities come out of the first MFMA already in the B-operand layout of
// the second. K is read from its swizzled LDS tile by rows; V^T comes from the
// same row-major V tile through the transposing LDS read. Q is loaded once
// into registers, multiplied by scale*log2(e) before rounding, so the softmax
// runs on exp2. Operands are fp16 (rounded from the fp32 inputs on load);
// accumulation and softmax are fp32.
//
// Output: O [S, H*64] fp32 and, when lse != nullptr, lse [H, S] (natural log)
// — the row statistic the backward recomputes P from.
#include "dfattn_internal.h"

namespace dfattn {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kD = 64;
constexpr int kBN = 64;    // keys per LDS tile
constexpr int kBM = 128;   // query rows per workgroup (4 row groups of 32)
constexpr int kTile = kBN * kD;
constexpr int kF4 = kBN * kD / 4 / kThreads;  // float4 of K (and of V) per thread per tile
static_assert(kF4 * kThreads * 4 == kBN * kD, "tile split");
// Merge buffer: per partner wave, 32 output registers + max + sum, lane-major.
constexpr int kMergeRegs = 34;
constexpr float kRescale = 8.f;  // log2 headroom of the softmax reference point
constexpr int kLdsBytes = 4 * kMergeRegs * 64 * 4 > 2 * 2 * kTile * 2 ? 4 * kMergeRegs * 64 * 4
                                                                       : 2 * 2 * kTile * 2;

__global__ __launch_bounds__(kThreads) void fwd_d64_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    float *__restrict__ O, float *__restrict__ LSE, int H, int S, float qscale, int causal,
    int n_qtiles) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[kLdsBytes];
  half_t(*lds)[2][kTile] = reinterpret_cast<half_t(*)[2][kTile]>(lds_raw);  // [stage][K, V]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, hh = lane >> 5;
  const int qg = wave & 3;   // query row group
  const int kh = wave >> 2;  // key half of every tile
  const int head = blockIdx.x % H;
  // Longest query tiles first under causal masking (they see the most keys).
  const int qtile = causal ? (n_qtiles - 1 - (int)(blockIdx.x / H)) : (int)(blockIdx.x / H);
  const size_t ld = (size_t)H * kD;
  const size_t hoff = (size_t)head * kD;

  const int q_blk0 = qtile * kBM;
  const int q_w0 = q_blk0 + qg * 32;
  const int query = q_w0 + c;
  const bool wave_active = q_w0 < S;
  const int wave_qlast = min(q_w0 + 32, S) - 1;
  // Keys above key_lim are masked for this lane's row; no key of a half tile
  // starting at k0 is masked for any row of the wave when k0 + 31 <= key_lim_lo.
  const int key_lim = causal ? min(query, S - 1) : S - 1;
  const int key_lim_lo = causal ? min(q_w0, S - 1) : S - 1;
  const int kv_end = causal ? min(S, q_blk0 + kBM) : S;
  const int n_tiles = (kv_end + kBN - 1) / kBN;

  // Q^T fragments (B operand): lane c holds its query, slots d = 16*ds + 8*hh + j.
  half8_t qf[4];
  {
    const bool ok = query < S;
    const float *p = Q + (ok ? (size_t)query * ld + hoff : 0);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      const half4_t lo = to_half4(scale4(load4_or_zero(p + ds * 16 + hh * 8, ok), qscale));
      const half4_t hi = to_half4(scale4(load4_or_zero(p + ds * 16 + hh * 8 + 4, ok), qscale));
      qf[ds] = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }

  // Rows past the end are read from row S-1 (finite values) and masked out of
  // the softmax, so the loads need no branch.
  float4 kreg[kF4], vreg[kF4];
  auto load_tile = [&](int t) {
    const int kv0 = t * kBN;
#pragma unroll
    for (int i = 0; i < kF4; ++i) {
      const int idx = tid + i * kThreads;
      const int key = min(kv0 + (idx >> 4), S - 1), c4 = idx & 15;
      const size_t off = (size_t)key * ld + hoff + c4 * 4;
      kreg[i] = *reinterpret_cast<const float4 *>(K + off);
      vreg[i] = *reinterpret_cast<const float4 *>(V + off);
    }
  };
  auto store_tile = [&](int stage) {
#pragma unroll
    for (int i = 0; i < kF4; ++i) {
      const int idx = tid + i * kThreads;
      tile_store4(lds[stage][0], idx >> 4, (idx & 15) * 4, kreg[i]);
      tile_store4(lds[stage][1], idx >> 4, (idx & 15) * 4, vreg[i]);
    }
  };

  f32x16 o[2];
  o[0] = o[1] = f32x16{};
  float m = -INFINITY, l = 0.f;
  f32x16 negm = f32x16{};  // -m_use in every register (m_use = 0 while m = -inf)

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int stage = t & 1;
    if (t + 1 < n_tiles) load_tile(t + 1);
    const int k0 = t * kBN + kh * 32;  // first key of this wave's half tile
    if (wave_active && k0 < S && (!causal || k0 <= wave_qlast)) {
      const half_t *kt = lds[stage][0];
      const half_t *vt = lds[stage][1];

      // S^T - m: register r is key k0 + 8*(r/4) + 4*hh + r%4. The first
      // MFMA's accumulator input is -m, so the product arrives already shifted
      // by the softmax reference point.
      f32x16 s = mfma32x32x16(tile_row8(kt, kh * 32 + c, hh), qf[0], negm);
#pragma unroll
      for (int ds = 1; ds < 4; ++ds)
        s = mfma32x32x16(tile_row8(kt, kh * 32 + c, 2 * ds + hh), qf[ds], s);

      if (k0 + 31 > key_lim_lo) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0 + (r >> 2) * 8 + hh * 4 + (r & 3) > key_lim) s[r] = -INFINITY;
      }

      // Online softmax in the log2 domain; one query row per lane pair (hh =
      // 0, 1 hold alternating groups of 4 keys). The reference point m moves
      // only when a row's maximum exceeds it by more than kRescale, so P^T
      // stays below 2^kRescale (exact in fp16) and the rescale of l and O is
      // rare; m + log2(l) is unchanged by the choice of m.
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
      mx = pair_max(mx);  // row max of S^T - m_use
      if (__any(mx > kRescale || (m == -INFINITY && mx > -INFINITY))) {
        const float m_use = (m == -INFINITY) ? 0.f : m;
        const float m_new = fmaxf(m, m_use + mx);
        const float alpha = (m == -INFINITY) ? 0.f : fast_exp2(m - m_new);
        const float shift = (m_new == -INFINITY) ? 0.f : m_new - m_use;
        l *= alpha;
        o[0] *= alpha;
        o[1] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] -= shift;
        m = m_new;
#pragma unroll
        for (int r = 0; r < 16; ++r) negm[r] = (m == -INFINITY) ? 0.f : -m;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = fast_exp2(s[r]);

      // O^T += V^T P^T over this wave's two key steps of 16; V^T through
      // transposed reads whose k-slots follow the row order of P^T. The row
      // sum l adds the same fp16 P the product uses.
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const half8_t pf = acc_to_slots(s, j);
        l = sum8_f16(pf, l);
#pragma unroll
        for (int db = 0; db < 2; ++db)
          o[db] = mfma32x32x16(tile_tr8(vt, 2 * kh + j, db, lane), pf, o[db]);
      }
    }
    if (t + 1 < n_tiles) store_tile(stage ^ 1);
    __syncthreads();
  }

  // Merge the key halves: wave qg+4 hands (o, m, l) to wave qg through LDS.
  float *mbuf = reinterpret_cast<float *>(lds_raw) + (size_t)qg * kMergeRegs * 64;
  if (kh == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      mbuf[r * 64 + lane] = o[0][r];
      mbuf[(16 + r) * 64 + lane] = o[1][r];
    }
    mbuf[32 * 64 + lane] = m;
    mbuf[33 * 64 + lane] = l;
  }
  __syncthreads();
  if (kh == 1 || !wave_active) return;
  {
    const float m1 = mbuf[32 * 64 + lane], l1 = mbuf[33 * 64 + lane];
    const float mt = fmaxf(m, m1);
    const float mu = (mt == -INFINITY) ? 0.f : mt;
    const float a0 = fast_exp2(m - mu), a1 = fast_exp2(m1 - mu);
    l = l * a0 + l1 * a1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      o[0][r] = o[0][r] * a0 + mbuf[r * 64 + lane] * a1;
      o[1][r] = o[1][r] * a0 + mbuf[(16 + r) * 64 + lane] * a1;
    }
    m = mt;
  }
  const float lt = pair_sum(l);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (query < S) {
    float *orow = O + (size_t)query * ld + hoff;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 val = make_float4(o[db][4 * g] * inv, o[db][4 * g + 1] * inv,
                                       o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
        *reinterpret_cast<float4 *>(orow + db * 32 + g * 8 + hh * 4) = val;
      }
    if (LSE != nullptr && hh == 0)
      LSE[(size_t)head * S + query] = lt > 0.f ? (m + log2f(lt)) * kLn2 : -INFINITY;
  }
}

}  // namespace

hipError_t launch_fwd_d64(const float *q, const float *k, const float *v, float *o, float *lse,
                          int n_heads, int seq_len, float scale, bool causal,
                          hipStream_t stream) {
  const int n_qtiles = (seq_len + kBM - 1) / kBM;
  const dim3 grid((unsigned)(n_qtiles * n_heads));
  hipLaunchKernelGGL(fwd_d64_kernel, grid, dim3(kThreads), 0, stream, q, k, v, o, lse, n_heads,
                     seq_len, scale * kLog2e, causal ? 1 : 0, n_qtiles);
  return hipGetLastError();
}

}  // namespace dfattn
