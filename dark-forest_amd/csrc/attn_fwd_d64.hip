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

#include <type_traits>

namespace dfattn {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kD = 64;
constexpr int kBN = 64;    // keys per LDS tile
constexpr int kBM = 128;   // query rows per workgroup (4 row groups of 32)
constexpr int kTile = kBN * kD;           // halves per K or V tile
constexpr int kStageHalves = 2 * kTile;   // one ring stage: K tile, then V tile
constexpr int kStages = 4;
constexpr int kF4 = kBN * kD / 4 / kThreads;  // float4 of K (and of V) per thread per tile
static_assert(kF4 * kThreads * 4 == kBN * kD, "tile split");
// Merge buffer: per partner wave, 32 output registers + max + sum, lane-major.
constexpr int kMergeRegs = 34;
constexpr float kRescale = 8.f;  // log2 headroom of the softmax reference point
constexpr int kRingBytes = kStages * kStageHalves * 2;
constexpr int kMergeBytes = 4 * kMergeRegs * 64 * 4;
// After the ring: the workgroup's 128 Q rows as a [128][64] fp16 tile (c2 Q),
// staged once with coalesced loads; each wave reads its fragments from it.
constexpr int kQTileBytes = kBM * kD * 2;
constexpr int kQF4 = kBM * kD / 4 / kThreads;  // float4 of Q per thread
constexpr int kLdsBytes = (kMergeBytes > kRingBytes ? kMergeBytes : kRingBytes) + kQTileBytes;

template <int N>
using Stage = std::integral_constant<int, N>;

__global__ __launch_bounds__(kThreads) void fwd_d64_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    float *__restrict__ O, float *__restrict__ LSE, int H, int S, float qscale, int causal,
    int n_qtiles) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[kLdsBytes];
  half_t *ring = reinterpret_cast<half_t *>(lds_raw);

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, hh = lane >> 5;
  const int qg = wave & 3;   // query row group
  const int kh = wave >> 2;  // key half of every tile
  const int head = blockIdx.x % H;
  // Longest query tiles first under causal masking (they see the most keys).
  const int qtile = causal ? (n_qtiles - 1 - (int)(blockIdx.x / H)) : (int)(blockIdx.x / H);
  const int ld = H * kD;
  const int hoff = head * kD;

  const int q_blk0 = qtile * kBM;
  const int q_w0 = q_blk0 + qg * 32;
  const int query = q_w0 + c;
  const bool wave_active = q_w0 < S;
  const int wave_qlast = min(q_w0 + 32, S) - 1;
  // Keys above key_lim are masked for this lane's row.
  const int key_lim = causal ? min(query, S - 1) : S - 1;
  const int kv_end = causal ? min(S, q_blk0 + kBM) : S;
  const int n_tiles = (kv_end + kBN - 1) / kBN;
  // Tiles below n_full need no mask for any row of the workgroup: under
  // causal masking every key is below the first row; otherwise every key is
  // below S. The software-pipelined loop runs over them (while a next tile
  // exists) in groups of four; the rest take the general tail.
  const int n_full = causal ? min(q_blk0 / kBN, n_tiles) : S / kBN;
  const int n_main = min(n_full, n_tiles - 1);

  // The workgroup's Q rows arrive here by coalesced buffer loads; they are
  // rounded into LDS after the prologue has issued every load, and each wave
  // then reads its Q^T fragments from there.
  half8_t qf[4];
  float4 qraw[kQF4];
  {
    const unsigned rows = (unsigned)max(0, min(S - q_blk0, kBM));
    const size_t base = (size_t)min(q_blk0, S) * ld;
    const auto rq = __builtin_amdgcn_make_buffer_rsrc((void *)(Q + base), 0, rows * (unsigned)ld * 4, kBufferFlags);
#pragma unroll
    for (int k = 0; k < kQF4; ++k) {
      const int idx = tid + k * kThreads;
      qraw[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, ((idx >> 4) * ld + hoff + (idx & 15) * 4) * 4, 0, 0));
    }
  }

  // Per-thread offsets, fixed for the whole loop (the stage adds a constant):
  // K rows (A operand of S^T), V^T slots through transposed reads (A operand
  // of O^T), the thread's share of the tile stores, and its global float4s.
  int koff[4], voff[2][2][2], soff[kF4], goff[kF4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) koff[ds] = tile_off(kh * 32 + c, 8 * (2 * ds + hh));
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        voff[j][db][hf] = tile_tr4_off(16 * (2 * kh + j) + 8 * hf + 4 * hh, 32 * db + 16 * ((lane >> 4) & 1), lane);
#pragma unroll
  for (int i = 0; i < kF4; ++i) {
    const int idx = tid + i * kThreads;
    soff[i] = tile_off(idx >> 4, (idx & 15) * 4);
    goff[i] = ((idx >> 4) * ld + hoff + (idx & 15) * 4) * 4;
  }

  // Tile t of K and V through buffer loads on a descriptor based at key row
  // 64*t that covers rows up to S-1: rows past the end read as zeros (and are
  // masked out of the softmax), tiles past the end read as all zeros.
  // Two register sets of staged K/V float4s (set t % 2 holds tile t), so a
  // tile is fetched two iterations before it is written to LDS.
  float4 kreg[2][kF4], vreg[2][kF4];
  auto load_regs = [&](int t, float4 (&kr)[kF4], float4 (&vr)[kF4]) {
    const int kv0 = t * kBN;
    const long long rem = (long long)(S - kv0) * ld * 4;
    const unsigned nrec = rem <= 0 ? 0u : (unsigned)min(rem, (long long)kBN * ld * 4);
    const size_t base = (size_t)min(kv0, S) * ld;
    const auto rk = __builtin_amdgcn_make_buffer_rsrc((void *)(K + base), 0, nrec, kBufferFlags);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc((void *)(V + base), 0, nrec, kBufferFlags);
#pragma unroll
    for (int i = 0; i < kF4; ++i) {
      kr[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, goff[i], 0, 0));
      vr[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, goff[i], 0, 0));
    }
  };
  auto store_regs = [&](int stage, const float4 (&kr)[kF4], const float4 (&vr)[kF4]) {
    half_t *kt = ring + stage * kStageHalves;
#pragma unroll
    for (int i = 0; i < kF4; ++i) {
      *reinterpret_cast<half4_t *>(kt + soff[i]) = to_half4(kr[i]);
      *reinterpret_cast<half4_t *>(kt + kTile + soff[i]) = to_half4(vr[i]);
    }
  };
  auto load_tile = [&](int t, auto set) {
    constexpr int b = decltype(set)::value;
    load_regs(t, kreg[b], vreg[b]);
  };
  auto store_tile = [&](int stage, auto set) {
    constexpr int b = decltype(set)::value;
    store_regs(stage, kreg[b], vreg[b]);
  };
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;

  f32x16 o[2];
  o[0] = o[1] = f32x16{};
  float m = -INFINITY, l = 0.f;
  f32x16 negm = f32x16{};  // -m_use in every register (m_use = 0 while m = -inf)

  // K rows of this wave's key half (A operand of S^T = K Q^T).
  auto read_k = [&](int stage, half8_t (&kf)[4]) {
    const half_t *kt = ring + stage * kStageHalves;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) kf[ds] = *reinterpret_cast<const half8_t *>(kt + koff[ds]);
  };
  // V^T slots of this wave's two key steps (A operand of O^T += V^T P^T),
  // whose k-slots follow the row order of P^T.
  auto read_v = [&](int stage, half8_t (&vf)[2][2]) {
    const half_t *vt = ring + stage * kStageHalves + kTile;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const half4_t lo = tile_tr4_at(vt, voff[j][db][0]);
        const half4_t hi = tile_tr4_at(vt, voff[j][db][1]);
        vf[j][db] = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
  };
  // S^T - m: register r is key k0 + 8*(r/4) + 4*hh + r%4. The first MFMA's
  // accumulator input is -m, so the product arrives already shifted by the
  // softmax reference point.
  auto scores = [&](const half8_t (&kf)[4]) {
    f32x16 s = mfma32x32x16(kf[0], qf[0], negm);
#pragma unroll
    for (int ds = 1; ds < 4; ++ds) s = mfma32x32x16(kf[ds], qf[ds], s);
    return s;
  };
  // Online softmax in the log2 domain; one query row per lane pair (hh = 0,
  // 1 hold alternating groups of 4 keys). The reference point m moves only
  // when a row's maximum exceeds it by more than kRescale, so P^T stays below
  // 2^kRescale (exact in fp16) and the rescale of l and O is rare; m + log2(l)
  // is unchanged by the choice of m. The row sum l adds the same fp16 P the
  // product uses. `full`: no row of the tile is empty (every lane has a
  // finite maximum), which shortens the rescale test.
  auto softmax = [&](f32x16 &s, half8_t (&pf)[2], auto full) {
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = pair_max(mx);  // row max of S^T - m_use
    const bool need = decltype(full)::value ? (mx > kRescale || m == -INFINITY)
                                            : (mx > kRescale || (m == -INFINITY && mx > -INFINITY));
    if (__any(need)) {
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
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      pf[j] = acc_to_slots(s, j);
      l = sum8_f16(pf[j], l);
    }
  };
  auto pv = [&](const half8_t (&vf)[2][2], const half8_t (&pf)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 2; ++db) o[db] = mfma32x32x16(vf[j][db], pf[j], o[db]);
  };

  // Prologue: every load is issued before the first wait (Q above, tiles 0-2
  // into prologue registers, tiles 3 and 4 into their sets), then tiles 0-2
  // go into the ring and S of tile 0 is computed.
  {
    float4 kp[3][kF4], vp[3][kF4];
#pragma unroll
    for (int p = 0; p < 3; ++p) load_regs(p, kp[p], vp[p]);
    load_tile(3, Set1{});
    load_tile(4, Set0{});
    half_t *qt = reinterpret_cast<half_t *>(lds_raw + kLdsBytes - kQTileBytes);
#pragma unroll
    for (int k = 0; k < kQF4; ++k) {
      const int idx = tid + k * kThreads;
      *reinterpret_cast<half4_t *>(qt + tile_off(idx >> 4, (idx & 15) * 4)) = round_scaled4(qraw[k], qscale);
    }
#pragma unroll
    for (int p = 0; p < 3; ++p) store_regs(p, kp[p], vp[p]);
  }
  __syncthreads();
  {
    // Q^T fragments (B operand): lane c holds query q_w0 + c, slots d =
    // 16*ds + 8*hh + j.
    const half_t *qt = reinterpret_cast<const half_t *>(lds_raw + kLdsBytes - kQTileBytes);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
      qf[ds] = *reinterpret_cast<const half8_t *>(qt + tile_off(qg * 32 + c, 8 * (2 * ds + hh)));
  }
  f32x16 s;
  {
    half8_t kf[4];
    read_k(0, kf);
    s = scores(kf);
  }

  // Steady state, iteration t (stage p = t % 4 a compile-time constant): the
  // operands of S of tile t+1 and of P V of tile t are read from LDS first,
  // the softmax of tile t hides their latency, then both products run, tile
  // t+3 is written into stage (p+3) % 4 (last read in iteration t-1) and tile
  // t+5 is fetched into the register set tile t+3 has just left.
  auto iter = [&](int t, auto stage) {
    constexpr int p = decltype(stage)::value;
    half8_t kf[4], vf[2][2], pf[2];
    read_k((p + 1) & 3, kf);
    read_v(p, vf);
    softmax(s, pf, std::true_type{});
    s = scores(kf);
    pv(vf, pf);
    store_tile((p + 3) & 3, std::integral_constant<int, (p + 1) & 1>{});
    load_tile(t + 5, std::integral_constant<int, (p + 1) & 1>{});
    __syncthreads();
  };
  int t = 0;
  for (; t + 4 <= n_main; t += 4) {
    iter(t, Stage<0>{});
    iter(t + 1, Stage<1>{});
    iter(t + 2, Stage<2>{});
    iter(t + 3, Stage<3>{});
  }

  // Tail: the last (up to three) unmasked tiles of the pipelined range and
  // the tiles that hold the causal diagonal or the end of the keys.
  for (; t < n_tiles; ++t) {
    const int k0 = t * kBN + kh * 32;  // first key of this wave's half tile
    // Under causal masking a wave that sees none of tile t sees none after it.
    const bool act = wave_active && k0 < S && (!causal || k0 <= wave_qlast);
    if (act) {
      half8_t kf[4], vf[2][2], pf[2];
      if (t + 1 < n_tiles) read_k((t + 1) & 3, kf);
      read_v(t & 3, vf);
      if (t >= n_full) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0 + (r >> 2) * 8 + hh * 4 + (r & 3) > key_lim) s[r] = -INFINITY;
      }
      softmax(s, pf, std::false_type{});
      if (t + 1 < n_tiles) s = scores(kf);
      pv(vf, pf);
    }
    if (t + 3 < n_tiles) {
      if (t & 1) {
        store_tile((t + 3) & 3, Set0{});
        if (t + 5 < n_tiles) load_tile(t + 5, Set0{});
      } else {
        store_tile((t + 3) & 3, Set1{});
        if (t + 5 < n_tiles) load_tile(t + 5, Set1{});
      }
    }
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
