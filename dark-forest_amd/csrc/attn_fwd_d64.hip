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
constexpr int kTile = kBN * kD;  // halves per K or V tile
constexpr int kTileBytes = kTile * 2;
// Two LDS rings of kStages stages: K tile t in K stage t % 4, V tile t in V
// stage t % 4 (the V ring follows the K ring).
constexpr int kStages = 4;
constexpr int kVRingBytes = kStages * kTileBytes;
constexpr int kF4 = kBN * kD / 4 / kThreads;  // float4 of K (and of V) per thread per tile
static_assert(kF4 * kThreads * 4 == kBN * kD, "tile split");
static_assert(kThreads * 8 == kTile, "one half8 per thread clears a tile");
// Merge buffer: per wave, the 16 output registers it hands to its partner +
// max + sum, lane-major.
constexpr int kMergeRegs = 18;
constexpr float kRescale = 8.f;  // log2 headroom of the softmax reference point
constexpr float kRescaleSum = 256.f;  // 2^kRescale
constexpr int kRingBytes = 2 * kStages * kTileBytes;
constexpr int kMergeBytes = kWaves * kMergeRegs * 64 * 4;
// After the rings: the workgroup's 128 Q rows as a [128][64] fp16 tile (c2 Q),
// staged once with coalesced loads; each wave reads its fragments from it.
constexpr int kQTileBytes = kBM * kD * 2;
constexpr int kQF4 = kBM * kD / 4 / kThreads;  // float4 of Q per thread
constexpr int kLdsBytes = (kMergeBytes > kRingBytes ? kMergeBytes : kRingBytes) + kQTileBytes;
// Rows of each head whose c2*Q and K rounding residues the training forward
// writes for the backward (its correction of the first keys and rows).
constexpr int kLoRows = 64;

template <int N>
using Stage = std::integral_constant<int, N>;

// ds_read_b64_tr_b16 at an LDS byte address (lane layout as in tile_tr4).
__device__ __forceinline__ half4_t lds_tr4(const unsigned char *p) {
  return __builtin_bit_cast(half4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                         (lds_i16x4 *)(const __attribute__((address_space(3))) unsigned char *)p));
}

// Q16, K16, V16 (all null, or none): the training forward also writes c2*Q,
// K and V as fp16 into these [H][S][64] copies, rounded exactly as the
// backward would round them, so the backward need not convert them again.
// Each workgroup writes its own 128 rows of c2*Q from its prologue
// registers. Under causal masking the K and V rows of its own query tile are
// the last key tiles the workgroup stages, and it writes them from LDS after
// the loop; without masking each workgroup copies those rows from the
// inputs at the end. QLO (with Q16): the residues fp16(x - fp16(x)) of each
// head's rows 0-63 of c2*Q and then of K, two [64][64] tiles every
// qlo_stride halves, which the backward adds for the first keys and rows.
__global__ __launch_bounds__(kThreads) void fwd_d64_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    float *__restrict__ O, float *__restrict__ LSE, int H, int S, float qscale, int causal,
    int n_qtiles, half_t *__restrict__ Q16, half_t *__restrict__ K16, half_t *__restrict__ V16,
    half_t *__restrict__ QLO, int qlo_stride, int ldi) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[kLdsBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, hh = lane >> 5;
  const int qg = wave & 3;   // query row group
  const int kh = wave >> 2;  // key half of every tile
  const int head = blockIdx.x % H;
  // Longest query tiles first under causal masking (they see the most keys).
  const int qtile = causal ? (n_qtiles - 1 - (int)(blockIdx.x / H)) : (int)(blockIdx.x / H);
  const int ld = H * kD;  // row stride of O
  // (ldi: the row stride of Q, K and V, which may be column blocks of a wider
  // tensor such as a fused [S, 3 H D] projection.)
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
  const bool save = Q16 != nullptr;
  {
    const unsigned rows = (unsigned)max(0, min(S - q_blk0, kBM));
    const size_t base = (size_t)min(q_blk0, S) * ldi;
    const auto rq = buffer_rsrc(Q + base, rows * (unsigned)ldi * 4);
#pragma unroll
    for (int k = 0; k < kQF4; ++k) {
      const int idx = tid + k * kThreads;
      qraw[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rq, ((idx >> 4) * ldi + hoff + (idx & 15) * 4) * 4, 0, 0));
    }
  }

  // Per-thread byte offsets within a tile, fixed for the whole loop (the
  // stage adds a constant): K rows (A operand of S^T), V^T slots through
  // transposed reads (A operand of O^T), the thread's share of a tile store
  // (one 16-byte granule: row tid/8, granule tid%8) and its two global
  // float4s (the granule's 8 floats).
  static_assert(kF4 == 2, "one granule per thread per tile");
  int koff[4], voff[2][2][2], soff, goff;
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) koff[ds] = 2 * tile_off(kh * 32 + c, 8 * (2 * ds + hh));
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        voff[j][db][hf] = 2 * tile_tr4_off(16 * (2 * kh + j) + 8 * hf + 4 * hh, 32 * db + 16 * ((lane >> 4) & 1), lane);
  soff = 2 * tile_off(tid >> 3, (tid & 7) * 8);
  goff = ((tid >> 3) * ldi + hoff + (tid & 7) * 8) * 4;

  // LDS stages: K tile t in K stage t % 4, V tile t in V stage t % 4.
  auto kstage = [&](int t) { return lds_raw + (t & (kStages - 1)) * kTileBytes; };
  auto vstage = [&](int t) { return lds_raw + kVRingBytes + (t & (kStages - 1)) * kTileBytes; };

  // Rows of tile t of X (K or V) through buffer loads on a descriptor based
  // at key row 64*t that covers rows up to S-1: rows past the end read as
  // zeros (and are masked out of the softmax), tiles past the end read as
  // all zeros. K tile t is staged in kreg[t % 2], V tile t in vreg[t % 2].
  float4 kreg[2][kF4], vreg[2][kF4];
  auto load_rows = [&](const float *X, int t, float4 (&xr)[kF4]) {
    const int kv0 = t * kBN;
    const int rows = uniform_clamp0<kBN>(S - kv0);  // (n_heads <= 65535: 64 rows span < 2^30 bytes)
    const auto rx = buffer_rsrc(X + (size_t)min(kv0, S) * ldi, (unsigned)rows * (unsigned)(ldi * 4));
#pragma unroll
    for (int i = 0; i < kF4; ++i)
      xr[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, goff + 16 * i, 0, 0));
  };
  auto store_rows = [&](unsigned char *dst, const float4 (&xr)[kF4]) {
    const half4_t lo = to_half4(xr[0]), hi = to_half4(xr[1]);
    *reinterpret_cast<half8_t *>(dst + soff) = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  f32x16 o[2];
  o[0] = o[1] = f32x16{};
  float m = -INFINITY, l = 0.f;
  f32x16 negm = f32x16{};  // -m_use in every register (m_use = 0 while m = -inf)

  // K rows of this wave's key half of tile t (A operand of S^T = K Q^T).
  auto read_k = [&](int t, half8_t (&kf)[4]) {
    const unsigned char *kt = kstage(t);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) kf[ds] = *reinterpret_cast<const half8_t *>(kt + koff[ds]);
  };
  // V^T slots of this wave's two key steps of tile t (A operand of O^T +=
  // V^T P^T), whose k-slots follow the row order of P^T.
  auto read_v = [&](int t, half8_t (&vf)[2][2]) {
    const unsigned char *vt = vstage(t);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const half4_t lo = lds_tr4(vt + voff[j][db][0]);
        const half4_t hi = lds_tr4(vt + voff[j][db][1]);
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
  // product uses.
  //
  // P^T = exp2(s) is computed before the rescale test is known, so that the
  // common case runs straight through; the rare rescale recomputes it. `sn`
  // holds the next tile's scores, already issued against the old reference
  // point, and O already holds the previous tile's product: a move of m
  // shifts and rescales them too. `full`: no row of the tile is empty (every
  // lane has a finite maximum), which shortens the rescale test.
  // (The empty asm keeps the compiler from merging the speculative and the
  // recomputed P^T into one computation after the rescale test.)
  auto probs = [&](const f32x16 &s, half8_t (&pf)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int i = 0; i < 8; ++i) pf[j][i] = (half_t)fast_exp2(s[8 * j + i]);
      asm volatile("" : "+v"(pf[j]));
    }
  };
  auto row_max = [&](const f32x16 &s) {
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    return pair_max(mx);  // row max of S^T - m_use
  };
  auto rowsum = [&](const half8_t (&pf)[2]) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) a = sum8_f16(pf[j], a);
    asm volatile("" : "+v"(a));
    return a;
  };
  // The rescale test and the rare rescale, after row_max, probs and rowsum.
  auto softmax_fix = [&](f32x16 &s, f32x16 &sn, half8_t (&pf)[2], float mx, float psum, auto full) {
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
      // The reference point moves by `shift` in place (the scores, the
      // issued next scores and the accumulator input alike); m is read back
      // from the accumulator input so that lse uses exactly the point the
      // products were shifted by.
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] -= shift;
        sn[r] -= shift;
        negm[r] -= shift;
      }
      m = (m_new == -INFINITY) ? m_new : -negm[0];
      probs(s, pf);
      psum = rowsum(pf);
    }
    l += psum;
  };
  auto pv = [&](const half8_t (&vf)[2][2], const half8_t (&pf)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 2; ++db) o[db] = mfma32x32x16(vf[j][db], pf[j], o[db]);
  };

  // Iteration t reads K of tile t+1 (its scores) and V of tile t-1 (the
  // product of the previous tile's P, one iteration late so that both
  // products are independent of the softmax of tile t they run beside). It
  // writes K of tile t+3 and V of tile t+1 into their stages and fetches K of
  // tile t+5 and V of tile t+3 into the register sets those have just left.
  // The workgroup synchronises after every second iteration (odd t): what an
  // iteration writes is read two or more iterations later, and a stage read
  // in iteration i is next written in iteration i+2, so one barrier always
  // lies between them.
  //
  // Prologue: every load is issued before the first wait (Q above, K tiles
  // 0-2 and V tile 0 into prologue registers, K tiles 3, 4 and V tiles 1, 2
  // into their sets), then those go into the rings, the V stage of tile -1
  // is cleared (tile 0 runs as a steady iteration whose pending product
  // adds zero) and S of tile 0 is computed.
  {
    float4 kp[3][kF4], vp[kF4];
#pragma unroll
    for (int p = 0; p < 3; ++p) load_rows(K, p, kp[p]);
    load_rows(V, 0, vp);
    load_rows(K, 3, kreg[1]);
    load_rows(V, 1, vreg[1]);
    load_rows(K, 4, kreg[0]);
    load_rows(V, 2, vreg[0]);
    half_t *qt = reinterpret_cast<half_t *>(lds_raw + kLdsBytes - kQTileBytes);
#pragma unroll
    for (int k = 0; k < kQF4; ++k) {
      const int idx = tid + k * kThreads;
      const half4_t qh = round_scaled4(qraw[k], qscale);
      *reinterpret_cast<half4_t *>(qt + tile_off(idx >> 4, (idx & 15) * 4)) = qh;
      const int row = q_blk0 + (idx >> 4);
      if (save && row < S) *reinterpret_cast<half4_t *>(Q16 + ((size_t)head * S + row) * kD + (idx & 15) * 4) = qh;
      if (save && row < min(S, kLoRows))
        *reinterpret_cast<half4_t *>(QLO + (size_t)head * qlo_stride + row * kD + (idx & 15) * 4) =
            scaled_residue4(qraw[k], qscale);
    }
#pragma unroll
    for (int p = 0; p < 3; ++p) store_rows(kstage(p), kp[p]);
    // The workgroup of query tile 0 also writes the residues of K's rows 0-63
    // (key tile 0), one granule of 8 values per thread.
    if (save && qtile == 0 && (tid >> 3) < min(S, kLoRows)) {
      half_t *dst = QLO + (size_t)head * qlo_stride + kLoRows * kD + (tid >> 3) * kD + (tid & 7) * 8;
      const half4_t lo = scaled_residue4(kp[0][0], 1.f), hi = scaled_residue4(kp[0][1], 1.f);
      *reinterpret_cast<half8_t *>(dst) = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    store_rows(vstage(0), vp);
    *reinterpret_cast<half8_t *>(vstage(-1) + tid * 16) = half8_t{};
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
  half8_t pprev[2] = {};  // P^T of the previous tile, waiting for its product

  // Whether this wave sees any key of tile t (under causal masking a wave
  // that sees none of tile t sees none after it).
  auto active = [&](int t) {
    const int k0 = t * kBN + kh * 32;  // first key of this wave's half tile
    return wave_active && k0 < S && (!causal || k0 <= wave_qlast);
  };
  // The tile stores and fetches of iteration t, from and into register set
  // b = (t+1) % 2; q = t mod 4 (a constant in the steady state) places the
  // stores. `all`: no range checks (the steady state, where K tiles past the
  // end are fetched as zeros into stages no later iteration reads).
  auto stage_tiles = [&](int t, int q, auto set, bool all) {
    constexpr int b = decltype(set)::value;
    if (all || t + 3 < n_tiles) {
      store_rows(kstage(q + 3), kreg[b]);
      if (all || t + 5 < n_tiles) load_rows(K, t + 5, kreg[b]);
    }
    if (all || t + 1 < n_tiles) {
      store_rows(vstage(q + 1), vreg[b]);
      if (all || t + 3 < n_tiles) load_rows(V, t + 3, vreg[b]);
    }
  };
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;

  // General iteration: runtime stage and register set, masks, tile range
  // ends. Used for the remainder of the unmasked range and for the tiles
  // that hold the causal diagonal or the end of the keys.
  auto step = [&](int t) {
    const bool act_prev = t >= 1 && active(t - 1);
    const bool act_cur = active(t);
    const bool act_next = t + 1 < n_tiles && active(t + 1);
    half8_t kf[4], vf[2][2], pf[2];
    f32x16 sn = f32x16{};
    if (act_next) {
      read_k(t + 1, kf);
      sn = scores(kf);
    }
    if (act_prev) {
      read_v(t - 1, vf);
      pv(vf, pprev);
    }
    if (act_cur) {
      if (t >= n_full) {
        // Register r holds key t*64 + 32*kh + 4*hh + 8*(r/4) + r%4.
        const int lim = key_lim - (t * kBN + kh * 32 + hh * 4);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if ((r >> 2) * 8 + (r & 3) > lim) s[r] = -INFINITY;
      }
      const float mx = row_max(s);
      probs(s, pf);
      softmax_fix(s, sn, pf, mx, rowsum(pf), std::false_type{});
      s = sn;
      pprev[0] = pf[0];
      pprev[1] = pf[1];
    }
    if (t & 1)
      stage_tiles(t, t, Set0{}, false);
    else
      stage_tiles(t, t, Set1{}, false);
    if (t & 1) __syncthreads();
  };

  // Steady state, iteration t (stage p = t % 4 a compile-time constant, so
  // every LDS offset is an immediate): unmasked, with a next tile, every
  // wave active. Both products are issued before the softmax of tile t, and
  // the tile stores and fetches come before the rare rescale branch, so that
  // all of it is one block for the scheduler.
  auto iter = [&](int t, auto stage) {
    constexpr int p = decltype(stage)::value;
    half8_t kf[4], vf[2][2], pf[2];
    read_k(p + 1, kf);
    read_v(p + kStages - 1, vf);
    f32x16 sn = scores(kf);
    pv(vf, pprev);
    probs(s, pf);
    const float psum = rowsum(pf);
    stage_tiles(t, p, std::integral_constant<int, (p + 1) & 1>{}, true);
    // Every P is >= 0, so a lane's sum bounds its largest P, and a score more
    // than kRescale above the reference point makes P >= 2^kRescale: the
    // exact row maximum (and the rescale test) is needed only when a sum
    // reaches that, or before the first reference point.
    if (__any(psum >= kRescaleSum || m == -INFINITY))
      softmax_fix(s, sn, pf, row_max(s), psum, std::true_type{});
    else
      l += psum;
    s = sn;
    pprev[0] = pf[0];
    pprev[1] = pf[1];
    if (p & 1)
      __syncthreads();
    else
      __builtin_amdgcn_sched_barrier(0);  // keep the iterations' register live ranges apart
  };
  // Register r of S^T holds key t*64 + 32*kh + 4*hh + 8*(r/4) + r%4; keys
  // above the lane's row are masked.
  auto mask_diag = [&](f32x16 &x, int tile) {
    const int lim = key_lim - (tile * kBN + kh * 32 + hh * 4);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if ((r >> 2) * 8 + (r & 3) > lim) x[r] = -INFINITY;
  };
  // The two tiles on the causal diagonal (t and t+1, the last two) of a
  // query tile that ends at or before S, as steady iterations with
  // compile-time stages: tile t stores V of tile t+1 (the only staging left)
  // and issues the scores of tile t+1; tile t+1 has no next tile. Waves that
  // see no key of a tile compute fully masked scores (P = 0) instead of
  // skipping it. The ring stages and barriers are those of `step`.
  auto diag = [&](int t, auto stage) {
    constexpr int p = decltype(stage)::value;
    static_assert((p & 1) == 0, "the diagonal starts at an even tile");
    half8_t kf[4], vf[2][2], pf[2];
    read_k(p + 1, kf);
    read_v(p + kStages - 1, vf);
    f32x16 sn = scores(kf);
    pv(vf, pprev);
    mask_diag(s, t);
    probs(s, pf);
    float psum = rowsum(pf);
    store_rows(vstage(p + 1), vreg[1]);
    if (__any(psum >= kRescaleSum || m == -INFINITY))
      softmax_fix(s, sn, pf, row_max(s), psum, std::false_type{});
    else
      l += psum;
    s = sn;
    pprev[0] = pf[0];
    pprev[1] = pf[1];
    __builtin_amdgcn_sched_barrier(0);
    read_v(p, vf);
    pv(vf, pprev);
    mask_diag(s, t + 1);
    probs(s, pf);
    psum = rowsum(pf);
    f32x16 none = f32x16{};  // no next tile
    if (__any(psum >= kRescaleSum || m == -INFINITY))
      softmax_fix(s, none, pf, row_max(s), psum, std::false_type{});
    else
      l += psum;
    pprev[0] = pf[0];
    pprev[1] = pf[1];
    __syncthreads();
  };
  int t = 0;
  for (; t + 4 <= n_main; t += 4) {
    iter(t, Stage<0>{});
    iter(t + 1, Stage<1>{});
    iter(t + 2, Stage<2>{});
    iter(t + 3, Stage<3>{});
  }
  // Under causal masking a query tile that ends at or before S has n_main =
  // n_tiles - 2 (even): after the loop above at most two unmasked tiles
  // remain (stages 0 and 1), then the diagonal pair.
  if (causal && q_blk0 + kBM <= S) {
    if (t + 2 <= n_main) {
      iter(t, Stage<0>{});
      iter(t + 1, Stage<1>{});
      t += 2;
    }
    if ((t & 3) == 0)
      diag(t, Stage<0>{});
    else
      diag(t, Stage<2>{});
    t = n_tiles;
  }
  for (; t < n_tiles; ++t) step(t);
  // The last tile's product.
  if (n_tiles > 0 && active(n_tiles - 1)) {
    half8_t vf[2][2];
    read_v(n_tiles - 1, vf);
    pv(vf, pprev);
  }
  __syncthreads();  // the merge below reuses the rings

  if (save) {
    if (causal) {
      // The key tiles of the workgroup's own rows (2*qtile and, below S,
      // 2*qtile+1) were the loop's last and still sit in their ring stages,
      // rounded to fp16 exactly as the backward rounds K and V: one 16-byte
      // granule per thread and tile goes out (rows past S are not written).
      const int r = tid >> 3, g = tid & 7;
      for (int kt = 2 * qtile; kt < n_tiles; ++kt) {
        const int row = kt * kBN + r;
        const int off = 2 * tile_off(r, 8 * g);
        const half8_t kx = *reinterpret_cast<const half8_t *>(kstage(kt) + off);
        const half8_t vx = *reinterpret_cast<const half8_t *>(vstage(kt) + off);
        if (row < S) {
          const size_t dst = ((size_t)head * S + row) * kD + 8 * g;
          *reinterpret_cast<half8_t *>(K16 + dst) = kx;
          *reinterpret_cast<half8_t *>(V16 + dst) = vx;
        }
      }
      __syncthreads();  // the merge below overwrites the K ring
    } else {
      // Every workgroup sees every key tile: each copies the K and V rows of
      // its own query tile from the inputs.
      const int r0 = q_blk0;
      const unsigned rows = (unsigned)max(0, min(S - r0, kBM));
      const size_t base = (size_t)min(r0, S) * ldi;
      const auto rk = buffer_rsrc(K + base, rows * (unsigned)ldi * 4);
      const auto rv = buffer_rsrc(V + base, rows * (unsigned)ldi * 4);
      float4 kx[kQF4], vx[kQF4];
#pragma unroll
      for (int k = 0; k < kQF4; ++k) {
        const int idx = tid + k * kThreads;
        const int off = ((idx >> 4) * ldi + hoff + (idx & 15) * 4) * 4;
        kx[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
        vx[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
      }
#pragma unroll
      for (int k = 0; k < kQF4; ++k) {
        const int idx = tid + k * kThreads;
        const int row = r0 + (idx >> 4);
        if (row < S) {
          const size_t dst = ((size_t)head * S + row) * kD + (idx & 15) * 4;
          *reinterpret_cast<half4_t *>(K16 + dst) = to_half4(kx[k]);
          *reinterpret_cast<half4_t *>(V16 + dst) = to_half4(vx[k]);
        }
      }
    }
  }

  // Merge the key halves: waves qg (kh 0) and qg+4 (kh 1) swap halves of their
  // output through LDS, each handing over the 32-column block the other
  // finishes (with its m and l); wave kh then merges and stores columns
  // 32*kh .. +31, so both halves of the merge and of the stores run at once.
  float *slot = reinterpret_cast<float *>(lds_raw) + (size_t)wave * kMergeRegs * 64;
  const float *other = reinterpret_cast<const float *>(lds_raw) + (size_t)(wave ^ 4) * kMergeRegs * 64;
#pragma unroll
  for (int r = 0; r < 16; ++r) slot[r * 64 + lane] = kh == 0 ? o[1][r] : o[0][r];
  slot[16 * 64 + lane] = m;
  slot[17 * 64 + lane] = l;
  __syncthreads();
  if (!wave_active) return;
  const float mp = other[16 * 64 + lane], lp = other[17 * 64 + lane];
  const float m0 = kh == 0 ? m : mp, m1 = kh == 0 ? mp : m;
  const float l0 = kh == 0 ? l : lp, l1 = kh == 0 ? lp : l;
  const float mt = fmaxf(m0, m1);
  const float mu = (mt == -INFINITY) ? 0.f : mt;
  const float a0 = fast_exp2(m0 - mu), a1 = fast_exp2(m1 - mu);
  const float lt = pair_sum(l0 * a0 + l1 * a1);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (query < S) {
    float *orow = O + (size_t)query * ld + hoff + kh * 32;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * g + j;
        const float mine = kh == 0 ? o[0][r] : o[1][r], theirs = other[r * 64 + lane];
        const float x0 = kh == 0 ? mine : theirs, x1 = kh == 0 ? theirs : mine;
        v[j] = (x0 * a0 + x1 * a1) * inv;
      }
      *reinterpret_cast<float4 *>(orow + g * 8 + hh * 4) = make_float4(v[0], v[1], v[2], v[3]);
    }
    if (LSE != nullptr && kh == 0 && hh == 0)
      LSE[(size_t)head * S + query] = lt > 0.f ? (mt + log2f(lt)) * kLn2 : -INFINITY;
  }
}

}  // namespace

hipError_t launch_fwd_d64(const float *q, const float *k, const float *v, float *o, float *lse,
                          int n_heads, int seq_len, float scale, bool causal,
                          hipStream_t stream, void *bwd_workspace, int ldi) {
  const int n_qtiles = (seq_len + kBM - 1) / kBM;
  const dim3 grid((unsigned)(n_qtiles * n_heads));
  half_t *q16 = nullptr, *k16 = nullptr, *v16 = nullptr, *qlo = nullptr;
  int qlo_stride = 0;
  if (bwd_workspace != nullptr)
    bwd_ws_qkv_copies(bwd_workspace, n_heads, seq_len, &q16, &k16, &v16, &qlo, &qlo_stride);
  hipLaunchKernelGGL(fwd_d64_kernel, grid, dim3(kThreads), 0, stream, q, k, v, o, lse, n_heads,
                     seq_len, scale * kLog2e, causal ? 1 : 0, n_qtiles, q16, k16, v16, qlo, qlo_stride,
                     ldi > 0 ? ldi : n_heads * kD);
  return hipGetLastError();
}

}  // namespace dfattn
