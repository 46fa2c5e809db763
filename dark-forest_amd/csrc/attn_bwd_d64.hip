// attn_bwd_d64.hip — fused causal attention backward for d_head = 64 on gfx950.
//
// Replaces kernel_mha_bwd_all_heads (darkforest-cuda/kernels/attention_fused.cu:390-516),
// which recomputes each row's softmax with four serial passes over the keys,
// stores P and dS in an [H, 2, S, S] fp32 scratch and accumulates dK and dV
// with one atomicAdd per (query, key, d). Here, with no O(S^2) memory and no
// atomics:
//
//  1. bwd_prep (one launch, independent 64-row blocks): per block of one
//     head, a power-of-two scale sigma_b of dO (from the block's max |dO|),
//     the fp16 copy of sigma_b * dO, Delta_i = dO_i . O_i (scaled by sigma_b,
//     formed from the rounded copy) and -lse_i * log2(e); without a training
//     forward also the fp16 copies of c2*Q, K and V.
//  2. bwd_main, one launch holding two kinds of workgroup, interleaved
//     longest-first so both fill the chip together:
//     * dK/dV workgroups own 128 keys of one head (32 per wave, their K and V
//       rows held in registers) and stream the query rows in blocks of 64
//       through LDS:
//          S = (c2 Q) K^T, dP = dO V^T         (queries x keys, lane = key)
//          P = exp2(S - lse*log2e), dS = P * (dP - Delta)
//          dV += P^T dO, dK += dS^T (c2 Q)      (keys x d, in registers)
//     * dQ workgroups own 128 query rows (32 per wave, Q and dO in
//       registers) and stream the keys in tiles of 64 through LDS:
//          S^T = K (c2 Q)^T, dP^T = V dO^T      (keys x queries, lane = query)
//          dQ^T += K^T dS^T                     (d x queries, in registers)
//     Recomputing S and dP for dQ costs two more products than accumulating
//     dQ with atomics from the dK/dV workgroups, and removes the atomics'
//     traffic (one fp32 read-modify-write per query, column and key block).
//
// Operands that must be transposed (dO^T and Q^T for dV and dK, K^T for dQ)
// come from the same row-major swizzled tiles through the transposing LDS
// read, with k-slots in the row order of the P and dS registers they pair with.
//
#include "dfattn_internal.h"

#include <type_traits>

namespace dfattn {
namespace {

constexpr int kPreRows = 64;  // rows per phase-1 workgroup (one dO scale per block)
inline int pre_blocks(int S) { return (S + kPreRows - 1) / kPreRows; }
// Under causal masking the first keys of a head see few query rows, with
// probabilities near one (row 0 sees key 0 alone), so one fp16 rounding of
// dO, dS or Q in rows 0-63 lands almost undamped in dV and dK of those keys:
// for N(0,1) inputs these are the largest absolute errors of the backward.
// The dK/dV workgroup of keys 0-127 therefore adds the rounding residues of
// those rows (lo = fp16(x - fp16(x)) of sigma*dO, c2*Q and dS) with three
// more products per block: dV += P^T dO_lo, dK += dS_lo^T (c2 Q) + dS^T (c2 Q)_lo.
// Likewise the dQ workgroup of rows 0-127 adds, for keys 0-63 (its first
// tile), dQ += dS K_lo + dS_lo K.
constexpr int kLoRows = 64;
constexpr int kLoTiles = 3;  // per head: sigma*dO, c2*Q, K (rows 0-63)

// Power-of-two scale of a 64-row block of dO: sigma = 2^e with e = 1 (mod 4)
// and max|sigma * x| in [2, 32) for amax = max|x| (1 if amax is 0 or not
// finite). fp16 then holds sigma * dO with full precision down to 2^-15 of
// the block's maximum, and dS = P * (dP - Delta) formed from it keeps well
// inside the fp16 range. The exponent moves in steps of 4 so that blocks of
// similar magnitude share one scale (N(0,1) blocks all get 2): the dK/dV
// accumulators, which add products of many blocks, change units only where
// the scale changes.
__device__ __forceinline__ float block_scale(float amax) {
  if (!(amax > 0.f) || !(amax < INFINITY)) return 1.f;
  const int e_fine = 3 - ilogbf(amax);  // max|2^e_fine x| in [8, 16)
  const int e = e_fine - 2 + (((3 - e_fine) % 4) + 4) % 4;  // the one e = 1 (mod 4) in [e_fine - 2, e_fine + 1]
  return ldexpf(1.f, max(-123, min(125, e)));
}

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kD = 64;
constexpr int kKeysPerWg = 128;     // dK/dV workgroup: keys owned (4 groups of 32)
constexpr int kQBlock = 64;         // dK/dV workgroup: query rows per step (2 halves of 32)
constexpr int kQueriesPerWg = 128;  // dQ workgroup: query rows owned (4 groups of 32)
constexpr int kKTile = 64;          // dQ workgroup: keys per step (2 halves of 32)
constexpr int kTile = 64 * kD;      // halves per staged [64][64] tile
// fp16 copies are staged one 16-byte granule (8 halves) per thread per
// [64][64] tile: thread t takes row t/8, granule t%8.
static_assert(64 * kD / 8 == kThreads, "one granule per thread per staged tile");
// LDS ring of kStages stages, each two fp16 tiles (Q and dO, or K and V) and,
// for the dK/dV path, the block's two row statistics and its dO scale (first
// value of a 64-float slot). After the loop the same
// bytes carry the partner waves' partial results (8 waves x 32 registers x 64
// lanes fp32).
constexpr int kStages = 4;
constexpr int kStageBytes = 2 * kTile * 2 + 3 * kQBlock * 4;
constexpr int kStageSigma = 2 * kTile * 2 + 2 * kQBlock * 4;  // byte offset of the block's dO scale
constexpr int kRingBytes = kStages * kStageBytes;
constexpr int kMergeBytes = 8 * 32 * 64 * 4;
// After the ring: the workgroup's own 128 rows of K and V (dK/dV path) or of
// c2*Q and sigma*dO (dQ path) as two [128][64] fp16 tiles, staged once with
// coalesced loads; each wave reads its register fragments from there.
constexpr int kOwnTile = 128 * kD;  // halves
constexpr int kOwnBytes = 2 * kOwnTile * 2;
// Last, the dQ workgroup's 128 values of -lse*log2(e) and of -Delta*sigma.
constexpr int kRowStatBytes = 2 * 128 * 4;
// Then the dK/dV workgroup of keys 0-127 (causal) keeps the residue tiles of
// rows 0-63, sigma*dO_lo and (c2 Q)_lo, as two [64][64] fp16 tiles.
constexpr int kLoBytes = 2 * kTile * 2;
constexpr int kLdsBytes = (kRingBytes > kMergeBytes ? kRingBytes : kMergeBytes) + kOwnBytes + kRowStatBytes + kLoBytes;
constexpr int kOwnOffset = kLdsBytes - kLoBytes - kRowStatBytes - kOwnBytes;
constexpr int kRowStatOffset = kLdsBytes - kLoBytes - kRowStatBytes;
constexpr int kLoOffset = kLdsBytes - kLoBytes;

template <int N>
using Const = std::integral_constant<int, N>;

// Workspace layout (bytes, each part 256-byte aligned): the dO scale of
// every 64-row block, sigma [H][ceil(S/64)] fp32; the row statistics as the
// main kernel's products take them, -lse*log2(e) and -Delta*sigma_b, each
// [H][S] fp32; the fp16 copies c2*Q, K, V and sigma_b*dO, each [H][S][64];
// the fp16 rounding residues of rows 0-63 of sigma_b*dO, c2*Q and K,
// [H][3][64][64] (see kLoRows).
struct WsLayout {
  size_t sigma, lse2n, deltan, q16, k16, v16, do16, lo16, total;
};
inline size_t align256(size_t x) { return (x + 255) / 256 * 256; }
inline WsLayout ws_layout(int H, int S) {
  WsLayout w;
  const size_t stat = align256((size_t)H * S * sizeof(float));
  const size_t copy = align256((size_t)H * S * kD * sizeof(half_t));
  w.sigma = 0;
  w.lse2n = align256((size_t)H * pre_blocks(S) * sizeof(float));
  w.deltan = w.lse2n + stat;
  w.q16 = w.deltan + stat;
  w.k16 = w.q16 + copy;
  w.v16 = w.k16 + copy;
  w.do16 = w.v16 + copy;
  w.lo16 = w.do16 + copy;
  w.total = w.lo16 + align256((size_t)H * kLoTiles * kLoRows * kD * sizeof(half_t));
  return w;
}

// Phase 1: 64 rows of one head per workgroup (256 threads; thread t owns row
// t/4, columns 4*(t%4) + 16*i .. +3 for i = 0..3 of each tensor, so that the
// four threads of a row read one contiguous 64 bytes per load). The block's dO scale sigma_b
// comes from the block's own max |dO|, so blocks are independent and phase 1
// is one launch. Delta is summed from the same rounded sigma_b * dO that the
// main kernel's dP products use, so the rows of dS = P * (dP - Delta) sum to
// zero for the rounded operands. Without a training forward (convert_qkv)
// the workgroup also writes c2*Q (rounded as the forward rounds it,
// round_scaled4), K and V.
__global__ __launch_bounds__(256) void bwd_prep_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    const float *__restrict__ O, const float *__restrict__ dO, const float *__restrict__ lse,
    float *__restrict__ sigma_out, float *__restrict__ lse2n, float *__restrict__ deltan,
    half_t *__restrict__ q16, half_t *__restrict__ k16, half_t *__restrict__ v16, half_t *__restrict__ do16,
    half_t *__restrict__ lo16, int H, int S, float c2, int convert_qkv, int ldi) {
  __shared__ float wmax[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int head = blockIdx.y;
  const int row = blockIdx.x * kPreRows + (tid >> 2);
  const bool ok = row < S;
  const size_t src = ok ? (size_t)row * H * kD + (size_t)head * kD + (tid & 3) * 4 : 0;
  const size_t src_in = ok ? (size_t)row * ldi + (size_t)head * kD + (tid & 3) * 4 : 0;  // Q, K, V
  const size_t dst = ((size_t)head * S + row) * kD + (tid & 3) * 4;
  const size_t r = (size_t)head * S + row;
  // Every load first.
  float4 g[4], o[4], x[3][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    g[i] = load4_or_zero(dO + src + 16 * i, ok);
    o[i] = load4_or_zero(O + src + 16 * i, ok);
  }
  const float *in[3] = {Q, K, V};
  if (convert_qkv) {
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) x[t][i] = load4_or_zero(in[t] + src_in + 16 * i, ok);
  }
  const bool lo_block = blockIdx.x == 0;
  const float l = ok ? lse[r] : 0.f;
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(g[i].x), fabsf(g[i].y)), fmaxf(fabsf(g[i].z), fabsf(g[i].w))));
  mx = wave_max(mx);
  if (lane == 0) wmax[wave] = mx;
  __syncthreads();
  const float sig = block_scale(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])));
  if (tid == 0) sigma_out[(size_t)head * gridDim.x + blockIdx.x] = sig;
  // sigma_b * dO in fp16, and Delta from exactly those values.
  float acc = 0.f;
  half4_t h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = to_half4(scale4(g[i], sig));
    acc += (float)h[i][0] * o[i].x;
    acc += (float)h[i][1] * o[i].y;
    acc += (float)h[i][2] * o[i].z;
    acc += (float)h[i][3] * o[i].w;
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  if (!ok) return;
  if ((tid & 3) == 0) {
    lse2n[r] = -l * kLog2e;
    deltan[r] = -acc;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<half4_t *>(do16 + dst + 16 * i) = h[i];
  // Rows 0-63: the rounding residues fp16(x - fp16(x)) of sigma_b*dO and (when
  // this launch converts Q, K and V; otherwise the training forward wrote
  // them) of c2*Q and K, x the fp32 value the fp16 copy was rounded from (the
  // difference is exact in fp32).
  half_t *lo = lo16 + ((size_t)head * kLoTiles * kLoRows + row) * kD + (tid & 3) * 4;
  if (lo_block) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 gp = scale4(g[i], sig);
      *reinterpret_cast<half4_t *>(lo + 16 * i) = to_half4(make_float4(
          gp.x - (float)h[i][0], gp.y - (float)h[i][1], gp.z - (float)h[i][2], gp.w - (float)h[i][3]));
    }
  }
  if (!convert_qkv) return;
  if (lo_block) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<half4_t *>(lo + kLoRows * kD + 16 * i) = scaled_residue4(x[0][i], c2);
      *reinterpret_cast<half4_t *>(lo + 2 * kLoRows * kD + 16 * i) = scaled_residue4(x[1][i], 1.f);
    }
  }
  half_t *out[3] = {q16, k16, v16};
#pragma unroll
  for (int t = 0; t < 3; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<half4_t *>(out[t] + dst + 16 * i) =
          t == 0 ? round_scaled4(x[t][i], c2) : to_half4(x[t][i]);
}

// Relative cost of one step of each item kind (measured at C2: a dK/dV step,
// four products over a 64-row block, takes about 1.3 times a dQ step).
constexpr int kCostKvStep = 32;
constexpr int kCostQStep = 25;

// The main kernel reads fp16 copies of its inputs, written in [H][S][64]
// order by phase 1 (or, for c2*Q, K and V, by the training forward): c2*Q
// (c2 = scale*log2(e), the forward's rounding), K, V and sigma_b*dO (sigma_b
// the power-of-two scale of the row's 64-row block, sigma [H][n_blocks]).
struct BwdArgs {
  const half_t *Q16, *K16, *V16, *dO16, *lo16;
  const float *lse2n, *deltan, *sigma;
  float *dQ, *dK, *dV;
  int H, S, causal, n_blocks;
  int ldg;  // row stride of dQ, dK and dV in floats
  float scale;
};


// Direct-to-LDS fetch of rows row0 .. row0+127 of head `head` in an fp16
// copy ([H][S][64]) into a swizzled [128][64] LDS tile: wave w fetches rows
// 16w .. 16w+15 in two 1 KB pieces; lane l's 16 bytes land at byte 16*l of
// a piece, so it fetches the global granule the swizzle places there. Rows
// past S read as zeros. Two fetches per wave.
__device__ __forceinline__ void dma_rows128(const half_t *p, int head, int S, int row0, unsigned char *tile) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned nrec = (unsigned)max(0, min(S - row0, 128)) * kD * 2;
  const i32x4 rs = sgpr_rsrc(p + ((size_t)head * S + min(row0, S)) * kD, nrec);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = 16 * wave + 8 * j + (lane >> 3);
    lds_fetch16(rs, lds_addr32(tile + (16 * wave + 8 * j) * 128), row * 128 + (((lane & 7) ^ tile_swz(row)) << 4));
  }
}


// Partner waves (w, w+4) hold partial sums of the same 32x32 accumulator
// blocks. Each hands the N blocks it gives up to the other through LDS and
// adds the N it keeps from the other's slot, so both halves of the final
// sums (and of the output stores) are finished in parallel. LDS slot of wave
// w: 4N groups of 4 registers x 64 lanes, one 16-byte store per group and
// lane. The caller has ended all use of the staging tiles (a barrier) before;
// the buffer is not reused after.
template <int N>
__device__ __forceinline__ void exchange_pair(float *buf, int wave, int lane, f32x16 (&keep)[N],
                                              const f32x16 (&give)[N]) {
  float4 *mine = reinterpret_cast<float4 *>(buf) + (size_t)wave * 4 * N * 64;
  const float4 *theirs = reinterpret_cast<const float4 *>(buf) + (size_t)(wave ^ 4) * 4 * N * 64;
#pragma unroll
  for (int n = 0; n < N; ++n)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      mine[(4 * n + g) * 64 + lane] =
          make_float4(give[n][4 * g], give[n][4 * g + 1], give[n][4 * g + 2], give[n][4 * g + 3]);
  __syncthreads();
#pragma unroll
  for (int n = 0; n < N; ++n)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 v = theirs[(4 * n + g) * 64 + lane];
      keep[n][4 * g] += v.x;
      keep[n][4 * g + 1] += v.y;
      keep[n][4 * g + 2] += v.z;
      keep[n][4 * g + 3] += v.w;
    }
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
  return v;
}

// dK and dV of keys [kv_blk0, kv_blk0 + 128) of one head. Wave w owns keys
// kv_blk0 + 32*(w%4) .. +31 and query half w/4 of every 64-row block.
//
// Query block i (rows qb0 = 64*(first_qb + i) ..) goes through ring stage
// (i - i0) % 4, i0 being the number of blocks that hold the causal diagonal
// (two, or none without masking): in the unrolled steady loop the stage is
// a compile-time constant. The blocks are fetched straight into LDS and
// processed in pairs (see `pair` below).
__device__ void dkdv_path(const BwdArgs &a, int head, int kv_blk0, unsigned char *lds_raw) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, hh = lane >> 5;
  const int kg = wave & 3, qh = wave >> 2;
  const int S = a.S;
  const int ld = a.ldg, hoff = head * kD;
  const int key0 = kv_blk0 + kg * 32;  // this wave's first key
  const int key = key0 + c;

  // K^T / V^T fragments (B operands of S = Q K^T and dP = dO V^T): lane c
  // holds its key, slots d = 16*ds + 8*hh + j.
  // (Read from the workgroup's K/V tiles after the prologue; the rows of keys
  // kv_blk0 .. +127 are fetched with coalesced buffer loads first.)
  half8_t kf[4], vf[4];

  const int n_qblocks = (S + kQBlock - 1) / kQBlock;
  const int first_qb = a.causal ? kv_blk0 / kQBlock : 0;
  const int nb = max(n_qblocks - first_qb, 0);
  // Under causal masking the first two blocks hold the diagonal of the
  // workgroup's 128 keys; every later row sees every key.
  const int i0 = a.causal ? 2 : 0;
  // The workgroup of keys 0-127 adds the first block's rounding residues (kLoRows).
  const bool lo_corr = a.causal && kv_blk0 == 0;

  // Per-thread offsets, fixed for the whole loop: rows qh*32 + c of a tile
  // (A operands of S and dP), this wave's transposed reads (B operands of dV
  // and dK).
  int roff[4], troff[2][2][2];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) roff[ds] = tile_off(qh * 32 + c, 8 * (2 * ds + hh));
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        troff[j][db][hf] = tile_tr4_off(16 * (2 * qh + j) + 8 * hf + 4 * hh, 32 * db + 16 * ((lane >> 4) & 1), lane);
  // Direct-to-LDS staging of query block i (its c2*Q and sigma_b*dO rows,
  // its two row statistics and its dO scale) into ring stage st: wave w
  // fetches rows 8w .. 8w+7 of each tile (1 KB; lane l's 16 bytes land at
  // byte 16*l of the wave's kilobyte, so it fetches the global granule the
  // swizzle places there); waves 0 and 1 also fetch the 64 values of
  // -lse*log2(e) and -Delta*sigma_b, wave 2 the block's scale (and the next
  // ones', unused). Rows past S read as zeros (they then contribute nothing:
  // their Q and dO rows are zero too).
  auto stage_base = [&](int st) { return lds_raw + st * kStageBytes; };
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int drow = 8 * wave + (lane >> 3);
  const int dma_off = drow * 128 + (((lane & 7) ^ tile_swz(drow)) << 4);
  auto dma_block = [&](int i, int st) {
    const int qb0 = (first_qb + i) * kQBlock;
    const int rows = uniform_clamp0<kQBlock>(S - qb0);
    const size_t base = (size_t)head * S + min(qb0, S);
    const unsigned qt = lds_addr32(stage_base(st) + wave * 1024);
    lds_fetch16(sgpr_rsrc(a.Q16 + base * kD, (unsigned)rows * kD * 2), qt, dma_off);
    lds_fetch16(sgpr_rsrc(a.dO16 + base * kD, (unsigned)rows * kD * 2), qt + kTile * 2, dma_off);
    if (wave_u < 2)
      lds_fetch4(sgpr_rsrc((wave_u == 0 ? a.lse2n : a.deltan) + base, (unsigned)rows * 4),
                 lds_addr32(stage_base(st) + 2 * kTile * 2 + wave_u * kQBlock * 4), lane * 4);
    if (wave_u == 2) {
      const int qb = first_qb + i;
      const int left = uniform_clamp0<64>(a.n_blocks - qb);
      lds_fetch4(sgpr_rsrc(a.sigma + (size_t)head * a.n_blocks + min(qb, a.n_blocks), (unsigned)left * 4),
                 lds_addr32(stage_base(st) + kStageSigma), lane * 4);
    }
  };

  f32x16 dk[2], dv[2];
  dk[0] = dk[1] = dv[0] = dv[1] = f32x16{};
  // dO scales. The accumulators hold sig_min * (dK, dV), sig_min the
  // smallest dO scale of the blocks this item walks (that of the block of
  // largest magnitude). A block with a larger scale sig_b adds its products
  // scaled by sig_min / sig_b = 2^lr (lr a negative integer), which the
  // scores' starting values carry into P's exponent (dS = P (dP - Delta)
  // inherits the factor), so the accumulators never move to a larger unit and
  // cannot overflow for finite inputs; contributions that the factor pushes
  // below the fp16 range are negligible against the block of largest
  // magnitude. When every block has one scale (the usual case: blocks of
  // similar magnitude share it) no block's scale is read back.
  int sig_min;
  bool sig_uniform;
  {
    const float *sg = a.sigma + (size_t)head * a.n_blocks;
    const float s0 = sg[min(first_qb, a.n_blocks - 1)];
    float mn = s0;
    bool differs = false;
    for (int b = first_qb + lane; b < n_qblocks; b += 64) {
      const float sb = sg[b];
      differs |= sb != s0;
      mn = fminf(mn, sb);
    }
    sig_uniform = !__any(differs);
    sig_min = __builtin_amdgcn_readfirstlane(__float_as_int(sig_uniform ? s0 : wave_min(mn)));
  }

  // One block. `masked`: the block may hold the causal diagonal, so rows
  // below this wave's keys are masked and a wave whose rows are all below
  // its keys skips the block.
  auto compute = [&](int i, int st, bool masked) {
    const int q0 = (first_qb + i) * kQBlock + qh * 32;  // this wave's first query row
    if (masked && q0 + 31 < key0) return;
    const half_t *qt = reinterpret_cast<const half_t *>(stage_base(st));
    const half_t *gt = qt + kTile;
    const float *sl = reinterpret_cast<const float *>(gt + kTile);
    // S - lse2 and dP - Delta: register r is query q0 + 8*(r/4) + 4*hh + r%4
    // (lane = key); each chain starts from the rows' -lse2 / -Delta.
    f32x16 s, dp;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float4 nl = *reinterpret_cast<const float4 *>(sl + qh * 32 + g * 8 + hh * 4);
      const float4 nd = *reinterpret_cast<const float4 *>(sl + kQBlock + qh * 32 + g * 8 + hh * 4);
      s[4 * g] = nl.x; s[4 * g + 1] = nl.y; s[4 * g + 2] = nl.z; s[4 * g + 3] = nl.w;
      dp[4 * g] = nd.x; dp[4 * g + 1] = nd.y; dp[4 * g + 2] = nd.z; dp[4 * g + 3] = nd.w;
    }
    if (!sig_uniform) {
      const int sig_b = __builtin_amdgcn_readfirstlane(
          __float_as_int(*reinterpret_cast<const float *>(stage_base(st) + kStageSigma)));
      if (sig_b != sig_min) {
        const float lr = (float)(((sig_min >> 23) & 0xff) - ((sig_b >> 23) & 0xff));
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] += lr;
      }
    }
    half8_t qa[4], ga[4];
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      qa[ds] = *reinterpret_cast<const half8_t *>(qt + roff[ds]);
      ga[ds] = *reinterpret_cast<const half8_t *>(gt + roff[ds]);
    }
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      s = mfma32x32x16(qa[ds], kf[ds], s);
      dp = mfma32x32x16(ga[ds], vf[ds], dp);
    }
    // The transposed reads start after the products that consume qa and ga,
    // so their registers are free again (the exp of S hides the reads).
    __builtin_amdgcn_sched_barrier(0);
    // dO^T and (c2 Q)^T slots for this wave's two query steps.
    half8_t gtr[2][2], qtr[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const half4_t g0 = tile_tr4_at(gt, troff[j][db][0]), g1 = tile_tr4_at(gt, troff[j][db][1]);
        const half4_t q0v = tile_tr4_at(qt, troff[j][db][0]), q1v = tile_tr4_at(qt, troff[j][db][1]);
        gtr[j][db] = half8_t{g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
        qtr[j][db] = half8_t{q0v[0], q0v[1], q0v[2], q0v[3], q1v[0], q1v[1], q1v[2], q1v[3]};
      }
    // P and dS (dS overwrites dP).
    if (masked && q0 < key0 + 31) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (key > q0 + (r >> 2) * 8 + hh * 4 + (r & 3)) s[r] = -INFINITY;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = fast_exp2(s[r]);
      dp[r] *= s[r];
    }
    // dV += P^T dO, dK += dS^T (c2 Q): A from registers (lane = key).
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const half8_t pf = acc_to_slots(s, j);
      const half8_t dsf = acc_to_slots(dp, j);
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        dv[db] = mfma32x32x16(pf, gtr[j][db], dv[db]);
        dk[db] = mfma32x32x16(dsf, qtr[j][db], dk[db]);
      }
    }
    // Rows 0-63 (the first block of keys 0-127): the residues' products,
    // dV += P^T dO_lo, dK += dS^T (c2 Q)_lo + dS_lo^T (c2 Q).
    if (masked && lo_corr && i == 0) {
      const half_t *glo = reinterpret_cast<const half_t *>(lds_raw + kLoOffset);
      const half_t *qlo = glo + kTile;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const half8_t pf = acc_to_slots(s, j);
        const half8_t dsf = acc_to_slots(dp, j);
        half8_t dsl;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) dsl[jj] = (half_t)(dp[8 * j + jj] - (float)dsf[jj]);
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const half4_t g0 = tile_tr4_at(glo, troff[j][db][0]), g1 = tile_tr4_at(glo, troff[j][db][1]);
          const half4_t q0v = tile_tr4_at(qlo, troff[j][db][0]), q1v = tile_tr4_at(qlo, troff[j][db][1]);
          dv[db] = mfma32x32x16(pf, half8_t{g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]}, dv[db]);
          dk[db] = mfma32x32x16(dsf, half8_t{q0v[0], q0v[1], q0v[2], q0v[3], q1v[0], q1v[1], q1v[2], q1v[3]},
                                dk[db]);
          dk[db] = mfma32x32x16(dsl, qtr[j][db], dk[db]);
        }
      }
    }
  };

  // Blocks go through the ring in pairs: iteration k computes blocks i = 2k
  // and i+1 (stages st, st+1) after fetching blocks i+2 and i+3 into the
  // other two stages, which the previous iteration read, and ends with one
  // barrier once every fetch has landed. `all`: no range checks (blocks past
  // the end are fetched as zeros into stages no later iteration reads).
  auto pair = [&](int i, int st, bool masked, bool all) {
    if (all || i + 2 < nb) dma_block(i + 2, (st + 2) & 3);
    if (all || i + 3 < nb) dma_block(i + 3, (st + 3) & 3);
    compute(i, st, masked);
    if (all || i + 1 < nb) compute(i + 1, (st + 1) & 3, masked);
    lds_fetch_barrier<0>();
  };

  // Prologue: the workgroup's K and V rows and blocks 0 and 1 are fetched
  // straight into LDS (blocks past the end into stages nothing reads).
  dma_rows128(a.K16, head, S, kv_blk0, lds_raw + kOwnOffset);
  dma_rows128(a.V16, head, S, kv_blk0, lds_raw + kOwnOffset + kOwnTile * 2);
  dma_block(0, (0 - i0) & 3);
  dma_block(1, (1 - i0) & 3);
  // The residue tiles of rows 0-63 (the first block) for the workgroup of
  // keys 0-127 (rows past S read as zeros).
  if (lo_corr) {
    const unsigned nrec = (unsigned)min(S, kLoRows) * kD * 2;
    const half_t *lo = a.lo16 + (size_t)head * kLoTiles * kLoRows * kD;
    const unsigned lt = lds_addr32(lds_raw + kLoOffset + wave * 1024);
    lds_fetch16(sgpr_rsrc(lo, nrec), lt, dma_off);
    lds_fetch16(sgpr_rsrc(lo + kLoRows * kD, nrec), lt + kTile * 2, dma_off);
  }
  lds_fetch_barrier<0>();
  {
    // K^T / V^T fragments (B operands of S = Q K^T and dP = dO V^T): lane c
    // holds key key0 + c, slots d = 16*ds + 8*hh + j.
    const half_t *own = reinterpret_cast<const half_t *>(lds_raw + kOwnOffset);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      kf[ds] = *reinterpret_cast<const half8_t *>(own + tile_off(kg * 32 + c, 8 * (2 * ds + hh)));
      vf[ds] = *reinterpret_cast<const half8_t *>(own + kOwnTile + tile_off(kg * 32 + c, 8 * (2 * ds + hh)));
    }
  }

  int i = 0;
  // Under causal masking blocks 0 and 1 hold the diagonal (stages 2 and 3).
  if (i0 > 0 && nb > 0) {
    pair(0, (0 - i0) & 3, true, false);
    i = 2;
  }
  // Steady state: no mask, every wave active; the stages are constants
  // (i - i0 is a multiple of 4 at the top of each trip).
  for (; i + 4 <= nb; i += 4) {
    pair(i, 0, false, true);
    pair(i + 2, 2, false, true);
  }
  for (; i < nb; i += 2) pair(i, (i - i0) & 3, false, false);
  // Fetches of blocks past the end may still be landing in the ring, which
  // the exchange below reuses.
  lds_fetch_barrier<0>();

  // Wave w finishes dK and wave w+4 dV of the same 32 keys.
  float *buf = reinterpret_cast<float *>(lds_raw);
  if (qh == 0)
    exchange_pair<2>(buf, wave, lane, dk, dv);
  else
    exchange_pair<2>(buf, wave, lane, dv, dk);

  // dK = scale * dS^T Q = ln2 * dS^T (c2 Q) / sigma, dV = P^T dO / sigma; row
  // r is key key0 + 8*(r/4) + 4*hh + r%4, column d = 32*db + c.
  // (Each wave picks its result by value: a pointer chosen between the two
  // register arrays would put both in scratch memory.)
  f32x16 res[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) res[db][r] = qh == 0 ? dk[db][r] : dv[db][r];
  float *out = qh == 0 ? a.dK : a.dV;
  const float sigma = __int_as_float(sig_min);
  const float out_scale = qh == 0 ? kLn2 / sigma : 1.f / sigma;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int kr = key0 + (r >> 2) * 8 + hh * 4 + (r & 3);
    if (kr < S) {
      float *row = out + (size_t)kr * ld + hoff;
#pragma unroll
      for (int db = 0; db < 2; ++db) row[db * 32 + c] = res[db][r] * out_scale;
    }
  }
}

// dQ of query rows [q_blk0, q_blk0 + 128) of one head. Wave w owns rows
// q_blk0 + 32*(w%4) .. +31 and key half w/4 of every 64-key tile.
__device__ void dq_path(const BwdArgs &a, int head, int q_blk0, unsigned char *lds_raw) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, hh = lane >> 5;
  const int qg = wave & 3, kh = wave >> 2;
  const int S = a.S;
  const size_t ld = (size_t)a.ldg, hoff = (size_t)head * kD;
  const int q_w0 = q_blk0 + qg * 32;
  const int query = q_w0 + c;
  const bool q_ok = query < S;
  const bool wave_active = q_w0 < S;
  const int wave_qlast = min(q_w0 + 32, S) - 1;
  // Keys above key_lim are masked for this lane's row; no key of a half tile
  // starting at k0 is masked for any row of the wave when k0 + 31 <= key_lim_lo.
  const int key_lim = a.causal ? min(query, S - 1) : S - 1;
  const int key_lim_lo = a.causal ? min(q_w0, S - 1) : S - 1;
  // The workgroup of rows 0-127 adds the residues of keys 0-63 (kLoRows).
  const bool lo_corr = a.causal && q_blk0 == 0;

  half8_t qf[4], gf[4];
  f32x16 negL, negD;

  const int kv_end = a.causal ? min(S, q_blk0 + kQueriesPerWg) : S;
  const int n_tiles = (kv_end + kKTile - 1) / kKTile;
  // Tiles below n_full need no mask for any row of the workgroup (causal:
  // every key is below the first row; otherwise every key is below S). They
  // run first, software-pipelined; the rest take the general loop.
  const int n_full = a.causal ? min(q_blk0 / kKTile, n_tiles) : S / kKTile;

  // Per-thread offsets: K/V rows kh*32 + c (A operands of S^T and dP^T) and
  // K^T slots through transposed reads (A operand of dQ^T).
  int koff[4], ktoff[2][2][2];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) koff[ds] = tile_off(kh * 32 + c, 8 * (2 * ds + hh));
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
        ktoff[j][db][hf] = tile_tr4_off(16 * (2 * kh + j) + 8 * hf + 4 * hh, 32 * db + 16 * ((lane >> 4) & 1), lane);
  // Tile t goes through ring stage t % 4; tile t+3 is fetched at the start
  // of iteration t (into the stage last read in iteration t-1). Keys past S
  // read as zeros and are masked to P = 0.
  auto stage_base = [&](int st) { return reinterpret_cast<half_t *>(lds_raw + st * kStageBytes); };
  // Direct-to-LDS: wave w fetches rows 8w .. 8w+7 of each K and V tile (1 KB
  // each); lane l's 16 bytes land at byte 16*l of the wave's kilobyte, so
  // it fetches the global granule the swizzle places there.
  const int drow = 8 * wave + (lane >> 3);
  const int dma_off = drow * 128 + (((lane & 7) ^ tile_swz(drow)) << 4);
  auto dma_tile = [&](int t, int st) {
    const unsigned kt = lds_addr32(lds_raw + st * kStageBytes + wave * 1024);
    const int row0 = t * kKTile;
    const unsigned nrec = (unsigned)uniform_clamp0<kKTile>(S - row0) * kD * 2;
    const size_t base = ((size_t)head * S + min(row0, S)) * kD;
    lds_fetch16(sgpr_rsrc(a.K16 + base, nrec), kt, dma_off);
    lds_fetch16(sgpr_rsrc(a.V16 + base, nrec), kt + kTile * 2, dma_off);
  };

  f32x16 dq[2];
  dq[0] = dq[1] = f32x16{};

  // Scores of the tile in stage st: S^T - lse2 and dP^T - Delta, register r
  // is key k0 + 8*(r/4) + 4*hh + r%4 (lane = query); the chains start from
  // the lane's -lse2 / -Delta.
  auto scores = [&](int st, f32x16 &s, f32x16 &dp) {
    const half_t *kt = stage_base(st);
    const half_t *vt = kt + kTile;
    half8_t ka[4], va[4];
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      ka[ds] = *reinterpret_cast<const half8_t *>(kt + koff[ds]);
      va[ds] = *reinterpret_cast<const half8_t *>(vt + koff[ds]);
    }
    s = mfma32x32x16(ka[0], qf[0], negL);
    dp = mfma32x32x16(va[0], gf[0], negD);
#pragma unroll
    for (int ds = 1; ds < 4; ++ds) {
      s = mfma32x32x16(ka[ds], qf[ds], s);
      dp = mfma32x32x16(va[ds], gf[ds], dp);
    }
  };
  // The gradient work of tile t (stage st) from its scores: dS = P * (dP -
  // Delta) (the mask first when `masked`), then dQ^T += K^T dS^T over this
  // wave's two key steps.
  auto grads = [&](int t, int st, f32x16 &s, f32x16 &dp, bool masked) {
    const half_t *kt = stage_base(st);
    half8_t ktr[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        const half4_t lo = tile_tr4_at(kt, ktoff[j][db][0]), hi = tile_tr4_at(kt, ktoff[j][db][1]);
        ktr[j][db] = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    if (masked) {
      const int k0 = t * kKTile + kh * 32;
      if (k0 + 31 > key_lim_lo) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0 + (r >> 2) * 8 + hh * 4 + (r & 3) > key_lim) s[r] = -INFINITY;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) dp[r] *= fast_exp2(s[r]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const half8_t dsf = acc_to_slots(dp, j);
#pragma unroll
      for (int db = 0; db < 2; ++db) dq[db] = mfma32x32x16(ktr[j][db], dsf, dq[db]);
    }
    // Keys 0-63 (tile 0) of rows 0-127: dQ^T += K_lo^T dS^T + K^T dS_lo^T.
    if (masked && lo_corr && t == 0) {
      const half_t *klo = reinterpret_cast<const half_t *>(lds_raw + kLoOffset);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const half8_t dsf = acc_to_slots(dp, j);
        half8_t dsl;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) dsl[jj] = (half_t)(dp[8 * j + jj] - (float)dsf[jj]);
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const half4_t lo = tile_tr4_at(klo, ktoff[j][db][0]), hi = tile_tr4_at(klo, ktoff[j][db][1]);
          dq[db] = mfma32x32x16(half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}, dsf, dq[db]);
          dq[db] = mfma32x32x16(ktr[j][db], dsl, dq[db]);
        }
      }
    }
  };
  // One tile, unpipelined. `masked`: the tile may hold the causal diagonal or
  // the end of the keys; a wave that sees none of it skips it.
  auto compute = [&](int t, int st, bool masked) {
    const int k0 = t * kKTile + kh * 32;  // first key of this wave's half tile
    if (masked && !(wave_active && k0 < S && (!a.causal || k0 <= wave_qlast))) return;
    f32x16 s, dp;
    scores(st, s, dp);
    grads(t, st, s, dp, masked);
  };

  // Prologue: the workgroup's c2*Q and sigma*dO rows, its rows' -lse*log2(e)
  // and -Delta*sigma (waves 0-3, 64 values each) and tiles 0-2 are fetched
  // straight into LDS (tiles past the end into stages nothing reads); the
  // first products wait for all but tiles 1 and 2.
  dma_rows128(a.Q16, head, S, q_blk0, lds_raw + kOwnOffset);
  dma_rows128(a.dO16, head, S, q_blk0, lds_raw + kOwnOffset + kOwnTile * 2);
  // The residue tile of K's rows 0-63 for the workgroup of rows 0-127 (keys
  // past S read as zeros).
  if (lo_corr) {
    const unsigned nrec = (unsigned)min(S, kLoRows) * kD * 2;
    lds_fetch16(sgpr_rsrc(a.lo16 + ((size_t)head * kLoTiles + 2) * kLoRows * kD, nrec),
                lds_addr32(lds_raw + kLoOffset + wave * 1024), dma_off);
  }
  {
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    if (wave_u < 4) {
      const int row0 = q_blk0 + 64 * (wave_u & 1);
      const unsigned nrec = (unsigned)max(0, min(S - row0, 64)) * 4;
      const float *stat = (wave_u < 2 ? a.lse2n : a.deltan) + (size_t)head * S + min(row0, S);
      lds_fetch4(sgpr_rsrc(stat, nrec), lds_addr32(lds_raw + kRowStatOffset + wave_u * 256), lane * 4);
    }
  }
#pragma unroll
  for (int p = 0; p < 3; ++p) dma_tile(p, p);
  lds_fetch_barrier<2>();  // tiles 0 and 1 have landed
  {
    // The lane's -lse*log2(e) and -Delta*sigma (rows past S: P = 0), and the
    // (c2 Q)^T and (sigma dO)^T fragments (B operands): lane c holds query
    // q_w0 + c, slots d = 16*ds + 8*hh + j.
    const float *rs = reinterpret_cast<const float *>(lds_raw + kRowStatOffset);
    const float nl = q_ok ? rs[qg * 32 + c] : -INFINITY;
    const float nd = q_ok ? rs[128 + qg * 32 + c] : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      negL[r] = nl;
      negD[r] = nd;
    }
    const half_t *own = reinterpret_cast<const half_t *>(lds_raw + kOwnOffset);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      qf[ds] = *reinterpret_cast<const half8_t *>(own + tile_off(qg * 32 + c, 8 * (2 * ds + hh)));
      gf[ds] = *reinterpret_cast<const half8_t *>(own + kOwnTile + tile_off(qg * 32 + c, 8 * (2 * ds + hh)));
    }
  }

  // Unmasked tiles 0 .. n_full-1, software-pipelined: iteration t issues the
  // scores of tile t+1 (stage t+1) before the gradient work of tile t
  // (stage t), which does not depend on them, so the products of one run
  // beside the exponentials of the other. Tile t+3 is fetched at the start
  // of iteration t into the stage last read in iteration t-1; the barrier at
  // the end leaves tile t+2 landed, with tile t+3 in flight.
  int t = 0;
  if (n_full > 0) {
    f32x16 s, dp;
    scores(0, s, dp);
    auto iter = [&](int tt, int st, int stn) {
      dma_tile(tt + 3, (st + 3) & 3);
      f32x16 sn, dpn;
      scores(stn, sn, dpn);
      grads(tt, st, s, dp, false);
      s = sn;
      dp = dpn;
      lds_fetch_barrier<2>();
    };
    for (; t + 4 < n_full; t += 4) {
      iter(t, 0, 1);
      iter(t + 1, 1, 2);
      iter(t + 2, 2, 3);
      iter(t + 3, 3, 0);
    }
    for (; t + 1 < n_full; ++t) iter(t, t & 3, (t + 1) & 3);
    // The last unmasked tile: its gradient work, and the fetch that
    // iteration t would have issued.
    if (t + 3 < n_tiles) dma_tile(t + 3, (t + 3) & 3);
    grads(t, t & 3, s, dp, false);
    lds_fetch_barrier<0>();
    ++t;
  }
  // The rest (masked tiles, and the keys' end), unpipelined: tile t has
  // landed at the top of each iteration.
  for (; t < n_tiles; ++t) {
    if (t + 3 < n_tiles) dma_tile(t + 3, (t + 3) & 3);
    compute(t, t & 3, true);
    lds_fetch_barrier<0>();
  }
  // Fetches of tiles past the end may still be landing in the ring, which
  // the exchange below reuses.
  lds_fetch_barrier<0>();

  // Wave w finishes columns 0-31 of dQ and wave w+4 columns 32-63 of the
  // same 32 rows (each gives up the other block).
  f32x16 res[1] = {kh == 0 ? dq[0] : dq[1]};
  const f32x16 give[1] = {kh == 0 ? dq[1] : dq[0]};
  exchange_pair<1>(reinterpret_cast<float *>(lds_raw), wave, lane, res, give);

  // dQ = scale * dS K / sigma_b, sigma_b the dO scale of the wave's 64-row
  // block; register r of block db is column 32*db + 8*(r/4) + 4*hh + r%4.
  if (q_ok) {
    const float sigma = a.sigma[(size_t)head * a.n_blocks + q_w0 / kPreRows];
    const float dq_scale = a.scale / sigma;
    float *qrow = a.dQ + (size_t)query * ld + hoff + kh * 32;
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4 *>(qrow + g * 8 + hh * 4) =
          make_float4(res[0][4 * g] * dq_scale, res[0][4 * g + 1] * dq_scale, res[0][4 * g + 2] * dq_scale,
                      res[0][4 * g + 3] * dq_scale);
  }
}

// Dispatch order. A dK/dV item of key rank i (keys 128*i ..) walks
// steps_kv(i) query blocks, a dQ item of query rank j (the j-th longest
// query tile) steps_q(j) key tiles; their costs are w_kv and w_q per step
// (a dK/dV step runs four products, a dQ step three). Workgroup b takes the
// b-th item of both lists merged by decreasing cost (each rank contributes
// one item per head), so the greedy dispatcher approximates a
// longest-processing-time schedule, and consecutive items, which the
// dispatcher deals to different XCDs, mix both kinds.
//
// When the whole grid fits in `wg`, the items are also kept on the XCD of
// their head: the dispatcher deals workgroup b to XCD b % 8, so position
// b = 8j + x holds the j-th item of XCD x's list. XCD x takes every head
// h < H - H%8 with h % 8 == x, and the H%8 remaining heads are each shared
// by 8/(H%8) XCDs, item by item in merged order; each list keeps the merged
// (cost) order. A head's fp16 copies then stay in the L2 of one or two XCDs
// instead of being fetched into all eight. Head counts that do not divide
// that way keep the plain order.
constexpr int kSchedTable = 512;  // merged ranks listed in the kernel arguments when they fit
constexpr int kWgTable = 768;     // workgroups listed one by one when the grid fits
struct Sched {
  int n_qblocks, n_qtiles, S, causal, w_kv, w_q, r_kv, r_q;
  int use_table;
  unsigned short table[kSchedTable];  // (is dK/dV) << 15 | rank, in merged order
  int use_wg;
  unsigned short wg[kWgTable];  // per workgroup: (is dK/dV) << 15 | head << 11 | rank
  __host__ __device__ int cost_kv(int i) const {
    const int first_qb = causal ? i * (kKeysPerWg / kQBlock) : 0;
    return w_kv * max(n_qblocks - first_qb, 0);
  }
  __host__ __device__ int cost_q(int j) const {
    const int qtile = causal ? n_qtiles - 1 - j : j;
    const int kv_end = causal ? min(S, (qtile + 1) * kQueriesPerWg) : S;
    return w_q * ((kv_end + kKTile - 1) / kKTile);
  }
  // Number of query ranks costlier than x (cost_q does not increase with j).
  __host__ __device__ int q_above(int x) const {
    int lo = 0, hi = r_q;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (cost_q(mid) > x) lo = mid + 1; else hi = mid;
    }
    return lo;
  }
  // Rank k of the merged list (ties: dK/dV first) -> (is dK/dV, rank).
  __host__ __device__ void pick(int k, bool &kv, int &rank) const {
    int lo = 0, hi = r_kv;  // count of dK/dV ranks merged before position k
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (mid + q_above(cost_kv(mid)) < k) lo = mid + 1; else hi = mid;
    }
    kv = lo < r_kv && lo + q_above(cost_kv(lo)) == k;
    rank = kv ? lo : k - lo;
  }
};

__global__ __launch_bounds__(kThreads) void bwd_main_kernel(BwdArgs a, Sched sched) {
  __shared__ __attribute__((aligned(16))) unsigned char lds_raw[kLdsBytes];
  const int b = blockIdx.x;
  bool kv_item;
  int rank, head;
  if (sched.use_wg) {
    const unsigned t = sched.wg[b];
    kv_item = (t >> 15) != 0;
    head = (int)((t >> 11) & 15);
    rank = (int)(t & 0x7ff);
  } else {
    head = b % a.H;
    if (sched.use_table) {
      const unsigned t = sched.table[b / a.H];
      kv_item = (t >> 15) != 0;
      rank = (int)(t & 0x7fff);
    } else {
      sched.pick(b / a.H, kv_item, rank);
    }
  }
  // The item is the same for the whole workgroup; saying so keeps every
  // address and buffer descriptor derived from it in scalar registers (the
  // table entry arrives through a vector load).
  rank = __builtin_amdgcn_readfirstlane(rank);
  head = __builtin_amdgcn_readfirstlane(head);
  kv_item = __builtin_amdgcn_readfirstlane(kv_item ? 1 : 0) != 0;
  if (kv_item) {
    dkdv_path(a, head, rank * kKeysPerWg, lds_raw);
  } else {
    const int qtile = a.causal ? sched.n_qtiles - 1 - rank : rank;
    dq_path(a, head, qtile * kQueriesPerWg, lds_raw);
  }
}

}  // namespace

size_t bwd_workspace_bytes_d64(int n_heads, int seq_len) { return ws_layout(n_heads, seq_len).total; }

void bwd_ws_qkv_copies(void *workspace, int n_heads, int seq_len, half_t **q16, half_t **k16, half_t **v16,
                       half_t **qlo, int *qlo_head_stride) {
  const WsLayout w = ws_layout(n_heads, seq_len);
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  *q16 = reinterpret_cast<half_t *>(ws + w.q16);
  *k16 = reinterpret_cast<half_t *>(ws + w.k16);
  *v16 = reinterpret_cast<half_t *>(ws + w.v16);
  *qlo = reinterpret_cast<half_t *>(ws + w.lo16) + kLoRows * kD;
  *qlo_head_stride = kLoTiles * kLoRows * kD;
}

hipError_t launch_bwd_pre_d64(const float *q, const float *k, const float *v, const float *o,
                              const float *d_o, const float *lse, void *workspace, int n_heads, int seq_len,
                              float scale, hipStream_t stream, bool qkv_saved, int ldi) {
  const WsLayout w = ws_layout(n_heads, seq_len);
  unsigned char *ws = static_cast<unsigned char *>(workspace);
  hipLaunchKernelGGL(bwd_prep_kernel, dim3(pre_blocks(seq_len), n_heads), dim3(256), 0, stream, q, k, v, o, d_o,
                     lse, reinterpret_cast<float *>(ws + w.sigma), reinterpret_cast<float *>(ws + w.lse2n),
                     reinterpret_cast<float *>(ws + w.deltan), reinterpret_cast<half_t *>(ws + w.q16),
                     reinterpret_cast<half_t *>(ws + w.k16), reinterpret_cast<half_t *>(ws + w.v16),
                     reinterpret_cast<half_t *>(ws + w.do16), reinterpret_cast<half_t *>(ws + w.lo16), n_heads,
                     seq_len, scale * kLog2e,
                     qkv_saved ? 0 : 1, ldi > 0 ? ldi : n_heads * kD);
  return hipGetLastError();
}

// Fills sched.wg with the XCD-local order (see Sched) from the merged table;
// leaves use_wg = 0 when the grid or the head count does not allow it.
void build_xcd_order(Sched &sched, int n_heads) {
  constexpr int kXcds = 8;
  sched.use_wg = 0;
  const int per = sched.r_kv + sched.r_q;  // items per head
  const int n = n_heads * per;
  const int rest = n_heads % kXcds, full = n_heads - rest;
  const int share = rest ? kXcds / rest : 1;  // XCDs per remaining head
  if (!sched.use_table || n > kWgTable || n_heads > 16 || sched.r_kv > 0x7ff || sched.r_q > 0x7ff) return;
  if (rest && (kXcds % rest != 0 || per % share != 0)) return;
  // Per-XCD lists on the stack (no host allocation per launch).
  unsigned short lists[kXcds][kWgTable];
  int len[kXcds] = {};
  for (int k = 0; k < per; ++k) {
    const unsigned t = sched.table[k];
    for (int h = 0; h < n_heads; ++h) {
      const int x = h < full ? h % kXcds : (h - full) * share + k % share;
      lists[x][len[x]++] = (unsigned short)((t & 0x8000u) | ((unsigned)h << 11) | (t & 0x7ffu));
    }
  }
  for (int x = 0; x < kXcds; ++x)
    if (len[x] * kXcds != n) return;
  for (int b = 0; b < n; ++b) sched.wg[b] = lists[b % kXcds][b / kXcds];
  sched.use_wg = 1;
}

hipError_t launch_bwd_main_d64(const float *lse, float *d_q, float *d_k, float *d_v, const void *workspace,
                               int n_heads, int seq_len, float scale, bool causal, hipStream_t stream,
                               int ldg) {
  const WsLayout w = ws_layout(n_heads, seq_len);
  const unsigned char *ws = static_cast<const unsigned char *>(workspace);
  BwdArgs a;
  a.Q16 = reinterpret_cast<const half_t *>(ws + w.q16);
  a.K16 = reinterpret_cast<const half_t *>(ws + w.k16);
  a.V16 = reinterpret_cast<const half_t *>(ws + w.v16);
  a.dO16 = reinterpret_cast<const half_t *>(ws + w.do16);
  a.lo16 = reinterpret_cast<const half_t *>(ws + w.lo16);
  a.lse2n = reinterpret_cast<const float *>(ws + w.lse2n);
  a.deltan = reinterpret_cast<const float *>(ws + w.deltan);
  a.sigma = reinterpret_cast<const float *>(ws + w.sigma);
  a.dQ = d_q;
  a.dK = d_k;
  a.dV = d_v;
  a.H = n_heads;
  a.S = seq_len;
  a.causal = causal ? 1 : 0;
  a.n_blocks = pre_blocks(seq_len);
  a.scale = scale;
  a.ldg = ldg > 0 ? ldg : n_heads * kD;
  Sched sched;
  sched.n_qblocks = (seq_len + kQBlock - 1) / kQBlock;
  sched.n_qtiles = (seq_len + kQueriesPerWg - 1) / kQueriesPerWg;
  sched.S = seq_len;
  sched.causal = causal ? 1 : 0;
  sched.w_kv = kCostKvStep;
  sched.w_q = kCostQStep;
  sched.r_kv = (seq_len + kKeysPerWg - 1) / kKeysPerWg;
  sched.r_q = sched.n_qtiles;
  // The merged order, computed here once when it fits in the arguments (the
  // in-kernel search costs each workgroup about 2 us).
  sched.use_table = sched.r_kv + sched.r_q <= kSchedTable ? 1 : 0;
  for (int k = 0; k < kSchedTable; ++k) {
    bool kv = false;
    int rank = 0;
    if (sched.use_table && k < sched.r_kv + sched.r_q) sched.pick(k, kv, rank);
    sched.table[k] = (unsigned short)((kv ? 0x8000u : 0u) | (unsigned)rank);
  }
  build_xcd_order(sched, n_heads);
  const unsigned n_items = (unsigned)(n_heads * (sched.r_kv + sched.r_q));
  hipLaunchKernelGGL(bwd_main_kernel, dim3(n_items), dim3(kThreads), 0, stream, a, sched);
  return hipGetLastError();
}

hipError_t launch_bwd_d64(const float *q, const float *k, const float *v, const float *o,
                          const float *d_o, const float *lse, float *d_q, float *d_k,
                          float *d_v, void *workspace, int n_heads, int seq_len, float scale,
                          bool causal, hipStream_t stream) {
  hipError_t err = launch_bwd_pre_d64(q, k, v, o, d_o, lse, workspace, n_heads, seq_len, scale, stream);
  if (err != hipSuccess) return err;
  return launch_bwd_main_d64(lse, d_q, d_k, d_v, workspace, n_heads, seq_len, scale, causal, stream);
}

}  // namespace dfattn
