// attn_bwd_d64.hip — fused causal attention backward for d_head = 64 on gfx950.
//
// Replaces kernel_mha_bwd_all_heads (darkforest-cuda/kernels/attention_fused.cu:390-516),
// which recomputes each row's softmax with four serial passes over the keys,
// stores P and dS in an [H, 2, S, S] fp32 scratch and accumulates dK and dV
// with one atomicAdd per (query, key, d). Here:
//
//  1. bwd_preprocess: Delta_i = dO_i . O_i per (head, row), the per-block
//     max |dO| (for a power-of-two operand scale of dO, see below), and dQ := 0.
//  2. bwd_main: a workgroup owns BN = 32*WAVES keys of one head (each wave 32
//     of them, with its K and V rows held in registers) and streams the query
//     rows in blocks of BM = 64 through LDS. Per block, on MFMA:
//        S2 = (c2 Q) K^T, dP = dO V^T           (queries x keys, lane = key)
//        P  = exp2(S2 - lse*log2e)              (recomputed from the forward's lse)
//        dS = P * (dP - Delta)
//        dV += P^T dO, dK += dS^T Q              (keys x d, in registers)
//        dQ += dS K                              (fp32 atomics into dQ)
//     dK and dV are written once at the end; no O(S^2) memory is touched.
//
// Numerics. Operands are fp16 (rounded from the fp32 inputs on load),
// accumulation and softmax fp32. Two rules keep the result within 2e-3
// max-abs of the fp32 reference without any split-precision products:
//  * the scores are recomputed with exactly the forward's rounding: Q is
//    multiplied by c2 = scale*log2(e) before it is rounded, as in
//    attn_fwd_d64.hip, so P's rows sum to one against the forward's lse;
//  * Delta is formed from the same fp16-rounded dO that dP is formed from,
//    so sum_j dS_ij = 0 holds for the rounded operands.
// The backward is then the exact gradient of attention on fp16-rounded
// inputs. dO is multiplied by a per-head power of two sigma before rounding,
// chosen so max|sigma*dO| lies in [8, 16): training gradients are often far
// below fp16's normal range. The results are divided by sigma exactly.
#include "dfattn_internal.h"

namespace dfattn {
namespace {

constexpr int kPreRows = 64;  // rows per preprocess workgroup

// Workspace layout (floats): delta [H*S] | dO block max [H*ceil(S/64)].
inline size_t ws_delta_floats(int H, int S) { return (size_t)H * S; }
inline int pre_blocks(int S) { return (S + kPreRows - 1) / kPreRows; }

// Power of two sigma with max|sigma * x| in [8, 16) for amax = max|x|; 1 if
// amax is 0 or not finite. Both kernels derive sigma from block maxima with
// this one function.
__device__ __forceinline__ float pow2_scale(float amax) {
  if (!(amax > 0.f) || !(amax < INFINITY)) return 1.f;
  const int e = max(-126, min(126, 3 - ilogbf(amax)));
  return ldexpf(1.f, e);
}

__device__ __forceinline__ float round_f16(float x) { return (float)(half_t)x; }

// One workgroup (256 threads) handles kPreRows = 64 rows of one head, d_head
// = 64: thread t owns row t/4 and columns 16*(t%4) .. 16*(t%4)+15.
// Delta of a row is summed from fp16(sigma_b * dO) * O / sigma_b, sigma_b the
// block's own scale. The main kernel rounds sigma_h * dO with the head's
// sigma_h <= sigma_b, both powers of two, so both roundings agree wherever
// sigma_h * dO is an fp16 normal number.
__global__ __launch_bounds__(256) void bwd_preprocess_kernel(
    const float *__restrict__ O, const float *__restrict__ dO, float *__restrict__ dQ,
    float *__restrict__ delta, float *__restrict__ blockmax, int H, int S) {
  __shared__ float wmax[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int head = blockIdx.y;
  const int row = blockIdx.x * kPreRows + (tid >> 2);
  const bool ok = row < S;
  const size_t base = ok ? (size_t)row * H * 64 + (size_t)head * 64 + (tid & 3) * 16 : 0;
  float4 g[4], o[4];
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    g[i] = load4_or_zero(dO + base + 4 * i, ok);
    o[i] = load4_or_zero(O + base + 4 * i, ok);
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(g[i].x), fabsf(g[i].y)), fmaxf(fabsf(g[i].z), fabsf(g[i].w))));
  }
  mx = wave_max(mx);
  if (lane == 0) wmax[wave] = mx;
  __syncthreads();
  const float bmax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const float sig = pow2_scale(bmax);
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc += round_f16(g[i].x * sig) * o[i].x;
    acc += round_f16(g[i].y * sig) * o[i].y;
    acc += round_f16(g[i].z * sig) * o[i].z;
    acc += round_f16(g[i].w * sig) * o[i].w;
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  if (ok) {
    if ((tid & 3) == 0) delta[(size_t)head * S + row] = acc / sig;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<float4 *>(dQ + base + 4 * i) = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (tid == 0) blockmax[(size_t)head * gridDim.x + blockIdx.x] = bmax;
}

template <int WAVES>
struct BwdCfg {
  static constexpr int D = 64;
  static constexpr int BN = 32 * WAVES;  // keys per workgroup
  static constexpr int BM = 64;          // query rows per iteration
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int QS = D + 8;       // [BM][QS] row-major Q and dO
  static constexpr int TS = BM + 8;      // [D][TS] transposed Q^T and dO^T
  static constexpr int DSS = BN + 8;     // [BM][DSS] dS
  static constexpr int KTS = BN + 8;     // [D][KTS] K^T
  static constexpr int PAIRS = (BM / 2) * (D / 4) / THREADS;  // staging items per thread
  static_assert(PAIRS * THREADS * 8 == BM * D, "staging split");
  static constexpr int OFF_Q = 0;
  static constexpr int OFF_QT = OFF_Q + BM * QS;
  static constexpr int OFF_DO = OFF_QT + D * TS;
  static constexpr int OFF_DOT = OFF_DO + BM * QS;
  static constexpr int OFF_DS = OFF_DOT + D * TS;
  static constexpr int OFF_KT = OFF_DS + BM * DSS;
  static constexpr int HALVES = OFF_KT + D * KTS;
  static constexpr int DQ_TILES = 4 / WAVES > 0 ? 4 / WAVES : 1;  // 32x32 dQ tiles per wave
  static_assert(WAVES == 1 || WAVES == 2 || WAVES == 4, "waves");
};

__device__ __forceinline__ float f4at(const float4 &v, int e) {
  return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

template <int WAVES>
__global__ __launch_bounds__(64 * WAVES) void bwd_main_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    const float *__restrict__ dO, const float *__restrict__ LSE,
    const float *__restrict__ delta, const float *__restrict__ blockmax,
    float *__restrict__ dQ, float *__restrict__ dK, float *__restrict__ dV, int H, int S,
    float scale, int causal, int n_pre_blocks) {
  using C = BwdCfg<WAVES>;
  __shared__ __attribute__((aligned(16))) half_t lds[C::HALVES];
  __shared__ __attribute__((aligned(16))) float lse2_lds[C::BM];
  __shared__ __attribute__((aligned(16))) float delta_lds[C::BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, hh = lane >> 5;
  const int head = blockIdx.x % H;
  const int kvtile = blockIdx.x / H;  // tile 0 sees the most queries: launched first
  const size_t ld = (size_t)H * C::D;
  const size_t hoff = (size_t)head * C::D;
  const int kv_blk0 = kvtile * C::BN;
  const int key = kv_blk0 + wave * 32 + c;  // this lane's key (B/A operand column)
  const bool key_ok = key < S;

  // Per-head power-of-two scale of dO.
  float gmax = 0.f;
  for (int i = lane; i < n_pre_blocks; i += 64)
    gmax = fmaxf(gmax, blockmax[(size_t)head * n_pre_blocks + i]);
  gmax = wave_max(gmax);
  const float sigma = pow2_scale(gmax);
  const float inv_sigma = 1.f / sigma;
  const float c2 = scale * kLog2e;

  half_t *q_lds = lds + C::OFF_Q, *qt_lds = lds + C::OFF_QT;
  half_t *do_lds = lds + C::OFF_DO, *dot_lds = lds + C::OFF_DOT;
  half_t *ds_lds = lds + C::OFF_DS, *kt_lds = lds + C::OFF_KT;

  // K^T / V^T fragments (B operands of S = Q K^T and dP = dO V^T): lane c
  // holds this lane's key, slots d = 16*ds + 8*hh + j. K^T also goes to LDS
  // for the dQ product.
  half8_t kf[4], vf[4];
  {
    const float *kp = K + (key_ok ? (size_t)key * ld + hoff : 0);
    const float *vp = V + (key_ok ? (size_t)key * ld + hoff : 0);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      const half4_t k0 = to_half4(load4_or_zero(kp + ds * 16 + hh * 8, key_ok));
      const half4_t k1 = to_half4(load4_or_zero(kp + ds * 16 + hh * 8 + 4, key_ok));
      const half4_t v0 = to_half4(load4_or_zero(vp + ds * 16 + hh * 8, key_ok));
      const half4_t v1 = to_half4(load4_or_zero(vp + ds * 16 + hh * 8 + 4, key_ok));
      kf[ds] = half8_t{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
      vf[ds] = half8_t{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
      for (int j = 0; j < 8; ++j) kt_lds[(ds * 16 + hh * 8 + j) * C::KTS + wave * 32 + c] = kf[ds][j];
    }
  }

  // Staging registers for one query block (prefetched one iteration ahead).
  float4 qreg[2 * C::PAIRS], doreg[2 * C::PAIRS];
  float lreg = 0.f, dreg = 0.f;
  auto load_stage = [&](int qb0) {
#pragma unroll
    for (int i = 0; i < C::PAIRS; ++i) {
      const int idx = tid + i * C::THREADS;
      const int row = qb0 + 2 * (idx >> 4), c4 = idx & 15;
      const bool ok0 = row < S, ok1 = row + 1 < S;
      const size_t o0 = ok0 ? (size_t)row * ld + hoff + c4 * 4 : 0;
      const size_t o1 = ok1 ? (size_t)(row + 1) * ld + hoff + c4 * 4 : 0;
      qreg[2 * i] = load4_or_zero(Q + o0, ok0);
      qreg[2 * i + 1] = load4_or_zero(Q + o1, ok1);
      doreg[2 * i] = load4_or_zero(dO + o0, ok0);
      doreg[2 * i + 1] = load4_or_zero(dO + o1, ok1);
    }
    if (tid < C::BM) {
      const int row = qb0 + tid;
      const bool ok = row < S;
      lreg = ok ? LSE[(size_t)head * S + row] * kLog2e : INFINITY;
      dreg = ok ? delta[(size_t)head * S + row] : 0.f;
    }
  };
  auto store_stage = [&]() {
#pragma unroll
    for (int i = 0; i < C::PAIRS; ++i) {
      const int idx = tid + i * C::THREADS;
      const int rp = idx >> 4, c4 = idx & 15;
      qreg[2 * i] = scale4(qreg[2 * i], c2);
      qreg[2 * i + 1] = scale4(qreg[2 * i + 1], c2);
      const float4 d0 = scale4(doreg[2 * i], sigma), d1 = scale4(doreg[2 * i + 1], sigma);
      *reinterpret_cast<half4_t *>(q_lds + (2 * rp) * C::QS + c4 * 4) = to_half4(qreg[2 * i]);
      *reinterpret_cast<half4_t *>(q_lds + (2 * rp + 1) * C::QS + c4 * 4) = to_half4(qreg[2 * i + 1]);
      *reinterpret_cast<half4_t *>(do_lds + (2 * rp) * C::QS + c4 * 4) = to_half4(d0);
      *reinterpret_cast<half4_t *>(do_lds + (2 * rp + 1) * C::QS + c4 * 4) = to_half4(d1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        half2_t pq, pd;
        pq[0] = (half_t)f4at(qreg[2 * i], e);
        pq[1] = (half_t)f4at(qreg[2 * i + 1], e);
        pd[0] = (half_t)f4at(d0, e);
        pd[1] = (half_t)f4at(d1, e);
        *reinterpret_cast<half2_t *>(qt_lds + (c4 * 4 + e) * C::TS + 2 * rp) = pq;
        *reinterpret_cast<half2_t *>(dot_lds + (c4 * 4 + e) * C::TS + 2 * rp) = pd;
      }
    }
    if (tid < C::BM) {
      lse2_lds[tid] = lreg;
      delta_lds[tid] = dreg * sigma;
    }
  };

  f32x16 dk[2], dv[2];
  dk[0] = dk[1] = dv[0] = dv[1] = f32x16{};

  const int n_qblocks = (S + C::BM - 1) / C::BM;
  const int first_qb = causal ? kv_blk0 / C::BM : 0;
  if (first_qb < n_qblocks) load_stage(first_qb * C::BM);

  for (int qbi = first_qb; qbi < n_qblocks; ++qbi) {
    const int qb0 = qbi * C::BM;
    __syncthreads();  // previous block's LDS reads are done
    store_stage();
    __syncthreads();  // staged block visible
    if (qbi + 1 < n_qblocks) load_stage(qb0 + C::BM);

    // S and dP for the two 32-row halves of the block (rows = queries, lane = key).
    f32x16 sacc[2], pacc[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      sacc[qb] = f32x16{};
      pacc[qb] = f32x16{};
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) {
        const half8_t aq =
            *reinterpret_cast<const half8_t *>(q_lds + (qb * 32 + c) * C::QS + ds * 16 + hh * 8);
        const half8_t ad =
            *reinterpret_cast<const half8_t *>(do_lds + (qb * 32 + c) * C::QS + ds * 16 + hh * 8);
        sacc[qb] = mfma32x32x16(aq, kf[ds], sacc[qb]);
        pacc[qb] = mfma32x32x16(ad, vf[ds], pacc[qb]);
      }
    }

    // P and dS; register r of half qb is query qb0 + 32*qb + 8*(r/4) + 4*hh + r%4.
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int ql = qb * 32 + g * 8 + hh * 4;
        const float4 L = *reinterpret_cast<const float4 *>(lse2_lds + ql);
        const float4 Dl = *reinterpret_cast<const float4 *>(delta_lds + ql);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          float p = fast_exp2(sacc[qb][r] - f4at(L, e));
          if (causal && key > qb0 + ql + e) p = 0.f;
          sacc[qb][r] = p;
          pacc[qb][r] = p * (pacc[qb][r] - f4at(Dl, e));
        }
      }

    // P^T and dS^T as A operands (M = keys): query step qs covers queries
    // 16*qs + (8*(j/4) + 4*hh + j%4) in slot j.
    half8_t pf[4], dsf[4];
#pragma unroll
    for (int qs = 0; qs < 4; ++qs) {
      const int base = (qs & 1) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pf[qs][j] = (half_t)sacc[qs >> 1][base + j];
        dsf[qs][j] = (half_t)pacc[qs >> 1][base + j];
      }
    }

#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int qs = 0; qs < 4; ++qs) {
        const int off = (db * 32 + c) * C::TS + qs * 16 + hh * 4;
        const half4_t d0 = *reinterpret_cast<const half4_t *>(dot_lds + off);
        const half4_t d1 = *reinterpret_cast<const half4_t *>(dot_lds + off + 8);
        const half4_t q0 = *reinterpret_cast<const half4_t *>(qt_lds + off);
        const half4_t q1 = *reinterpret_cast<const half4_t *>(qt_lds + off + 8);
        const half8_t bdo = half8_t{d0[0], d0[1], d0[2], d0[3], d1[0], d1[1], d1[2], d1[3]};
        const half8_t bq = half8_t{q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
        dv[db] = mfma32x32x16(pf[qs], bdo, dv[db]);
        dk[db] = mfma32x32x16(dsf[qs], bq, dk[db]);
      }

    // dS -> LDS, query-major, for dQ = dS K.
#pragma unroll
    for (int qs = 0; qs < 4; ++qs)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int ql = qs * 16 + (j >> 2) * 8 + hh * 4 + (j & 3);
        ds_lds[ql * C::DSS + wave * 32 + c] = dsf[qs][j];
      }
    __syncthreads();

    // dQ block (64 x 64) = dS (64 x BN) . K (BN x 64), split in 32x32 tiles.
#pragma unroll
    for (int tt = 0; tt < C::DQ_TILES; ++tt) {
      const int tile = wave * C::DQ_TILES + tt;
      const int qt = tile >> 1, dt = tile & 1;
      f32x16 acc = f32x16{};
#pragma unroll
      for (int ks = 0; ks < C::BN / 16; ++ks) {
        const half8_t a =
            *reinterpret_cast<const half8_t *>(ds_lds + (qt * 32 + c) * C::DSS + ks * 16 + hh * 8);
        const half8_t b =
            *reinterpret_cast<const half8_t *>(kt_lds + (dt * 32 + c) * C::KTS + ks * 16 + hh * 8);
        acc = mfma32x32x16(a, b, acc);
      }
      const float dq_scale = scale * inv_sigma;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int query = qb0 + qt * 32 + (r >> 2) * 8 + hh * 4 + (r & 3);
        if (query < S)
          unsafeAtomicAdd(dQ + (size_t)query * ld + hoff + dt * 32 + c, acc[r] * dq_scale);
      }
    }
  }

  // dK = scale * dS^T Q = ln2 * dS^T (c2 Q) / sigma, dV = P^T dO / sigma; row
  // r is key kv_blk0 + 32*wave + 8*(r/4) + 4*hh + r%4, column d = 32*db + c.
  const float dk_scale = kLn2 * inv_sigma;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int kr = kv_blk0 + wave * 32 + (r >> 2) * 8 + hh * 4 + (r & 3);
    if (kr < S) {
      float *dkrow = dK + (size_t)kr * ld + hoff;
      float *dvrow = dV + (size_t)kr * ld + hoff;
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        dkrow[db * 32 + c] = dk[db][r] * dk_scale;
        dvrow[db * 32 + c] = dv[db][r] * inv_sigma;
      }
    }
  }
}

}  // namespace

size_t bwd_workspace_bytes_d64(int n_heads, int seq_len) {
  const size_t floats = ws_delta_floats(n_heads, seq_len) + (size_t)n_heads * pre_blocks(seq_len);
  return (floats * sizeof(float) + 255) / 256 * 256;
}

hipError_t launch_bwd_pre_d64(const float *o, const float *d_o, float *d_q, void *workspace,
                              int n_heads, int seq_len, hipStream_t stream) {
  float *delta = static_cast<float *>(workspace);
  float *blockmax = delta + ws_delta_floats(n_heads, seq_len);
  hipLaunchKernelGGL(bwd_preprocess_kernel, dim3(pre_blocks(seq_len), n_heads), dim3(256), 0, stream,
                     o, d_o, d_q, delta, blockmax, n_heads, seq_len);
  return hipGetLastError();
}

hipError_t launch_bwd_main_d64(const float *q, const float *k, const float *v, const float *d_o,
                               const float *lse, float *d_q, float *d_k, float *d_v,
                               const void *workspace, int n_heads, int seq_len, float scale,
                               bool causal, hipStream_t stream) {
  constexpr int WAVES = 4;
  using C = BwdCfg<WAVES>;
  const float *delta = static_cast<const float *>(workspace);
  const float *blockmax = delta + ws_delta_floats(n_heads, seq_len);
  const int n_kvtiles = (seq_len + C::BN - 1) / C::BN;
  hipLaunchKernelGGL((bwd_main_kernel<WAVES>), dim3(n_kvtiles * n_heads), dim3(C::THREADS), 0,
                     stream, q, k, v, d_o, lse, delta, blockmax, d_q, d_k, d_v, n_heads, seq_len,
                     scale, causal ? 1 : 0, pre_blocks(seq_len));
  return hipGetLastError();
}

hipError_t launch_bwd_d64(const float *q, const float *k, const float *v, const float *o,
                          const float *d_o, const float *lse, float *d_q, float *d_k,
                          float *d_v, void *workspace, int n_heads, int seq_len, float scale,
                          bool causal, hipStream_t stream) {
  hipError_t err = launch_bwd_pre_d64(o, d_o, d_q, workspace, n_heads, seq_len, stream);
  if (err != hipSuccess) return err;
  return launch_bwd_main_d64(q, k, v, d_o, lse, d_q, d_k, d_v, workspace, n_heads, seq_len, scale,
                             causal, stream);
}

}  // namespace dfattn
