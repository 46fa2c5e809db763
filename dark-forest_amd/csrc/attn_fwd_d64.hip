// attn_fwd_d64.hip — fused causal attention forward for d_head = 64 on gfx950.
//
// Replaces kernel_fused_mha_fwd_tiled (darkforest-cuda/kernels/attention_fused.cu:41-159),
// which walks keys one at a time per query row with a warp-shuffle dot
// product. Here a workgroup owns BM query rows of one head and streams the
// keys in tiles of BN = 64 through LDS; both products run on MFMA:
//
//   S^T (keys x queries) = K (keys x d) . Q^T (d x queries)     [32x32x16 f16]
//   O^T (d x queries)   += V^T (d x keys) . P^T (keys x queries)
//
// Computing the transposed products puts one query row in one lane (the MFMA
// result's column), so the online-softmax row max and row sum are per-lane
// register reductions plus one exchange between the two lane halves, and the
// probabilities come out of the first MFMA already in the B-operand layout of
// the second. Q is loaded once into registers, pre-multiplied by
// scale * log2(e) so the softmax runs on exp2. Operands are fp16 (the fp32
// inputs are rounded on load), accumulation and softmax are fp32.
//
// Output: O [S, H*64] fp32 and, when lse != nullptr, lse [H, S] (natural log)
// — the row statistic the backward recomputes P from.
#include "dfattn_internal.h"

namespace dfattn {
namespace {

template <int NQ, int WAVES>
struct FwdCfg {
  static constexpr int D = 64;
  static constexpr int BN = 64;             // keys per LDS tile
  static constexpr int QPW = 32 * NQ;       // query rows per wave
  static constexpr int BM = QPW * WAVES;    // query rows per workgroup
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int KS = D + 8;          // K tile row stride (halves)
  static constexpr int VS = BN + 8;         // V^T tile row stride (halves)
  static constexpr int STAGE = BN * KS + D * VS;  // halves per pipeline stage
  static constexpr int K_F4 = BN * D / 4 / THREADS;         // float4 of K per thread
  static constexpr int V_PAIRS = (BN / 2) * (D / 4) / THREADS;  // (2 rows x float4) of V
  static_assert(K_F4 * THREADS * 4 == BN * D, "K tile split");
  static_assert(V_PAIRS * THREADS * 8 == BN * D, "V tile split");
};

__device__ __forceinline__ float f4at(const float4 &v, int e) {
  return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

template <int NQ, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void fwd_d64_kernel(
    const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
    float *__restrict__ O, float *__restrict__ LSE, int H, int S, float qscale, int causal,
    int n_qtiles) {
  using C = FwdCfg<NQ, WAVES>;
  __shared__ __attribute__((aligned(16))) half_t lds[2 * C::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, hh = lane >> 5;
  const int head = blockIdx.x % H;
  // Longest query tiles first under causal masking (they see the most keys).
  const int qtile = causal ? (n_qtiles - 1 - (int)(blockIdx.x / H)) : (int)(blockIdx.x / H);
  const size_t ld = (size_t)H * C::D;
  const size_t hoff = (size_t)head * C::D;

  const int q_blk0 = qtile * C::BM;
  const int q_w0 = q_blk0 + wave * C::QPW;
  const bool wave_active = q_w0 < S;
  const int wave_qlast = min(q_w0 + C::QPW, S) - 1;
  const int kv_end = causal ? min(S, q_blk0 + C::BM) : S;
  const int n_tiles = (kv_end + C::BN - 1) / C::BN;

  // Q^T fragments (B operand): lane c holds query q_w0 + 32*nq + c, slots
  // d = 16*ds + 8*hh + j.
  half8_t qf[NQ][4];
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    const int query = q_w0 + nq * 32 + c;
    const bool ok = query < S;
    const float *p = Q + (ok ? (size_t)query * ld + hoff : 0);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      const float4 a = scale4(load4_or_zero(p + ds * 16 + hh * 8, ok), qscale);
      const float4 b = scale4(load4_or_zero(p + ds * 16 + hh * 8 + 4, ok), qscale);
      const half4_t lo = to_half4(a), hi = to_half4(b);
      qf[nq][ds] = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }

  float4 kreg[C::K_F4];
  float4 vreg[2 * C::V_PAIRS];
  auto load_tile = [&](int t) {
    const int kv0 = t * C::BN;
#pragma unroll
    for (int i = 0; i < C::K_F4; ++i) {
      const int idx = tid + i * C::THREADS;
      const int key = kv0 + (idx >> 4), c4 = idx & 15;
      const bool ok = key < S;
      kreg[i] = load4_or_zero(K + (ok ? (size_t)key * ld + hoff + c4 * 4 : 0), ok);
    }
#pragma unroll
    for (int i = 0; i < C::V_PAIRS; ++i) {
      const int idx = tid + i * C::THREADS;
      const int key = kv0 + 2 * (idx >> 4), c4 = idx & 15;
      const bool ok0 = key < S, ok1 = key + 1 < S;
      vreg[2 * i] = load4_or_zero(V + (ok0 ? (size_t)key * ld + hoff + c4 * 4 : 0), ok0);
      vreg[2 * i + 1] = load4_or_zero(V + (ok1 ? (size_t)(key + 1) * ld + hoff + c4 * 4 : 0), ok1);
    }
  };
  auto store_tile = [&](int stage) {
    half_t *kl = lds + stage * C::STAGE;
    half_t *vl = kl + C::BN * C::KS;
#pragma unroll
    for (int i = 0; i < C::K_F4; ++i) {
      const int idx = tid + i * C::THREADS;
      const int row = idx >> 4, c4 = idx & 15;
      *reinterpret_cast<half4_t *>(kl + row * C::KS + c4 * 4) = to_half4(kreg[i]);
    }
#pragma unroll
    for (int i = 0; i < C::V_PAIRS; ++i) {
      const int idx = tid + i * C::THREADS;
      const int rp = idx >> 4, c4 = idx & 15;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        half2_t pr;
        pr[0] = (half_t)f4at(vreg[2 * i], e);
        pr[1] = (half_t)f4at(vreg[2 * i + 1], e);
        *reinterpret_cast<half2_t *>(vl + (c4 * 4 + e) * C::VS + 2 * rp) = pr;
      }
    }
  };

  f32x16 o[2][NQ];
  float m[NQ], l[NQ];
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    m[nq] = -INFINITY;
    l[nq] = 0.f;
#pragma unroll
    for (int db = 0; db < 2; ++db) o[db][nq] = f32x16{};
  }

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int stage = t & 1;
    if (t + 1 < n_tiles) load_tile(t + 1);
    const int kv0 = t * C::BN;
    if (wave_active && (!causal || kv0 <= wave_qlast)) {
      const half_t *kl = lds + stage * C::STAGE;
      const half_t *vl = kl + C::BN * C::KS;

      // S^T tile: rows = keys kv0 + 32*kb + (8*(r/4) + 4*hh + r%4), column = query.
      f32x16 s[2][NQ];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int nq = 0; nq < NQ; ++nq) s[kb][nq] = f32x16{};
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) {
          const half8_t a =
              *reinterpret_cast<const half8_t *>(kl + (kb * 32 + c) * C::KS + ds * 16 + hh * 8);
#pragma unroll
          for (int nq = 0; nq < NQ; ++nq) s[kb][nq] = mfma32x32x16(a, qf[nq][ds], s[kb][nq]);
        }
      }

      const bool need_mask = (kv0 + C::BN > S) || (causal && kv0 + C::BN - 1 > q_w0);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int nq = 0; nq < NQ; ++nq) {
            const int query = q_w0 + nq * 32 + c;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = kv0 + kb * 32 + (r >> 2) * 8 + hh * 4 + (r & 3);
              if (key >= S || (causal && key > query)) s[kb][nq][r] = -INFINITY;
            }
          }
      }

      // Online softmax in the log2 domain; one row per lane.
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][nq][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m[nq], mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = fast_exp2(m[nq] - m_use);
        m[nq] = m_new;
        l[nq] *= alpha;
#pragma unroll
        for (int db = 0; db < 2; ++db) o[db][nq] *= alpha;
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float p = fast_exp2(s[kb][nq][r] - m_use);
            s[kb][nq][r] = p;
            ls += p;
          }
        l[nq] += ls;
      }

      // P^T as the B operand of the PV product: key step ks covers keys
      // 16*ks + (8*(j/4) + 4*hh + j%4) in slot j.
      half8_t pf[NQ][4];
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int base = (ks & 1) * 8;
#pragma unroll
          for (int j = 0; j < 8; ++j) pf[nq][ks][j] = (half_t)s[ks >> 1][nq][base + j];
        }

#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const half_t *vrow = vl + (db * 32 + c) * C::VS + ks * 16 + hh * 4;
          const half4_t lo = *reinterpret_cast<const half4_t *>(vrow);
          const half4_t hi = *reinterpret_cast<const half4_t *>(vrow + 8);
          const half8_t a = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
          for (int nq = 0; nq < NQ; ++nq) o[db][nq] = mfma32x32x16(a, pf[nq][ks], o[db][nq]);
        }
    }
    if (t + 1 < n_tiles) store_tile(stage ^ 1);
    __syncthreads();
  }

  if (!wave_active) return;
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    const float lt = l[nq] + __shfl_xor(l[nq], 32, 64);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int query = q_w0 + nq * 32 + c;
    if (query < S) {
      float *orow = O + (size_t)query * ld + hoff;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 val = make_float4(o[db][nq][4 * g] * inv, o[db][nq][4 * g + 1] * inv,
                                         o[db][nq][4 * g + 2] * inv, o[db][nq][4 * g + 3] * inv);
          *reinterpret_cast<float4 *>(orow + db * 32 + g * 8 + hh * 4) = val;
        }
      if (LSE != nullptr && hh == 0)
        LSE[(size_t)head * S + query] = lt > 0.f ? (m[nq] + log2f(lt)) * kLn2 : -INFINITY;
    }
  }
}

}  // namespace

hipError_t launch_fwd_d64(const float *q, const float *k, const float *v, float *o, float *lse,
                          int n_heads, int seq_len, float scale, bool causal,
                          hipStream_t stream) {
  constexpr int NQ = 1, WAVES = 4;
  using C = FwdCfg<NQ, WAVES>;
  const int n_qtiles = (seq_len + C::BM - 1) / C::BM;
  const dim3 grid((unsigned)(n_qtiles * n_heads));
  hipLaunchKernelGGL((fwd_d64_kernel<NQ, WAVES>), grid, dim3(C::THREADS), 0, stream, q, k, v, o,
                     lse, n_heads, seq_len, scale * kLog2e, causal ? 1 : 0, n_qtiles);
  return hipGetLastError();
}

}  // namespace dfattn
