/*
 * attention_oracle.c — CPU restatement of Dark Forest's fp32 attention.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP
 * attention library and the CPU baseline that bench.py times beside it. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it; the product path (libdfattn.so and the dfattn package) never does.
 *
 * What it restates (the reference cannot be built here: it needs rustc and
 * nvcc, neither present):
 *   oracle_mha_forward_f32      darkforest-core/src/engine/static_gpt2.rs:2766-2798
 *                               (multi-head CPU forward, [S, H*D] layout,
 *                               index i*dm + h*dh + d), with the causal flag of
 *                               darkforest-cuda/src/lib.rs:2503 added.
 *   oracle_reference_attention_f32
 *                               darkforest-cuda/src/lib.rs:2493-2527
 *                               (single-head `reference_attention`).
 *   oracle_reference_backward_f32
 *                               darkforest-cuda/src/lib.rs:2529-2586
 *                               (`reference_backward`), applied per head with
 *                               row stride H*D exactly as the GPU kernel
 *                               indexes (attention_fused.cu:404-414).
 *   *_f64                       the same loops in double precision; used to
 *                               measure the fp32 restatement's own error.
 *   oracle_mha_forward_rows_f32 the forward for a chosen set of query rows
 *                               (row-sampled check of S=131072).
 *   oracle_decode_f32           attention_fused.cu:551-615, 800-866, 968-1033
 *                               (single-query KV-cache decode: contiguous,
 *                               paged, bf16 pools), plus its logsumexp.
 *   oracle_pos_embed_interpolate_f32
 *                               attention_fused.cu:1098-1121 (position
 *                               interpolation of a trained embedding table).
 *   oracle_apply_rope_f32/_f64  attention_fused.cu:1139-1162 (rotary
 *                               embedding of one row, in place).
 *   oracle_paged_copy_row, oracle_f32_to_bf16
 *                               attention_fused.cu:1178-1217 (a row written
 *                               into a paged fp32 or bf16 pool).
 *
 * Arithmetic follows the reference: fp32 throughout, sums accumulated
 * sequentially in index order, exp from libm (Rust's f32::exp), mul and add
 * never contracted into an FMA (build with -ffp-contract=off, no fast-math).
 *
 * New behaviour (not in the reference): the natural-log logsumexp of each
 * query row, lse = max + ln(sum exp(score - max)), written when `lse` is not
 * NULL. Layout [H, S].
 *
 * Pinning (what checks this restatement, see tests/test_oracle.py):
 *   - the reference's two known-answer tests (lib.rs:2605-2628, 2752-2829),
 *     inputs regenerated from their closed forms, against expected values
 *     computed by PyTorch float64 scaled_dot_product_attention + autograd
 *     (tests/golden/), at the reference's 2e-4 and at 1e-5;
 *   - central finite differences of the forward (lib.rs:2786-2828);
 *   - closed forms: O_0 = V_0, lse_0 = scale q_0.k_0, dQ_0 = 0; q = 0 gives
 *     running means of V and lse_i = ln(i+1); sum_j dK_j = 0; sum_j dV_j =
 *     sum_i dO_i; constant V gives constant O;
 *   - an independent vectorised float64 numpy implementation on seeded inputs;
 *   - planted mistakes (oracle_set_mutation) that each of those checks must
 *     catch;
 *   - for the elementwise kernels: a linear table (interpolation is exact on
 *     it up to rounding) and the trained-range copy; RoPE as the complex
 *     product z * exp(i pos theta) in float64, pos 0 = identity, preserved
 *     pair norms; the bf16 rounding against torch's own float -> bfloat16
 *     conversion, including ties, overflow, subnormals, infinities and NaN;
 *     a row written by oracle_paged_copy_row is the row oracle_decode reads.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- planted mistakes, for the tests that show the checks have teeth ---- */
enum {
  MUT_NONE = 0,
  MUT_CAUSAL_OFF_BY_ONE = 1, /* keys j < i instead of j <= i                */
  MUT_DROP_SCALE = 2,        /* scores not multiplied by scale              */
  MUT_K_FROM_V = 3,          /* scores use V where K belongs                */
  MUT_DROP_CORRECTION = 4,   /* dS = P*dP, the -sum(P*dP) term dropped      */
  MUT_DK_SIGN = 5,           /* dK accumulated with the wrong sign          */
  MUT_HEAD_INDEX = 6,        /* K read from head H-1-h                      */
  MUT_LSE_LOG2 = 7,          /* lse in log base 2                           */
  MUT_DV_FROM_DS = 8,        /* dV accumulates dS instead of P              */
  MUT_TRANSPOSE_DQ = 9,      /* dQ uses q where k belongs                   */
  MUT_ROPE_SIN_SIGN = 10,    /* RoPE rotates by -angle                      */
  MUT_ROPE_FREQ = 11,        /* RoPE theta = base^(-i / d_head)             */
  MUT_INTERP_SAME_ROW = 12,  /* interpolation between row p0 and itself     */
  MUT_BF16_TRUNCATE = 13,    /* bf16 by truncation instead of rounding      */
  MUT_PAGE_OFFSET = 14       /* paged row written at offset page_offset - 1 */
};
static int g_mutation = MUT_NONE;

void oracle_set_mutation(int m) { g_mutation = m; }
int oracle_get_mutation(void) { return g_mutation; }

static inline size_t max_key_of(size_t row, size_t seq_len, int causal) {
  if (!causal) return seq_len;
  if (g_mutation == MUT_CAUSAL_OFF_BY_ONE) return row; /* planted */
  return row + 1;
}

static inline int k_head(int h, int n_heads) {
  return g_mutation == MUT_HEAD_INDEX ? n_heads - 1 - h : h;
}

static int clamp_threads(int threads) {
  if (threads < 1) threads = 1;
  return threads;
}

/* ------------------------------------------------------------------------
 * Multi-head forward, static_gpt2.rs:2766-2798.
 * For each head and query row: scores[j] = (sum_d q*k) * scale for j <= i;
 * max; exp_scores[j] = exp(score - max); exp_sum sequential; inv_sum =
 * 1/exp_sum (0 if the sum is 0); out[i][d] = sum_j (exp_scores[j]*inv_sum)
 * * v[j][d], sequential in j. Rows are independent, so the (h, i) loop is
 * split over threads without changing any result bit.
 * ---------------------------------------------------------------------- */
#define DEFINE_MHA_FORWARD(NAME, T, EXP, LOG)                                    \
  void NAME(const T *q, const T *k, const T *v, T *out, T *lse, int n_heads,     \
            int seq_len, int d_head, T scale, int causal, int threads) {         \
    const size_t S = (size_t)seq_len, dh = (size_t)d_head;                       \
    const size_t dm = (size_t)n_heads * dh;                                      \
    const T *kk = (g_mutation == MUT_K_FROM_V) ? v : k;                          \
    const T sc = (g_mutation == MUT_DROP_SCALE) ? (T)1 : scale;                  \
    long long total = (long long)n_heads * (long long)seq_len;                   \
    (void)threads;                                                               \
    _Pragma("omp parallel num_threads(clamp_threads(threads))")                  \
    {                                                                            \
      T *scores = (T *)malloc((S ? S : 1) * sizeof(T));                          \
      T *exp_scores = (T *)malloc((S ? S : 1) * sizeof(T));                      \
      _Pragma("omp for schedule(dynamic, 16)")                                   \
      for (long long task = 0; task < total; ++task) {                           \
        const int h = (int)(task / seq_len);                                     \
        const size_t i = (size_t)(task % seq_len);                               \
        const int hk = k_head(h, n_heads);                                       \
        const size_t mk = max_key_of(i, S, causal);                              \
        for (size_t j = 0; j < mk; ++j) {                                        \
          T dot = 0;                                                             \
          for (size_t d = 0; d < dh; ++d) {                                      \
            T q_val = q[i * dm + (size_t)h * dh + d];                            \
            T k_val = kk[j * dm + (size_t)hk * dh + d];                          \
            dot += q_val * k_val;                                                \
          }                                                                      \
          scores[j] = dot * sc;                                                  \
        }                                                                        \
        T max_score = -INFINITY;                                                 \
        for (size_t j = 0; j < mk; ++j)                                          \
          max_score = (scores[j] > max_score) ? scores[j] : max_score;           \
        T exp_sum = 0;                                                           \
        for (size_t j = 0; j < mk; ++j) {                                        \
          exp_scores[j] = EXP(scores[j] - max_score);                            \
          exp_sum += exp_scores[j];                                              \
        }                                                                        \
        T inv_sum = exp_sum > 0 ? (T)1 / exp_sum : (T)0;                         \
        for (size_t d = 0; d < dh; ++d) {                                        \
          T val = 0;                                                             \
          for (size_t j = 0; j < mk; ++j) {                                      \
            T weight = exp_scores[j] * inv_sum;                                  \
            val += weight * v[j * dm + (size_t)h * dh + d];                      \
          }                                                                      \
          out[i * dm + (size_t)h * dh + d] = val;                                \
        }                                                                        \
        if (lse) {                                                               \
          T l = mk ? max_score + LOG(exp_sum) : -INFINITY;                       \
          if (g_mutation == MUT_LSE_LOG2) l = l / LOG((T)2);                     \
          lse[(size_t)h * S + i] = l;                                            \
        }                                                                        \
      }                                                                          \
      free(scores);                                                              \
      free(exp_scores);                                                          \
    }                                                                            \
  }

DEFINE_MHA_FORWARD(oracle_mha_forward_f32, float, expf, logf)
DEFINE_MHA_FORWARD(oracle_mha_forward_f64, double, exp, log)

/* ------------------------------------------------------------------------
 * Row-sampled multi-head forward: the rows listed in `rows` (n_rows of them),
 * every head. out_rows is [n_rows, H*D], lse_rows [n_rows, H]. Same
 * arithmetic as oracle_mha_forward_f32 for those rows.
 * ---------------------------------------------------------------------- */
void oracle_mha_forward_rows_f32(const float *q, const float *k, const float *v,
                                 const int64_t *rows, int n_rows,
                                 float *out_rows, float *lse_rows, int n_heads,
                                 int seq_len, int d_head, float scale,
                                 int causal, int threads) {
  const size_t S = (size_t)seq_len, dh = (size_t)d_head;
  const size_t dm = (size_t)n_heads * dh;
  long long total = (long long)n_rows * n_heads;
  (void)threads;
#pragma omp parallel num_threads(clamp_threads(threads))
  {
    float *scores = (float *)malloc((S ? S : 1) * sizeof(float));
    float *exp_scores = (float *)malloc((S ? S : 1) * sizeof(float));
#pragma omp for schedule(dynamic, 1)
    for (long long task = 0; task < total; ++task) {
      const int r = (int)(task / n_heads);
      const int h = (int)(task % n_heads);
      const size_t i = (size_t)rows[r];
      const size_t mk = max_key_of(i, S, causal);
      for (size_t j = 0; j < mk; ++j) {
        float dot = 0.0f;
        for (size_t d = 0; d < dh; ++d)
          dot += q[i * dm + (size_t)h * dh + d] * k[j * dm + (size_t)h * dh + d];
        scores[j] = dot * scale;
      }
      float max_score = -INFINITY;
      for (size_t j = 0; j < mk; ++j)
        max_score = (scores[j] > max_score) ? scores[j] : max_score;
      float exp_sum = 0.0f;
      for (size_t j = 0; j < mk; ++j) {
        exp_scores[j] = expf(scores[j] - max_score);
        exp_sum += exp_scores[j];
      }
      float inv_sum = exp_sum > 0.0f ? 1.0f / exp_sum : 0.0f;
      for (size_t d = 0; d < dh; ++d) {
        float val = 0.0f;
        for (size_t j = 0; j < mk; ++j)
          val += (exp_scores[j] * inv_sum) * v[j * dm + (size_t)h * dh + d];
        out_rows[(size_t)r * dm + (size_t)h * dh + d] = val;
      }
      if (lse_rows)
        lse_rows[(size_t)r * n_heads + h] =
            mk ? max_score + logf(exp_sum) : -INFINITY;
    }
    free(scores);
    free(exp_scores);
  }
}

/* ------------------------------------------------------------------------
 * Single-head forward, lib.rs:2493-2527 (`reference_attention`):
 * weight = exp(score - max) / normalizer, out[row][d] += weight * v[key][d]
 * with the key loop outside the d loop.
 * ---------------------------------------------------------------------- */
void oracle_reference_attention_f32(const float *q, const float *k,
                                    const float *v, float *out, int seq_len,
                                    int d_head, float scale, int causal) {
  const size_t S = (size_t)seq_len, dh = (size_t)d_head;
  const float *kk = (g_mutation == MUT_K_FROM_V) ? v : k;
  const float sc = (g_mutation == MUT_DROP_SCALE) ? 1.0f : scale;
  float *scores = (float *)malloc((S ? S : 1) * sizeof(float));
  float *weights = (float *)malloc((S ? S : 1) * sizeof(float));
  memset(out, 0, S * dh * sizeof(float));
  for (size_t row = 0; row < S; ++row) {
    const size_t mk = max_key_of(row, S, causal);
    for (size_t key = 0; key < mk; ++key) {
      float dot = 0.0f;
      for (size_t d = 0; d < dh; ++d) dot += q[row * dh + d] * kk[key * dh + d];
      scores[key] = dot * sc;
    }
    float max_score = -INFINITY;
    for (size_t key = 0; key < mk; ++key)
      max_score = (scores[key] > max_score) ? scores[key] : max_score;
    float normalizer = 0.0f;
    for (size_t key = 0; key < mk; ++key) {
      weights[key] = expf(scores[key] - max_score);
      normalizer += weights[key];
    }
    for (size_t key = 0; key < mk; ++key) {
      float weight = weights[key] / normalizer;
      for (size_t d = 0; d < dh; ++d) out[row * dh + d] += weight * v[key * dh + d];
    }
  }
  free(scores);
  free(weights);
}

/* ------------------------------------------------------------------------
 * Backward, lib.rs:2529-2586 (`reference_backward`), per head with row
 * stride H*D. For each row: scores; max; normalizer = sum exp(score-max);
 * P = exp(score-max)/normalizer; dP[key] = sum_d dO*v; correction =
 * sum_key P*dP; dS = P*(dP - correction); then for each key and d:
 *   dq[row][d] += scale*dS*k[key][d]
 *   dk[key][d] += scale*dS*q[row][d]
 *   dv[key][d] += P*dO[row][d]
 * dK and dV accumulate across rows in row order, so heads (not rows) are
 * split over threads; results do not depend on the thread count.
 * ---------------------------------------------------------------------- */
#define DEFINE_BACKWARD(NAME, T, EXP)                                            \
  void NAME(const T *q, const T *k, const T *v, const T *d_out, T *d_q, T *d_k,  \
            T *d_v, int n_heads, int seq_len, int d_head, T scale, int causal,   \
            int threads) {                                                       \
    const size_t S = (size_t)seq_len, dh = (size_t)d_head;                       \
    const size_t dm = (size_t)n_heads * dh;                                      \
    const T *kk = (g_mutation == MUT_K_FROM_V) ? v : k;                          \
    const T sc = (g_mutation == MUT_DROP_SCALE) ? (T)1 : scale;                  \
    (void)threads;                                                               \
    for (size_t row = 0; row < S; ++row)                                         \
      for (size_t c = 0; c < dm; ++c) {                                          \
        d_q[row * dm + c] = 0;                                                   \
        d_k[row * dm + c] = 0;                                                   \
        d_v[row * dm + c] = 0;                                                   \
      }                                                                          \
    _Pragma("omp parallel num_threads(clamp_threads(threads))")                  \
    {                                                                            \
      T *prob = (T *)malloc((S ? S : 1) * sizeof(T));                            \
      T *dprob = (T *)malloc((S ? S : 1) * sizeof(T));                           \
      _Pragma("omp for schedule(dynamic, 1)")                                    \
      for (int h = 0; h < n_heads; ++h) {                                        \
        const size_t ho = (size_t)h * dh;                                        \
        const size_t hko = (size_t)k_head(h, n_heads) * dh;                      \
        for (size_t row = 0; row < S; ++row) {                                   \
          const size_t mk = max_key_of(row, S, causal);                          \
          for (size_t key = 0; key < mk; ++key) {                                \
            T dot = 0;                                                           \
            for (size_t d = 0; d < dh; ++d)                                      \
              dot += q[row * dm + ho + d] * kk[key * dm + hko + d];              \
            prob[key] = dot * sc;                                                \
          }                                                                      \
          T max_score = -INFINITY;                                               \
          for (size_t key = 0; key < mk; ++key)                                  \
            max_score = (prob[key] > max_score) ? prob[key] : max_score;         \
          T normalizer = 0;                                                      \
          for (size_t key = 0; key < mk; ++key)                                  \
            normalizer += EXP(prob[key] - max_score);                            \
          for (size_t key = 0; key < mk; ++key)                                  \
            prob[key] = EXP(prob[key] - max_score) / normalizer;                 \
          for (size_t key = 0; key < mk; ++key) {                                \
            T dp = 0;                                                            \
            for (size_t d = 0; d < dh; ++d)                                      \
              dp += d_out[row * dm + ho + d] * v[key * dm + ho + d];             \
            dprob[key] = dp;                                                     \
          }                                                                      \
          T correction = 0;                                                      \
          for (size_t key = 0; key < mk; ++key) correction += prob[key] * dprob[key]; \
          if (g_mutation == MUT_DROP_CORRECTION) correction = 0;                 \
          for (size_t key = 0; key < mk; ++key) {                                \
            T d_score = prob[key] * (dprob[key] - correction);                   \
            T dv_coef = (g_mutation == MUT_DV_FROM_DS) ? d_score : prob[key];    \
            T dk_sign = (g_mutation == MUT_DK_SIGN) ? (T)-1 : (T)1;              \
            for (size_t d = 0; d < dh; ++d) {                                    \
              T kv = (g_mutation == MUT_TRANSPOSE_DQ) ? q[key * dm + ho + d]     \
                                                      : kk[key * dm + hko + d];  \
              d_q[row * dm + ho + d] += sc * d_score * kv;                       \
              d_k[key * dm + ho + d] += dk_sign * (sc * d_score * q[row * dm + ho + d]); \
              d_v[key * dm + ho + d] += dv_coef * d_out[row * dm + ho + d];      \
            }                                                                    \
          }                                                                      \
        }                                                                        \
      }                                                                          \
      free(prob);                                                                \
      free(dprob);                                                               \
    }                                                                            \
  }

DEFINE_BACKWARD(oracle_reference_backward_f32, float, expf)
DEFINE_BACKWARD(oracle_backward_f64, double, exp)

/* ------------------------------------------------------------------------
 * Single-query decode against a KV cache, attention_fused.cu:551-615
 * (kernel_fused_mha_decode_kv), with the paged addressing of 800-866
 * (kernel_paged_mha_decode_kv: row t lives in physical block
 * block_table[t / page_size] at offset t % page_size; pool rows are [d_model])
 * and the bf16 pools of 968-1033 (each element widened to fp32 exactly).
 * Per head, over keys t = 0 .. cur_len-1 in order: score = (sum_d q*k) *
 * scale; m_new = max(m, score); alpha = exp(m - m_new) (0 while m is the
 * initial -FLT_MAX); p = exp(score - m_new); l = fma(l, alpha, p); o =
 * fma(p, v, o*alpha) (the reference's fused forms); out = o / l (0 if l is 0). Nothing is written when cur_len is 0, as
 * the reference's kernels return early. New: lse = m + ln(l) per head (the
 * natural-log logsumexp of the scores), when lse is not NULL.
 * q, out: [H*D]; k, v: [cur_len or pool rows, H*D] as float (kv_bf16 = 0) or
 * as bf16 bit patterns in uint16 (kv_bf16 = 1); block_table NULL means a
 * contiguous cache.
 * ---------------------------------------------------------------------- */
static inline float bf16_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

#define DEFINE_DECODE(NAME, T, EXP, LOG, FMA)                                    \
  void NAME(const T *q, const void *k, const void *v, const int32_t *block_table, \
            int page_size, int kv_bf16, T *out, T *lse, int n_heads, int cur_len, \
            int d_head, T scale) {                                               \
    if (cur_len <= 0) return;                                                    \
    const size_t dh = (size_t)d_head, dm = (size_t)n_heads * dh;                 \
    for (int h = 0; h < n_heads; ++h) {                                          \
      T m = (T)-3.40282346638528859812e+38, l = 0;                               \
      T *o = out + (size_t)h * dh;                                               \
      for (size_t d = 0; d < dh; ++d) o[d] = 0;                                  \
      for (int t = 0; t < cur_len; ++t) {                                        \
        size_t row = (size_t)t;                                                  \
        if (block_table)                                                         \
          row = (size_t)block_table[t / page_size] * (size_t)page_size +         \
                (size_t)(t % page_size);                                         \
        const size_t base = row * dm + (size_t)h * dh;                           \
        T dot = 0;                                                               \
        for (size_t d = 0; d < dh; ++d) {                                        \
          const T kval = kv_bf16 ? (T)bf16_to_f32(((const uint16_t *)k)[base + d]) \
                                 : (T)((const T *)k)[base + d];                  \
          dot += q[(size_t)h * dh + d] * kval;                                   \
        }                                                                        \
        const T score = dot * scale;                                             \
        const T m_new = score > m ? score : m;                                   \
        const T alpha = (m == (T)-3.40282346638528859812e+38) ? (T)0 : EXP(m - m_new); \
        const T p = EXP(score - m_new);                                          \
        l = FMA(l, alpha, p);                                                    \
        m = m_new;                                                               \
        for (size_t d = 0; d < dh; ++d) {                                        \
          const T vval = kv_bf16 ? (T)bf16_to_f32(((const uint16_t *)v)[base + d]) \
                                 : (T)((const T *)v)[base + d];                  \
          o[d] = FMA(p, vval, o[d] * alpha);                                     \
        }                                                                        \
      }                                                                          \
      const T inv_l = l > 0 ? (T)1 / l : (T)0;                                   \
      for (size_t d = 0; d < dh; ++d) o[d] *= inv_l;                             \
      if (lse) lse[h] = l > 0 ? m + LOG(l) : (T)-INFINITY;                       \
    }                                                                            \
  }

DEFINE_DECODE(oracle_decode_f32, float, expf, logf, fmaf)
DEFINE_DECODE(oracle_decode_f64, double, exp, log, fma)

/* ------------------------------------------------------------------------
 * The elementwise kernels beside the decode family, one row each, in the
 * reference's fp32 arithmetic.
 * ---------------------------------------------------------------------- */

/* attention_fused.cu:1098-1121: copy inside the trained range, else linear
 * interpolation at pos * (trained - 1) / (max_ctx - 1) between rows p0 =
 * trunc and p1 = min(p0 + 1, trained - 1). New: where p0 would lie past the
 * table (the reference reads out of bounds there) the last row is returned.
 * trained >= 1. */
void oracle_pos_embed_interpolate_f32(const float *table, float *out, uint32_t pos,
                                      uint32_t trained, uint32_t max_ctx,
                                      uint32_t d_model) {
  for (uint32_t d = 0; d < d_model; ++d) {
    if (pos < trained && max_ctx <= trained) {
      out[d] = table[(size_t)pos * d_model + d];
      continue;
    }
    const float scale = (float)(trained - 1) / (float)(max_ctx - 1);
    const float p_scaled = (float)pos * scale;
    uint32_t p0 = (uint32_t)p_scaled;
    float alpha = p_scaled - (float)p0;
    if (p0 >= trained) {
      p0 = trained - 1;
      alpha = 0.0f;
    }
    uint32_t p1 = p0 + 1 < trained ? p0 + 1 : trained - 1;
    if (g_mutation == MUT_INTERP_SAME_ROW) p1 = p0; /* planted */
    const float v0 = table[(size_t)p0 * d_model + d];
    const float v1 = table[(size_t)p1 * d_model + d];
    out[d] = (1.0f - alpha) * v0 + alpha * v1;
  }
}

/* attention_fused.cu:1139-1162: values (2i, 2i+1) of every head of one row
 * rotated in place by pos * base^(-2i / d_head); an odd d_head leaves the
 * last value alone. */
#define DEFINE_ROPE(NAME, T, POW, COS, SIN)                                      \
  void NAME(T *qk, uint32_t pos, uint32_t n_heads, uint32_t d_head, T base) {    \
    for (uint32_t h = 0; h < n_heads; ++h)                                       \
      for (uint32_t i = 0; i < d_head / 2; ++i) {                                \
        const T two = g_mutation == MUT_ROPE_FREQ ? (T)1 : (T)2; /* planted */   \
        const T theta = POW(base, -two * (T)i / (T)d_head);                      \
        const T angle = (T)pos * theta;                                          \
        const T c = COS(angle);                                                  \
        const T s = g_mutation == MUT_ROPE_SIN_SIGN ? -SIN(angle) : SIN(angle);  \
        const size_t i0 = (size_t)h * d_head + 2 * (size_t)i;                    \
        const T x0 = qk[i0], x1 = qk[i0 + 1];                                    \
        qk[i0] = x0 * c - x1 * s;                                                \
        qk[i0 + 1] = x0 * s + x1 * c;                                            \
      }                                                                          \
  }

DEFINE_ROPE(oracle_apply_rope_f32, float, powf, cosf, sinf)
DEFINE_ROPE(oracle_apply_rope_f64, double, pow, cos, sin)

/* fp32 -> bf16 bit pattern, round to nearest even (__float2bfloat16_rn of
 * attention_fused.cu:1212); a NaN stays a NaN of the same sign, made quiet. */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  if (g_mutation == MUT_BF16_TRUNCATE) return (uint16_t)(u >> 16); /* planted */
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

/* attention_fused.cu:1178-1217: pool row phys_block * page_size + page_offset
 * := src, as fp32 (pool_bf16 = 0) or as bf16 bit patterns. */
void oracle_paged_copy_row(const float *src, void *pool, int pool_bf16, int32_t phys_block,
                           uint32_t page_offset, uint32_t page_size, uint32_t d_model) {
  const uint32_t off = g_mutation == MUT_PAGE_OFFSET && page_offset > 0 ? page_offset - 1 : page_offset;
  const size_t row = ((size_t)phys_block * page_size + off) * d_model; /* planted above */
  for (uint32_t d = 0; d < d_model; ++d) {
    if (pool_bf16)
      ((uint16_t *)pool)[row + d] = oracle_f32_to_bf16(src[d]);
    else
      ((float *)pool)[row + d] = src[d];
  }
}

/* Number of threads OpenMP would use by default (1 without OpenMP). */
int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
