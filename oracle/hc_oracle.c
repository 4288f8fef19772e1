/*
 * CPU oracle for the hot-tier kernels -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * this file, as the checker.  It is a plain-C restatement, written
 * independently of the HIP kernels, of the window-scoring arithmetic that
 * makes kept indices reproducible:
 *
 *   snapkv_importance  (src/hotcold_kv/baselines/scoring.py:50-79)
 *     _group_query_to_kv (scoring.py:17-26), pool1d (scoring.py:40-47)
 *   raw-logit scoring of HotColdLayer._compress_if_needed (src/hotcold_kv/cache.py:55-69)
 *
 * Contract (every step one IEEE-754 operation, so results are bit-exact):
 *   qf[w][d]   = (sum_g (double)q[g][w][d]) / G, g ascending, starting from q[0]
 *   dot[w][s]  = fma(qf[w][D-1], k[s][D-1], ... fma(qf[w][0], k[s][0], 0.0))
 *   snapkv:  L = (float)(dot * scaling), -inf for s > S-W+w (scoring.py:72-74)
 *            m_w = max_s L ; e = exp_det((double)L - (double)m_w)
 *            l_w = 2^-44 * sum_s rint(e * 2^44)          (exact integer sum)
 *            imp[s] = (float)(fma(e_{W-1}, 1/l_{W-1}, ... fma(e_0, 1/l_0, 0.0)))
 *   rawsum:  L = (float)(dot / sqrt(D)) ; imp[s] = (float)(sum_w (double)L), w ascending
 *   pool:    max over [s-P, s+P] within [0,S) (max_pool1d pads with -inf), or
 *            (float)((sum_j (double)imp[j], j ascending, pad = 0) / k) (avg_pool1d,
 *            count_include_pad=True)
 * exp_det: Cody-Waite reduction with fdlibm's ln2 split, degree-12 Taylor
 * polynomial in Horner form, 2^k from the exponent bits; 0 below -708.
 *
 * Inputs are fp64 arrays holding the exact values of the fp16/bf16/fp32
 * tensors (every such value is exactly representable in fp64).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define LN2_HI 6.93147180369123816490e-01
#define LN2_LO 1.90821492927058770002e-10
#define INV_LN2 1.44269504088896338700e+00

double hco_exp_det(double x) {
  if (!(x >= -708.0)) return 0.0;
  double kf = rint(x * INV_LN2);
  double r = fma(-kf, LN2_HI, x);
  r = fma(-kf, LN2_LO, r);
  /* Taylor coefficients 1/n!, n = 12 .. 0 */
  static const double c[13] = {
      2.08767569878680989792e-09, 2.50521083854417187751e-08, 2.75573192239858906526e-07,
      2.75573192239858906526e-06, 2.48015873015873015873e-05, 1.98412698412698412698e-04,
      1.38888888888888888889e-03, 8.33333333333333333333e-03, 4.16666666666666666667e-02,
      1.66666666666666666667e-01, 5.00000000000000000000e-01, 1.0, 1.0};
  double p = c[0];
  for (int i = 1; i < 13; ++i) p = fma(p, r, c[i]);
  int64_t k = (int64_t)kf;
  uint64_t bits = (uint64_t)(k + 1023) << 52;
  double scale;
  memcpy(&scale, &bits, sizeof scale);
  return p * scale;
}

static uint64_t fix44(double e) { return (uint64_t)rint(e * 17592186044416.0); }

/*
 * q: element (b, hq, row, d) at q[b*q_sb + hq*q_sh + row*q_ss + d], rows
 *    q_row0 .. q_row0+W-1 are the window.
 * k: element (b, hk, s, d) at k[b*k_sb + hk*k_sh + s*k_ss + d].
 * out: float [B][Hk][S].
 * mode 0 = snapkv, 1 = rawsum.  kernel_size <= 1: no pooling.  pooling 0 = max, 1 = avg.
 * Returns 0, or -1 on bad arguments / allocation failure.
 */
int hco_window_scores(int mode, int64_t B, int64_t Hq, int64_t Hk, int64_t S, int64_t D, int64_t W,
                      const double* q, int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t q_row0,
                      const double* k, int64_t k_sb, int64_t k_sh, int64_t k_ss, double scaling,
                      int64_t kernel_size, int pooling, float* out) {
  if (B <= 0 || Hq <= 0 || Hk <= 0 || S <= 0 || D <= 0 || W <= 0 || W > S) return -1;
  if (kernel_size > 1 && kernel_size % 2 == 0) return -1;
  double* qf = (double*)malloc(sizeof(double) * (size_t)(W * D));
  float* L = (float*)malloc(sizeof(float) * (size_t)(W * S));
  double* inv = (double*)malloc(sizeof(double) * (size_t)W);
  float* mx = (float*)malloc(sizeof(float) * (size_t)W);
  float* imp = (float*)malloc(sizeof(float) * (size_t)S);
  if (!qf || !L || !inv || !mx || !imp) {
    free(qf); free(L); free(inv); free(mx); free(imp);
    return -1;
  }
  const double sqrt_d = sqrt((double)D);
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < Hk; ++h) {
      /* GQA mean (scoring.py:17-26) */
      int64_t g0, G;
      if (Hq % Hk == 0) { G = Hq / Hk; g0 = h * G; } else { G = Hq; g0 = 0; }
      for (int64_t w = 0; w < W; ++w)
        for (int64_t d = 0; d < D; ++d) {
          const double* src = q + b * q_sb + (q_row0 + w) * q_ss + d;
          double sum = src[g0 * q_sh];
          for (int64_t g = 1; g < G; ++g) sum = sum + src[(g0 + g) * q_sh];
          qf[w * D + d] = sum / (double)G;
        }
      /* window logits */
      for (int64_t w = 0; w < W; ++w) {
        const int64_t qpos = S - W + w;
        for (int64_t s = 0; s < S; ++s) {
          const double* kr = k + b * k_sb + h * k_sh + s * k_ss;
          double acc = 0.0;
          for (int64_t d = 0; d < D; ++d) acc = fma(qf[w * D + d], kr[d], acc);
          float l;
          if (mode == 0) {
            l = (float)(acc * scaling);
            if (s > qpos) l = -INFINITY;
          } else {
            l = (float)(acc / sqrt_d);
          }
          L[w * S + s] = l;
        }
      }
      /* importance */
      if (mode == 0) {
        for (int64_t w = 0; w < W; ++w) {
          float m = -INFINITY;
          for (int64_t s = 0; s < S; ++s) m = fmaxf(m, L[w * S + s]);
          mx[w] = m;
          uint64_t tot = 0;
          for (int64_t s = 0; s < S; ++s) tot += fix44(hco_exp_det((double)L[w * S + s] - (double)m));
          inv[w] = 1.0 / ((double)tot * 0x1p-44);
        }
        for (int64_t s = 0; s < S; ++s) {
          double acc = 0.0;
          for (int64_t w = 0; w < W; ++w)
            acc = fma(hco_exp_det((double)L[w * S + s] - (double)mx[w]), inv[w], acc);
          imp[s] = (float)acc;
        }
      } else {
        for (int64_t s = 0; s < S; ++s) {
          double acc = 0.0;
          for (int64_t w = 0; w < W; ++w) acc = acc + (double)L[w * S + s];
          imp[s] = (float)acc;
        }
      }
      /* pooling (scoring.py:40-47) */
      float* o = out + (b * Hk + h) * S;
      if (kernel_size <= 1) {
        memcpy(o, imp, sizeof(float) * (size_t)S);
      } else {
        const int64_t P = kernel_size / 2;
        for (int64_t s = 0; s < S; ++s) {
          if (pooling == 0) {
            float m = -INFINITY;
            for (int64_t j = s - P; j <= s + P; ++j)
              if (j >= 0 && j < S) m = fmaxf(m, imp[j]);
            o[s] = m;
          } else {
            double sum = 0.0;
            for (int64_t j = s - P; j <= s + P; ++j)
              if (j >= 0 && j < S) sum = sum + (double)imp[j];
            o[s] = (float)(sum / (double)kernel_size);
          }
        }
      }
    }
  }
  free(qf); free(L); free(inv); free(mx); free(imp);
  return 0;
}

/* Mean over heads: out[b][s] = (float)((sum_h (double)x[b][h][s]) / H), h ascending. */
void hco_head_mean(int64_t B, int64_t H, int64_t S, const float* x, float* out) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t s = 0; s < S; ++s) {
      double acc = 0.0;
      for (int64_t h = 0; h < H; ++h) acc = acc + (double)x[(b * H + h) * S + s];
      out[b * S + s] = (float)(acc / (double)H);
    }
}
