/* Brute-force fp64 GQA softmax attention, forward and backward -- TEST
 * INFRASTRUCTURE ONLY (loaded by tests/ through ctypes to pin oracle/reference.py).
 *
 * Direct loops over the definition, independent of torch:
 *   s_ij  = sm_scale * q_i . k_j            (keys j <= i when causal)
 *   P_ij  = exp(s_ij - m_i) / l_i,  m_i = max_j s_ij,  l_i = sum_j exp(s_ij - m_i)
 *   o_i   = sum_j P_ij v_j
 *   lse2_i = log2(e) * (m_i + ln l_i)         (the kernel's log2-unit LSE,
 *                                              CODE/mimans/model/attention_tilelang.py:186-188)
 * Backward from the chain rule through the softmax (not from any kernel):
 *   dP_ij = dO_i . v_j,   Delta_i = sum_j P_ij dP_ij,   dS_ij = P_ij (dP_ij - Delta_i)
 *   dq_i  = sm_scale * sum_j dS_ij k_j
 *   dk_j += sm_scale * sum_i dS_ij q_i,   dv_j += sum_i P_ij dO_i
 * with dk/dv summed over the query heads h of KV head h / (H / Hkv).
 * brute_attn_bwd also returns Delta_i = sum_j P_ij dP_ij (the form of Delta
 * that does not go through O).
 *
 * brute_attn_bwd_emul: the same backward with the rounding points of the
 * reference's TileLang kernel (CODE/mimans/model/attention_tilelang.py),
 * everything else exact (fp64):
 *   O rounded to bf16 (the forward's bf16 output, :182-185) and
 *   Delta_i = sum_d bf16(O)_id dO_id                           (:212-214)
 *   dV_j += sum_i bf16(P_ij) dO_i                              (:306-307)
 *   dS_ij = bf16(P_ij (dP_ij - Delta_i) sm_scale)              (:310)
 *   dK_j += sum_i dS_ij Q_i,  dQ_i = sum_j dS_ij K_j           (:311-314)
 * bf16() rounds to fp32, then to 8 significant bits (both nearest even).
 * Layouts: q/o/dO/dq [B,S,H,D], k/v/dk/dv [B,S,Hkv,D], lse2/delta [B,H,S],
 * row-major.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

static long at4(int b, int s, int h, int d, int S, int H, int D) {
  return (((long)b * S + s) * H + h) * D + d;
}

/* Softmax row i of head (b, h): fills p[0..S) (zeros beyond the causal limit),
 * returns lse2. */
static double row_probs(const double* q, const double* k, int b, int i, int h, int g,
                        int S, int H, int Hkv, int D, int causal, double sm_scale, double* p) {
  const int jmax = causal ? i : S - 1;
  double m = -INFINITY;
  for (int j = 0; j < S; ++j) {
    if (j > jmax) { p[j] = 0.0; continue; }
    double acc = 0.0;
    for (int d = 0; d < D; ++d) acc += q[at4(b, i, h, d, S, H, D)] * k[at4(b, j, g, d, S, Hkv, D)];
    p[j] = acc * sm_scale;
    if (p[j] > m) m = p[j];
  }
  double l = 0.0;
  for (int j = 0; j <= jmax; ++j) { p[j] = exp(p[j] - m); l += p[j]; }
  for (int j = 0; j <= jmax; ++j) p[j] /= l;
  return (m + log(l)) * 1.4426950408889634;
}

void brute_attn_fwd(const double* q, const double* k, const double* v, double* o, double* lse2,
                    int B, int S, int H, int Hkv, int D, int causal, double sm_scale) {
  const int G = H / Hkv;
  double* p = (double*)malloc(sizeof(double) * S);
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int g = h / G;
      for (int i = 0; i < S; ++i) {
        lse2[((long)b * H + h) * S + i] = row_probs(q, k, b, i, h, g, S, H, Hkv, D, causal, sm_scale, p);
        for (int d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int j = 0; j < S; ++j) acc += p[j] * v[at4(b, j, g, d, S, Hkv, D)];
          o[at4(b, i, h, d, S, H, D)] = acc;
        }
      }
    }
  free(p);
}

/* bfloat16 rounding of a double as the kernels' fp32 values see it: round
 * to fp32 (nearest even), then to 8 significant bits (nearest even) -- the
 * same two steps as torch's float64 -> bfloat16 conversion. */
static double bf16_rne(double x) {
  const float f = (float)x;
  if (f == 0.0f || !isfinite(f)) return (double)f;
  int e;
  const double m = frexp((double)f, &e);  /* f = m * 2^e, 0.5 <= |m| < 1 */
  return ldexp(nearbyint(ldexp(m, 8)), e - 8);
}

double brute_bf16(double x) { return bf16_rne(x); }

void brute_attn_bwd(const double* q, const double* k, const double* v, const double* dO,
                    double* dq, double* dk, double* dv, double* delta_out,
                    int B, int S, int H, int Hkv, int D, int causal, double sm_scale) {
  const int G = H / Hkv;
  double* p = (double*)malloc(sizeof(double) * S);
  double* dp = (double*)malloc(sizeof(double) * S);
  memset(dk, 0, sizeof(double) * (size_t)B * S * Hkv * D);
  memset(dv, 0, sizeof(double) * (size_t)B * S * Hkv * D);
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int g = h / G;
      for (int i = 0; i < S; ++i) {
        row_probs(q, k, b, i, h, g, S, H, Hkv, D, causal, sm_scale, p);
        double delta = 0.0;
        for (int j = 0; j < S; ++j) {
          double acc = 0.0;
          for (int d = 0; d < D; ++d) acc += dO[at4(b, i, h, d, S, H, D)] * v[at4(b, j, g, d, S, Hkv, D)];
          dp[j] = acc;
          delta += p[j] * acc;
        }
        if (delta_out) delta_out[((long)b * H + h) * S + i] = delta;
        for (int d = 0; d < D; ++d) dq[at4(b, i, h, d, S, H, D)] = 0.0;
        for (int j = 0; j < S; ++j) {
          const double ds = p[j] * (dp[j] - delta);
          for (int d = 0; d < D; ++d) {
            dq[at4(b, i, h, d, S, H, D)] += sm_scale * ds * k[at4(b, j, g, d, S, Hkv, D)];
            dk[at4(b, j, g, d, S, Hkv, D)] += sm_scale * ds * q[at4(b, i, h, d, S, H, D)];
            dv[at4(b, j, g, d, S, Hkv, D)] += p[j] * dO[at4(b, i, h, d, S, H, D)];
          }
        }
      }
    }
  free(p);
  free(dp);
}

void brute_attn_bwd_emul(const double* q, const double* k, const double* v, const double* dO,
                         double* dq, double* dk, double* dv, double* delta_out,
                         int B, int S, int H, int Hkv, int D, int causal, double sm_scale) {
  const int G = H / Hkv;
  double* p = (double*)malloc(sizeof(double) * S);
  memset(dk, 0, sizeof(double) * (size_t)B * S * Hkv * D);
  memset(dv, 0, sizeof(double) * (size_t)B * S * Hkv * D);
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int g = h / G;
      for (int i = 0; i < S; ++i) {
        row_probs(q, k, b, i, h, g, S, H, Hkv, D, causal, sm_scale, p);
        /* Delta from the bf16-rounded forward output */
        double delta = 0.0;
        for (int d = 0; d < D; ++d) {
          double o = 0.0;
          for (int j = 0; j < S; ++j) o += p[j] * v[at4(b, j, g, d, S, Hkv, D)];
          delta += bf16_rne(o) * dO[at4(b, i, h, d, S, H, D)];
        }
        if (delta_out) delta_out[((long)b * H + h) * S + i] = delta;
        for (int d = 0; d < D; ++d) dq[at4(b, i, h, d, S, H, D)] = 0.0;
        for (int j = 0; j < S; ++j) {
          double dp = 0.0;
          for (int d = 0; d < D; ++d) dp += dO[at4(b, i, h, d, S, H, D)] * v[at4(b, j, g, d, S, Hkv, D)];
          const double ds = bf16_rne(p[j] * (dp - delta) * sm_scale);
          const double pb = bf16_rne(p[j]);
          for (int d = 0; d < D; ++d) {
            dq[at4(b, i, h, d, S, H, D)] += ds * k[at4(b, j, g, d, S, Hkv, D)];
            dk[at4(b, j, g, d, S, Hkv, D)] += ds * q[at4(b, i, h, d, S, H, D)];
            dv[at4(b, j, g, d, S, Hkv, D)] += pb * dO[at4(b, i, h, d, S, H, D)];
          }
        }
      }
    }
  free(p);
}
