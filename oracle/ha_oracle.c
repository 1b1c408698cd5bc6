/*
 * CPU oracle for the hybrid-attention hot path. TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C with fp64 arithmetic, what the reference engine computes for its two token
 * mixers and its prefix cache. It is the checker that the HIP kernels are compared against; nothing in the
 * product library links, loads or calls it. Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
 * leg use it.
 *
 * Reference (read as text; /root/reference, paths relative to it):
 *   web/public/engine/wgsl.js:124-139  CONV         depthwise causal conv (kernel 4) + SiLU over the qkv channels
 *   web/public/engine/wgsl.js:420-434  HIST_UPDATE  conv history <- last 3 pre-conv rows
 *   web/public/engine/wgsl.js:146-187  GDN          gated delta rule, sequential in t
 *   web/public/engine/wgsl.js:252-268  GNORM        per-head gated RMSNorm
 *   web/public/engine/wgsl.js:271-302  QK_PREP      q/k RMSNorm (stored weight = 1 + w) + rotate-half partial RoPE
 *   web/public/engine/wgsl.js:348-417  ATTN2        causal GQA, online softmax, sigmoid output gate
 *   web/public/engine/engine.js:105-106            RoPE table (angles in f64, stored f32)
 *   web/public/engine/engine.js:253-276            layer-kind dispatch and fused column offsets
 *   convert/export_engine.py:52-65                 fused row layouts and stored parameter forms
 * and the third-party fp32 semantics the reference's Python driver runs (transformers 5.17.0,
 * models/qwen3_5/modeling_qwen3_5.py, read as text): l2norm, torch_recurrent_gated_delta_rule,
 * torch_chunk_gated_delta_rule, Qwen3_5RMSNormGated, Qwen3_5RMSNorm, apply_rotary_pos_emb,
 * eager_attention_forward.
 *
 * Each function below says which of these it follows and which checks in tests/ pin it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_EPS 1e-6 /* hard-coded in every reference norm: wgsl.js:168-169 (l2), 263 (gnorm), 293 (rms) */

/* ---------------------------------------------------------------------------------------------------------- */
/* f16 rounding (round to nearest even), the engine's storage precision for Q, K/V and the attention output.     */
/* Pinned by tests/test_oracle.py::test_f16_round against numpy's float16 cast.                                  */
/* ---------------------------------------------------------------------------------------------------------- */
float orc_f16_round(float x) {
  union { float f; uint32_t u; } v = {x};
  uint32_t sign = v.u & 0x80000000u, a = v.u & 0x7fffffffu;
  if (a >= 0x7f800000u) return x;                      /* inf / nan pass through */
  if (a >= 0x477ff000u) { v.u = sign | 0x7f800000u; return v.f; } /* rounds past 65504 -> inf */
  if (a < 0x38800000u) {                               /* below the smallest normal f16: quantum 2^-24 */
    double q = ldexp(1.0, -24), m = fabs((double)x) / q, r = nearbyint(m);
    double y = r * q;
    return sign ? -(float)y : (float)y;
  }
  /* normal range: keep 10 mantissa bits, round to nearest even on the 13 dropped bits */
  uint32_t lsb = (a >> 13) & 1u, rounded = a + 0x0fffu + lsb;
  v.u = sign | (rounded & ~0x1fffu);
  return v.f;
}

/* ---------------------------------------------------------------------------------------------------------- */
/* RoPE table, engine.js:105-106: angle = t / theta^(2i/RD) in f64, stored as f32 (cos, sin) pairs, [LT][RD].   */
/* Pinned by tests/test_oracle.py::test_rope_table (closed form; position 0 is the identity rotation).          */
/* ---------------------------------------------------------------------------------------------------------- */
void orc_rope_table(int LT, int RD, double theta, float* out) {
  for (int t = 0; t < LT; t++)
    for (int i = 0; i < RD / 2; i++) {
      double a = (double)t / pow(theta, (2.0 * i) / RD);
      out[(size_t)t * RD + 2 * i] = (float)cos(a);
      out[(size_t)t * RD + 2 * i + 1] = (float)sin(a);
    }
}

static double silu(double x) { return x / (1.0 + exp(-x)); }
static double sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }
/* torch.nn.functional.softplus(beta=1, threshold=20), as wgsl.js:172 and HF GatedDeltaNet.forward use it */
static double softplus(double x) { return x > 20.0 ? x : log1p(exp(x)); }

/* ---------------------------------------------------------------------------------------------------------- */
/* Causal depthwise conv + SiLU (wgsl.js:124-139; HF causal_conv1d_fn / causal_conv1d_update) over channels     */
/* [0, C) of T fused rows; rows before t = 0 come from hist[KC-1][C]. Then the history roll of                    */
/* HIST_UPDATE (wgsl.js:420-434): hist <- last KC-1 pre-conv rows of (hist ++ rows).                              */
/* Pinned by tests/test_oracle.py::test_conv_* (direct sum, single-tap identity, history equivalence).           */
/* ---------------------------------------------------------------------------------------------------------- */
void orc_conv_silu(int T, int C, int KC, int stride, const float* rows, const float* w, float* hist, double* u) {
  for (int t = 0; t < T; t++)
    for (int c = 0; c < C; c++) {
      double s = 0.0;
      for (int j = 0; j < KC; j++) {
        int r = t - (KC - 1) + j;
        double x = r >= 0 ? rows[(size_t)r * stride + c] : hist[(size_t)(r + KC - 1) * C + c];
        s += (double)w[(size_t)c * KC + j] * x;
      }
      u[(size_t)t * C + c] = silu(s);
    }
  /* history roll */
  float* nh = (float*)malloc(sizeof(float) * (size_t)(KC - 1) * C);
  for (int r = 0; r < KC - 1; r++) {
    int src = T - (KC - 1) + r;
    for (int c = 0; c < C; c++)
      nh[(size_t)r * C + c] = src >= 0 ? rows[(size_t)src * stride + c] : hist[(size_t)(src + KC - 1) * C + c];
  }
  memcpy(hist, nh, sizeof(float) * (size_t)(KC - 1) * C);
  free(nh);
}

/* ---------------------------------------------------------------------------------------------------------- */
/* Per-token prologue of one head: l2-normalised q (times DK^-1/2) and k, beta = sigmoid(b),                     */
/* log-decay g = negA * softplus(a + dt_bias). wgsl.js:166-173; HF l2norm and GatedDeltaNet.forward              */
/* (beta = b.sigmoid(); g = -exp(A_log) * softplus(a + dt_bias); scale = 1/sqrt(d_k)).                            */
/* ---------------------------------------------------------------------------------------------------------- */
static void head_prologue(int DK, const double* uq, const double* uk, double* qn, double* kn) {
  double sq = 0.0, sk = 0.0;
  for (int i = 0; i < DK; i++) { sq += uq[i] * uq[i]; sk += uk[i] * uk[i]; }
  double rq = 1.0 / sqrt(sq + ORC_EPS) / sqrt((double)DK), rk = 1.0 / sqrt(sk + ORC_EPS);
  for (int i = 0; i < DK; i++) { qn[i] = uq[i] * rq; kn[i] = uk[i] * rk; }
}

/* GNORM (wgsl.js:252-268; HF Qwen3_5RMSNormGated): y = w * o * rsqrt(mean(o^2) + eps) * silu(z). */
static void gated_norm(int DV, const double* o, const float* z, const float* w, float* y) {
  double ss = 0.0;
  for (int j = 0; j < DV; j++) ss += o[j] * o[j];
  double inv = 1.0 / sqrt(ss / DV + ORC_EPS);
  for (int j = 0; j < DV; j++) y[j] = (float)((double)w[j] * o[j] * inv * silu((double)z[j]));
}

/* ---------------------------------------------------------------------------------------------------------- */
/* One gated-delta layer over T new rows of ONE sequence: conv + SiLU, normalised q/k, gates, the delta rule,   */
/* and (if gnorm_w) the gated RMSNorm. This is the engine's linear_attention step (engine.js:262-269).            */
/*                                                                                                              */
/* rows    [T][stride] fused in_proj rows: qkv at [0, C), z at C, a at C + H*DV, b at C + H*DV + H, with           */
/*         C = 2*H*DK + H*DV (engine.js:264-267; export_engine.py:52)                                            */
/* conv_w  [C][KC]; negA, dt_bias [H] (negA = -exp(A_log), export_engine.py:56-57); gnorm_w [DV] or NULL          */
/* hist    [KC-1][C] pre-conv rows before t = 0, updated in place                                                 */
/* S       [H][DK][DV] recurrent state in fp64, updated in place                                                  */
/* out     [T][H*DV]: gnorm output, or the raw core output o when gnorm_w is NULL                                  */
/* chunk   0: the sequential rule (wgsl.js:176-183; HF torch_recurrent_gated_delta_rule)                           */
/*         n>0: the chunked WY/UT form with chunks of n rows counted from t = 0 of this call                      */
/*              (HF torch_chunk_gated_delta_rule, incl. its forward substitution), in fp64                        */
/* Pinned by tests/test_oracle.py: one-token closed form, beta = 0 decay closed form, orthonormal-key recall,     */
/* brute force (numpy) on tiny shapes, prefix-state composition, sequential == chunked.                           */
/* ---------------------------------------------------------------------------------------------------------- */
int orc_gdn_forward(int T, int H, int DK, int DV, int KC, int stride, const float* rows, const float* conv_w,
                    const float* negA, const float* dt_bias, const float* gnorm_w, float* hist, double* S,
                    float* out, int chunk) {
  const int C = 2 * H * DK + H * DV;
  const int zoff = C, aoff = C + H * DV, boff = C + H * DV + H;
  if (T <= 0) return 0;
  double* u = (double*)malloc(sizeof(double) * (size_t)T * C);
  if (!u) return -1;
  orc_conv_silu(T, C, KC, stride, rows, conv_w, hist, u);

#pragma omp parallel for schedule(dynamic, 1)
  for (int h = 0; h < H; h++) {
    double* qn = (double*)malloc(sizeof(double) * (size_t)T * DK);
    double* kn = (double*)malloc(sizeof(double) * (size_t)T * DK);
    double* v = (double*)malloc(sizeof(double) * (size_t)T * DV);
    double* g = (double*)malloc(sizeof(double) * T);
    double* beta = (double*)malloc(sizeof(double) * T);
    double* o = (double*)malloc(sizeof(double) * (size_t)T * DV);
    double* Sh = S + (size_t)h * DK * DV;
    for (int t = 0; t < T; t++) {
      const double* ut = u + (size_t)t * C;
      head_prologue(DK, ut + h * DK, ut + H * DK + h * DK, qn + (size_t)t * DK, kn + (size_t)t * DK);
      for (int j = 0; j < DV; j++) v[(size_t)t * DV + j] = ut[2 * H * DK + h * DV + j];
      const float* row = rows + (size_t)t * stride;
      beta[t] = sigmoid((double)row[boff + h]);
      g[t] = (double)negA[h] * softplus((double)row[aoff + h] + (double)dt_bias[h]);
    }
    if (chunk <= 0) {
      double* r = (double*)malloc(sizeof(double) * DV);
      for (int t = 0; t < T; t++) {
        const double al = exp(g[t]), *k = kn + (size_t)t * DK, *q = qn + (size_t)t * DK;
        for (int e = 0; e < DK * DV; e++) Sh[e] *= al;                       /* S <- alpha S */
        for (int j = 0; j < DV; j++) r[j] = 0.0;
        for (int i = 0; i < DK; i++)
          for (int j = 0; j < DV; j++) r[j] += Sh[(size_t)i * DV + j] * k[i];  /* r = S^T k */
        for (int j = 0; j < DV; j++) r[j] = beta[t] * (v[(size_t)t * DV + j] - r[j]); /* delta */
        for (int i = 0; i < DK; i++)
          for (int j = 0; j < DV; j++) Sh[(size_t)i * DV + j] += k[i] * r[j]; /* S += k delta^T */
        double* ot = o + (size_t)t * DV;
        for (int j = 0; j < DV; j++) ot[j] = 0.0;
        for (int i = 0; i < DK; i++)
          for (int j = 0; j < DV; j++) ot[j] += Sh[(size_t)i * DV + j] * q[i]; /* o = S^T q */
      }
      free(r);
    } else {
      const int n = chunk;
      double* gc = (double*)malloc(sizeof(double) * n);
      double* A = (double*)malloc(sizeof(double) * (size_t)n * n);
      double* U = (double*)malloc(sizeof(double) * (size_t)n * DV);
      double* W = (double*)malloc(sizeof(double) * (size_t)n * DK);
      double* Vn = (double*)malloc(sizeof(double) * (size_t)n * DV);
      for (int c0 = 0; c0 < T; c0 += n) {
        const int m = T - c0 < n ? T - c0 : n; /* rows in this chunk; the rest is zero padding, as HF pads */
        double acc = 0.0;
        for (int i = 0; i < m; i++) { acc += g[c0 + i]; gc[i] = acc; }
        /* A = strictly-lower( beta_i (k_i . k_j) exp(g_i - g_j) ); T = (I + A)^-1 by forward substitution */
        for (int i = 0; i < m; i++)
          for (int j = 0; j < m; j++) {
            double s = 0.0;
            if (j < i) {
              for (int d = 0; d < DK; d++) s += kn[(size_t)(c0 + i) * DK + d] * kn[(size_t)(c0 + j) * DK + d];
              s *= beta[c0 + i] * exp(gc[i] - gc[j]);
            }
            A[(size_t)i * n + j] = s;
          }
        /* rows of T: T_i = e_i - sum_{j<i} A_ij T_j */
        for (int i = 0; i < m; i++) {
          double* Ti = A + (size_t)i * n; /* overwrite row i of A by row i of T, using rows j < i already done */
          double tmp[512];
          for (int c = 0; c < m; c++) tmp[c] = (c == i) ? 1.0 : 0.0;
          for (int j = 0; j < i; j++) {
            double aij = Ti[j];
            if (aij != 0.0)
              for (int c = 0; c <= j; c++) tmp[c] -= aij * A[(size_t)j * n + c];
          }
          for (int c = 0; c < m; c++) Ti[c] = tmp[c];
        }
        /* U = T (beta v), W = T (beta exp(g) k) */
        for (int i = 0; i < m; i++) {
          for (int j = 0; j < DV; j++) {
            double s = 0.0;
            for (int c = 0; c <= i; c++) s += A[(size_t)i * n + c] * beta[c0 + c] * v[(size_t)(c0 + c) * DV + j];
            U[(size_t)i * DV + j] = s;
          }
          for (int d = 0; d < DK; d++) {
            double s = 0.0;
            for (int c = 0; c <= i; c++)
              s += A[(size_t)i * n + c] * beta[c0 + c] * exp(gc[c]) * kn[(size_t)(c0 + c) * DK + d];
            W[(size_t)i * DK + d] = s;
          }
        }
        /* v_new = U - W S; o = (q exp(g)) S + (q k^T * decay, causal) v_new */
        for (int i = 0; i < m; i++)
          for (int j = 0; j < DV; j++) {
            double s = U[(size_t)i * DV + j];
            for (int d = 0; d < DK; d++) s -= W[(size_t)i * DK + d] * Sh[(size_t)d * DV + j];
            Vn[(size_t)i * DV + j] = s;
          }
        for (int i = 0; i < m; i++) {
          double* ot = o + (size_t)(c0 + i) * DV;
          const double* q = qn + (size_t)(c0 + i) * DK;
          double eg = exp(gc[i]);
          for (int j = 0; j < DV; j++) {
            double s = 0.0;
            for (int d = 0; d < DK; d++) s += q[d] * eg * Sh[(size_t)d * DV + j];
            ot[j] = s;
          }
          for (int c = 0; c <= i; c++) {
            double qk = 0.0;
            for (int d = 0; d < DK; d++) qk += q[d] * kn[(size_t)(c0 + c) * DK + d];
            qk *= exp(gc[i] - gc[c]);
            for (int j = 0; j < DV; j++) ot[j] += qk * Vn[(size_t)c * DV + j];
          }
        }
        /* S <- exp(g_last) S + (k exp(g_last - g))^T v_new */
        double gl = gc[m - 1], el = exp(gl);
        for (int e = 0; e < DK * DV; e++) Sh[e] *= el;
        for (int c = 0; c < m; c++) {
          double f = exp(gl - gc[c]);
          for (int d = 0; d < DK; d++) {
            double kd = kn[(size_t)(c0 + c) * DK + d] * f;
            for (int j = 0; j < DV; j++) Sh[(size_t)d * DV + j] += kd * Vn[(size_t)c * DV + j];
          }
        }
      }
      free(gc); free(A); free(U); free(W); free(Vn);
    }
    for (int t = 0; t < T; t++) {
      float* y = out + (size_t)t * H * DV + (size_t)h * DV;
      const double* ot = o + (size_t)t * DV;
      if (gnorm_w)
        gated_norm(DV, ot, rows + (size_t)t * stride + zoff + h * DV, gnorm_w, y);
      else
        for (int j = 0; j < DV; j++) y[j] = (float)ot[j];
    }
    free(qn); free(kn); free(v); free(g); free(beta); free(o);
  }
  free(u);
  return 0;
}

/* ---------------------------------------------------------------------------------------------------------- */
/* One gated causal GQA layer over T new rows of ONE sequence that continues P cached tokens.                     */
/* QK_PREP (wgsl.js:271-302; HF Qwen3_5RMSNorm with (1 + w), apply_rotary_pos_emb): q, k RMS-normalised with the   */
/* stored weights (already 1 + w, export_engine.py:64-65), rotate-half RoPE on dims [0, RD) at position P + t      */
/* from the engine's table; K, V written to the cache at row P + t. ATTN2 (wgsl.js:348-417; HF                      */
/* eager_attention_forward + sigmoid gate): scores q.k / sqrt(HD) over keys 0..P+t, softmax, value sum,            */
/* times sigmoid(gate).                                                                                           */
/*                                                                                                              */
/* rows  [T][stride]: head h has [q (HD) | gate (HD)] at h*2*HD, k at HQ*2*HD + kh*HD,                             */
/*       v at HQ*2*HD + HK*HD + kh*HD (wgsl.js:285-286; export_engine.py:61)                                     */
/* rope  [LT][RD] cos/sin pairs (orc_rope_table); Kc, Vc [HK][LT][HD]; out [T][HQ*HD]                             */
/* f16   1: round where the engine stores f16 (Q, K, V after prep; the score-side q/16; the output)               */
/* Pinned by tests/test_oracle.py: fp64 softmax brute force (numpy), position-0 identity, GQA head map,           */
/* RMSNorm closed form, gate closed form, prefix composition.                                                      */
/* ---------------------------------------------------------------------------------------------------------- */
int orc_gqa_forward(int T, int P, int LT, int HQ, int HK, int HD, int RD, int stride, const float* rows,
                    const float* q_norm_w, const float* k_norm_w, const float* rope, float* Kc, float* Vc,
                    float* out, int f16) {
  if (P + T > LT) return -2;
  if (T <= 0) return 0;
  const int G = HQ / HK, koff = HQ * 2 * HD, voff = HQ * 2 * HD + HK * HD;
  float* Q = (float*)malloc(sizeof(float) * (size_t)HQ * T * HD);
  double* nv = (double*)malloc(sizeof(double) * HD);
  /* prep: slots 0..HQ-1 are q heads, HQ.. are k heads (wgsl.js:283-301) */
  for (int t = 0; t < T; t++) {
    const int pos = P + t;
    const float* row = rows + (size_t)t * stride;
    for (int s = 0; s < HQ + HK; s++) {
      const int isq = s < HQ;
      const float* src = isq ? row + s * 2 * HD : row + koff + (s - HQ) * HD;
      const float* w = isq ? q_norm_w : k_norm_w;
      double ss = 0.0;
      for (int d = 0; d < HD; d++) ss += (double)src[d] * src[d];
      double inv = 1.0 / sqrt(ss / HD + ORC_EPS);
      for (int d = 0; d < HD; d++) nv[d] = (double)src[d] * inv * w[d];
      float* dst = isq ? Q + ((size_t)s * T + t) * HD : Kc + ((size_t)(s - HQ) * LT + pos) * HD;
      for (int d = 0; d < HD; d++) {
        double r = nv[d];
        if (d < RD) {
          int i = d % (RD / 2);
          double cs = rope[(size_t)pos * RD + 2 * i], sn = rope[(size_t)pos * RD + 2 * i + 1];
          r = d < RD / 2 ? nv[d] * cs - nv[d + RD / 2] * sn : nv[d] * cs + nv[d - RD / 2] * sn;
        }
        dst[d] = f16 ? orc_f16_round((float)r) : (float)r;
      }
    }
    for (int kh = 0; kh < HK; kh++)
      for (int d = 0; d < HD; d++) {
        float v = row[voff + kh * HD + d];
        Vc[((size_t)kh * LT + pos) * HD + d] = f16 ? orc_f16_round(v) : v;
      }
  }
  free(nv);
  const double scale = 1.0 / sqrt((double)HD);
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int h = 0; h < HQ; h++)
    for (int t = 0; t < T; t++) {
      const int kh = h / G, last = P + t;
      double* sc = (double*)malloc(sizeof(double) * (size_t)(last + 1));
      double acc[1024];
      const float* q = Q + ((size_t)h * T + t) * HD;
      double mx = -INFINITY;
      for (int j = 0; j <= last; j++) {
        const float* k = Kc + ((size_t)kh * LT + j) * HD;
        double s = 0.0;
        if (f16) {
          /* ATTN2 scales q by 1/sqrt(HD) and stores it as f16 before the dot products (wgsl.js:368) */
          for (int d = 0; d < HD; d++) s += (double)orc_f16_round((float)(q[d] * scale)) * k[d];
        } else {
          for (int d = 0; d < HD; d++) s += (double)q[d] * k[d];
          s *= scale;
        }
        sc[j] = s;
        if (s > mx) mx = s;
      }
      double l = 0.0;
      for (int d = 0; d < HD; d++) acc[d] = 0.0;
      for (int j = 0; j <= last; j++) {
        double p = exp(sc[j] - mx);
        l += p;
        const float* v = Vc + ((size_t)kh * LT + j) * HD;
        for (int d = 0; d < HD; d++) acc[d] += p * v[d];
      }
      const float* gate = rows + (size_t)t * stride + h * 2 * HD + HD;
      float* o = out + (size_t)t * HQ * HD + (size_t)h * HD;
      for (int d = 0; d < HD; d++) {
        double y = acc[d] / l * sigmoid((double)gate[d]);
        o[d] = f16 ? orc_f16_round((float)y) : (float)y;
      }
      free(sc);
    }
  free(Q);
  return 0;
}
