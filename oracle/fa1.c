/*
 * Float32 restatement of femtochat's blocked FlashAttention-1 CPU path.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ to cross-check the float64 oracle
 * (oracle/attention_ref.py).  Its products are scalar loops; the CPU baseline
 * bench.py times is oracle/fa1_blas.py, the same algorithm with BLAS
 * products as the reference's mul! calls.  Nothing in femtochat_amd calls it.
 *
 * fa1_forward restates flash_attention₁! (src/kernels.jl:131-219):
 *   512-wide key blocks (outer) x 512-wide query blocks (inner), no block
 *   skipping and no skipping of masked (zero) entries inside a block; S = K_j^T Q_i * (1/sqrt(D)); masked entries = -floatmax
 *   (:150, :194); block max m~ over the whole column (masked included),
 *   P~ = mask ? exp(S - m~) : 0, l~ = sum P~; m_new = max(m, m~);
 *   l_new = e^(m-m_new) l + e^(m~-m_new) l~; O re-normalised every block:
 *   O = (O l e^(m-m_new) + V_j P~ e^(m~-m_new)) / max(l_new, eps) (:207-210).
 *   Initial O = 0, l = 0, m = -Inf (:146).
 * fa1_backward restates Δflash_attention₁! (src/kernels.jl:287-379):
 *   P = mask ? exp(S - m)/max(l, eps) : 0; dV += dO P^T; dP = dO V^T;
 *   D = rowsum(dO . O) recomputed per block pair; dS = P (dP - D);
 *   dQ += tau K dS; dK += tau Q dS^T.  It ACCUMULATES into dQ/dK/dV.
 * The mask restates attention_mask! (src/kernels.jl:30-42); positions (may be
 * NULL) add the document rule k >= q - positions[q] (not in the reference).
 *
 * Layout (row-major): Q,O,dO,dQ [B][T][H][D]; K,V,dK,dV [B][T][Hkv][D];
 * l,m [B][H][T]; positions [B][T].  Work is split over (batch, head) in the
 * forward and (batch, KV head) in the backward with OpenMP.
 */
#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define BLK 512

static inline int visible(int q, int k, int left, int right, int causal, const int* pos) {
  int v = causal ? (k <= q) : (q - left <= k && k <= q + right);
  if (pos != NULL) v = v && (k >= q - pos[q]);
  return v;
}

typedef struct {
  int D, H, Hkv, T, B, left, right, causal;
} dims;

/* S[qq*nj + kk] = scale * sum_d X[qq][d] * Yt[d][kk]  (Yt = transposed key-side block) */
static void scores(float* S, const float* X, long xpitch, const float* Yt, int ni, int nj, int D, float scale) {
  for (int qq = 0; qq < ni; ++qq) {
    float* row = S + (long)qq * nj;
    const float* x = X + (long)qq * xpitch;
    for (int kk = 0; kk < nj; ++kk) row[kk] = 0.0f;
    for (int d = 0; d < D; ++d) {
      const float xv = x[d];
      const float* y = Yt + (long)d * nj;
      for (int kk = 0; kk < nj; ++kk) row[kk] += xv * y[kk];
    }
    for (int kk = 0; kk < nj; ++kk) row[kk] *= scale;
  }
}

static void transpose_block(float* Yt, const float* Y, long pitch, int nj, int D) {
  for (int kk = 0; kk < nj; ++kk)
    for (int d = 0; d < D; ++d) Yt[(long)d * nj + kk] = Y[(long)kk * pitch + d];
}

static void forward_head(const dims* z, int b, int h, const float* Q, const float* K, const float* V, float* O,
                         float* l, float* m, const int* positions, float* S, float* Yt, float* Ot) {
  const int D = z->D, T = z->T, H = z->H, Hkv = z->Hkv;
  const int kv = h / (H / Hkv);
  const long qp = (long)H * D, kp = (long)Hkv * D;
  const float* Qb = Q + ((long)b * T * H + h) * D;
  float* Ob = O + ((long)b * T * H + h) * D;
  const float* Kb = K + ((long)b * T * Hkv + kv) * D;
  const float* Vb = V + ((long)b * T * Hkv + kv) * D;
  float* lb = l + ((long)b * H + h) * T;
  float* mb = m + ((long)b * H + h) * T;
  const int* pos = positions ? positions + (long)b * T : NULL;
  const float scale = 1.0f / sqrtf((float)D);
  const float masked = -FLT_MAX;

  for (int t = 0; t < T; ++t) {
    for (int d = 0; d < D; ++d) Ob[t * qp + d] = 0.0f;
    lb[t] = 0.0f;
    mb[t] = -INFINITY;
  }
  for (int j0 = 0; j0 < T; j0 += BLK) {
    const int nj = T - j0 < BLK ? T - j0 : BLK;
    transpose_block(Yt, Kb + j0 * kp, kp, nj, D);
    for (int i0 = 0; i0 < T; i0 += BLK) {
      const int ni = T - i0 < BLK ? T - i0 : BLK;
      scores(S, Qb + i0 * qp, qp, Yt, ni, nj, D, scale);
      for (int qq = 0; qq < ni; ++qq) {
        const int q = i0 + qq;
        float* row = S + (long)qq * nj;
        float mt = -INFINITY;
        for (int kk = 0; kk < nj; ++kk) {
          if (!visible(q, j0 + kk, z->left, z->right, z->causal, pos)) row[kk] = masked;
          mt = row[kk] > mt ? row[kk] : mt;
        }
        float lt = 0.0f;
        for (int kk = 0; kk < nj; ++kk) {
          const float p = visible(q, j0 + kk, z->left, z->right, z->causal, pos) ? expf(row[kk] - mt) : 0.0f;
          row[kk] = p;
          lt += p;
        }
        const float mo = mb[q], lo = lb[q];
        const float mn = mo > mt ? mo : mt;
        const float em = expf(mo - mn), emt = expf(mt - mn);
        const float ln = em * lo + emt * lt;
        /* O~ = V_j P~ */
        float* ot = Ot;
        for (int d = 0; d < D; ++d) ot[d] = 0.0f;
        for (int kk = 0; kk < nj; ++kk) {
          const float p = row[kk];
          const float* v = Vb + (long)(j0 + kk) * kp;
          for (int d = 0; d < D; ++d) ot[d] += p * v[d];
        }
        const float denom = ln > FLT_EPSILON ? ln : FLT_EPSILON;
        float* o = Ob + (long)q * qp;
        for (int d = 0; d < D; ++d) o[d] = (o[d] * (lo * em) + ot[d] * emt) / denom;
        mb[q] = mn;
        lb[q] = ln;
      }
    }
  }
}

void fa1_forward(const float* Q, const float* K, const float* V, const int* positions, float* O, float* l, float* m,
                 int D, int H, int Hkv, int T, int B, int left, int right, int causal, int nthreads) {
  dims z = {D, H, Hkv, T, B, left, right, causal};
  const int units = B * H;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    float* S = (float*)malloc(sizeof(float) * BLK * BLK);
    float* Yt = (float*)malloc(sizeof(float) * BLK * (size_t)D);
    float* Ot = (float*)malloc(sizeof(float) * (size_t)D);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int u = 0; u < units; ++u) forward_head(&z, u / H, u % H, Q, K, V, O, l, m, positions, S, Yt, Ot);
    free(S);
    free(Yt);
    free(Ot);
  }
}

static void backward_group(const dims* z, int b, int kv, const float* dO, const float* Q, const float* K,
                           const float* V, const float* O, const float* l, const float* m, const int* positions,
                           float* dQ, float* dK, float* dV, float* S, float* dP, float* Kt, float* Vt, float* Dr) {
  const int D = z->D, T = z->T, H = z->H, Hkv = z->Hkv, G = H / Hkv;
  const long qp = (long)H * D, kp = (long)Hkv * D;
  const float* Kb = K + ((long)b * T * Hkv + kv) * D;
  const float* Vb = V + ((long)b * T * Hkv + kv) * D;
  float* dKb = dK + ((long)b * T * Hkv + kv) * D;
  float* dVb = dV + ((long)b * T * Hkv + kv) * D;
  const int* pos = positions ? positions + (long)b * T : NULL;
  const float scale = 1.0f / sqrtf((float)D);

  for (int h = kv * G; h < (kv + 1) * G; ++h) {
    const float* Qb = Q + ((long)b * T * H + h) * D;
    const float* Ob = O + ((long)b * T * H + h) * D;
    const float* dOb = dO + ((long)b * T * H + h) * D;
    float* dQb = dQ + ((long)b * T * H + h) * D;
    const float* lb = l + ((long)b * H + h) * T;
    const float* mb = m + ((long)b * H + h) * T;
    for (int j0 = 0; j0 < T; j0 += BLK) {
      const int nj = T - j0 < BLK ? T - j0 : BLK;
      transpose_block(Kt, Kb + j0 * kp, kp, nj, D);
      transpose_block(Vt, Vb + j0 * kp, kp, nj, D);
      for (int i0 = 0; i0 < T; i0 += BLK) {
        const int ni = T - i0 < BLK ? T - i0 : BLK;
        scores(S, Qb + i0 * qp, qp, Kt, ni, nj, D, scale);
        scores(dP, dOb + i0 * qp, qp, Vt, ni, nj, D, 1.0f);
        for (int qq = 0; qq < ni; ++qq) {
          const int q = i0 + qq;
          const float lq = lb[q] > FLT_EPSILON ? lb[q] : FLT_EPSILON;
          float dsum = 0.0f;
          for (int d = 0; d < D; ++d) dsum += dOb[(long)q * qp + d] * Ob[(long)q * qp + d];
          Dr[qq] = dsum;
          float* srow = S + (long)qq * nj;
          float* prow = dP + (long)qq * nj;
          for (int kk = 0; kk < nj; ++kk) {
            const int v = visible(q, j0 + kk, z->left, z->right, z->causal, pos);
            const float p = v ? expf(srow[kk] - mb[q]) / lq : 0.0f;
            srow[kk] = p;                      /* P  */
            prow[kk] = p * (prow[kk] - dsum);  /* dS */
          }
        }
        for (int qq = 0; qq < ni; ++qq) {
          const int q = i0 + qq;
          const float* prow = S + (long)qq * nj;
          const float* srow = dP + (long)qq * nj;
          const float* dov = dOb + (long)q * qp;
          const float* qv = Qb + (long)q * qp;
          float* dqv = dQb + (long)q * qp;
          for (int kk = 0; kk < nj; ++kk) {
            const float p = prow[kk], ds = srow[kk];
            float* dvv = dVb + (long)(j0 + kk) * kp;
            float* dkv = dKb + (long)(j0 + kk) * kp;
            const float* kvv = Kb + (long)(j0 + kk) * kp;
            const float sds = scale * ds;
            for (int d = 0; d < D; ++d) {
              dvv[d] += p * dov[d];
              dkv[d] += sds * qv[d];
              dqv[d] += sds * kvv[d];
            }
          }
        }
      }
    }
  }
}

void fa1_backward(const float* dO, const float* Q, const float* K, const float* V, const float* O, const float* l,
                  const float* m, const int* positions, float* dQ, float* dK, float* dV, int D, int H, int Hkv,
                  int T, int B, int left, int right, int causal, int nthreads) {
  dims z = {D, H, Hkv, T, B, left, right, causal};
  const int units = B * Hkv;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    float* S = (float*)malloc(sizeof(float) * BLK * BLK);
    float* dP = (float*)malloc(sizeof(float) * BLK * BLK);
    float* Kt = (float*)malloc(sizeof(float) * BLK * (size_t)D);
    float* Vt = (float*)malloc(sizeof(float) * BLK * (size_t)D);
    float* Dr = (float*)malloc(sizeof(float) * BLK);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int u = 0; u < units; ++u)
      backward_group(&z, u / Hkv, u % Hkv, dO, Q, K, V, O, l, m, positions, dQ, dK, dV, S, dP, Kt, Vt, Dr);
    free(S);
    free(dP);
    free(Kt);
    free(Vt);
    free(Dr);
  }
}
