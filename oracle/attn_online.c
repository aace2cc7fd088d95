/*
 * Plain-C fp64 restatement of the reference's tiled online-softmax attention.
 *
 * TEST INFRASTRUCTURE ONLY: built into oracle/build/libattn_oracle.so and called from
 * tests/ (and nowhere in the product path).
 *
 * Forward follows /root/reference/cuda_transformer/flash_attention.cu:57-169 loop by
 * loop: per query row, walk the keys in tiles of `tile` columns (BLOCKDIM = 32 in the
 * reference, ModuleLayer.cu:6); per tile take the row max of the scores
 * (flash_attention.cu:120-128), rescale the running denominator and weighted sum by
 * exp(m_old - m_new) (:130-131, :141-151), add exp(s - m_new) (:132-141), and at the end
 * divide (:161).  Scores are Q.K / sqrt(d), a division as at :116.
 *
 * Backward follows flash_attention.cu:226-326: per query row recompute
 * P = exp(S - m) / l (:297-298; here exp(S - LSE) with LSE = m + ln l),
 * delta = O.dO (:269-273), dS = P (dP - delta) / sqrt(d) (:299), dQ += dS K (:311).
 * dK and dV use the gradient of the forward, dK_j += dS_ij Q_i and dV_j += P_ij dO_i,
 * not the reference's defective :312-313.
 *
 * Departures, matching oracle/attention_fp64.py: causal masks j > i; keys j >= T do not
 * exist (the reference zero-pads them into the softmax, :104-117); LSE replaces (m, l).
 *
 * Layout: [BH, T, d] row-major per tensor, lse [BH, T].
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int64_t key_limit(int64_t row, int64_t T, int causal)
{
    return causal ? (row + 1 < T ? row + 1 : T) : T;
}

int attn_online_fwd(const double *q, const double *k, const double *v, double *o,
                    double *lse, int64_t BH, int64_t T, int64_t d, int causal, int64_t tile)
{
    if (BH < 0 || T < 0 || d <= 0 || tile <= 0) return 1;
    const double sqrt_d = sqrt((double)d);
    double *acc = (double *)malloc(sizeof(double) * (size_t)d);
    double *s = (double *)malloc(sizeof(double) * (size_t)tile);
    if (!acc || !s) { free(acc); free(s); return 2; }
    for (int64_t bh = 0; bh < BH; ++bh) {
        const double *Q = q + bh * T * d, *K = k + bh * T * d, *V = v + bh * T * d;
        for (int64_t i = 0; i < T; ++i) {
            const int64_t nkeys = key_limit(i, T, causal);
            double m = -INFINITY, l = 0.0;
            memset(acc, 0, sizeof(double) * (size_t)d);
            for (int64_t j0 = 0; j0 < nkeys; j0 += tile) {
                const int64_t jn = (j0 + tile < nkeys ? j0 + tile : nkeys) - j0;
                double tmax = -INFINITY;
                for (int64_t jj = 0; jj < jn; ++jj) {
                    double dot = 0.0;
                    for (int64_t c = 0; c < d; ++c) dot += Q[i * d + c] * K[(j0 + jj) * d + c];
                    s[jj] = dot / sqrt_d;
                    if (s[jj] > tmax) tmax = s[jj];
                }
                const double mnew = tmax > m ? tmax : m;
                const double rescale = (m == -INFINITY) ? 0.0 : exp(m - mnew);
                double psum = 0.0;
                for (int64_t c = 0; c < d; ++c) acc[c] *= rescale;
                for (int64_t jj = 0; jj < jn; ++jj) {
                    const double p = exp(s[jj] - mnew);
                    psum += p;
                    for (int64_t c = 0; c < d; ++c) acc[c] += p * V[(j0 + jj) * d + c];
                }
                l = l * rescale + psum;
                m = mnew;
            }
            for (int64_t c = 0; c < d; ++c) o[bh * T * d + i * d + c] = acc[c] / l;
            lse[bh * T + i] = m + log(l);
        }
    }
    free(acc);
    free(s);
    return 0;
}

int attn_online_bwd(const double *q, const double *k, const double *v, const double *o,
                    const double *dout, const double *lse, double *dq, double *dk,
                    double *dv, int64_t BH, int64_t T, int64_t d, int causal)
{
    if (BH < 0 || T < 0 || d <= 0) return 1;
    const double sqrt_d = sqrt((double)d);
    memset(dq, 0, sizeof(double) * (size_t)(BH * T * d));
    memset(dk, 0, sizeof(double) * (size_t)(BH * T * d));
    memset(dv, 0, sizeof(double) * (size_t)(BH * T * d));
    for (int64_t bh = 0; bh < BH; ++bh) {
        const int64_t off = bh * T * d;
        const double *Q = q + off, *K = k + off, *V = v + off, *O = o + off, *dO = dout + off;
        double *dQ = dq + off, *dK = dk + off, *dV = dv + off;
        for (int64_t i = 0; i < T; ++i) {
            double delta = 0.0;
            for (int64_t c = 0; c < d; ++c) delta += O[i * d + c] * dO[i * d + c];
            const int64_t nkeys = key_limit(i, T, causal);
            for (int64_t j = 0; j < nkeys; ++j) {
                double sdot = 0.0, pdot = 0.0;
                for (int64_t c = 0; c < d; ++c) {
                    sdot += Q[i * d + c] * K[j * d + c];
                    pdot += dO[i * d + c] * V[j * d + c];
                }
                const double p = exp(sdot / sqrt_d - lse[bh * T + i]);
                const double ds = p * (pdot - delta) / sqrt_d;
                for (int64_t c = 0; c < d; ++c) {
                    dQ[i * d + c] += ds * K[j * d + c];
                    dK[j * d + c] += ds * Q[i * d + c];
                    dV[j * d + c] += p * dO[i * d + c];
                }
            }
        }
    }
    return 0;
}
