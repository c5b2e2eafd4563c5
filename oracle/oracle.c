/* oracle.c — CPU restatement of the tagged-op hot path (see oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the timed CPU
 * baseline.  Built with -ffp-contract=off so every a*b+c rounds twice unless
 * the source writes fmaf, exactly where the restated code does.
 *
 * Parity status: the reference's own CPU conv arithmetic lives in the ggml
 * submodule (caojiachen1/ggml, branch ppdl, ~v0.17.0), which is absent, so
 * its SIMD partial-sum order cannot be reproduced: conv results are pinned to
 * tolerance (float64 truth, torch fixtures), not to ggml's bits.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static float act_f(float v, int act) {
    /* ggml_relu: x > 0 ? x : 0; ggml_silu: x / (1 + exp(-x)) */
    if (act == 1) return v > 0.0f ? v : 0.0f;
    if (act == 2) return v / (1.0f + expf(-v));
    return v;
}

static int nthr(int n) {
#ifdef _OPENMP
    return n > 0 ? n : omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Conv: ggml_im2col(F32) + ggml_mul_mat + permute/cont + add + act          */
/* (src/ppdoclayout.cpp:535-542).  The column matrix is stored [k][pixel]    */
/* here (ggml stores [pixel][k]); the values and the k order of each dot     */
/* product are the same.                                                     */
void orc_conv2d_ref(const float *x, int IC, int IH, int IW, const float *w, int OC, int K, int S,
                    int P, const float *bias, int act, float *out, int nthreads) {
    const int OH = (IH + 2 * P - K) / S + 1, OW = (IW + 2 * P - K) / S + 1;
    const int64_t NP = (int64_t)OH * OW, KT = (int64_t)IC * K * K;
    float *col = (float *)malloc((size_t)(KT * NP) * sizeof(float));
    const int nt = nthr(nthreads);

#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t k = 0; k < KT; k++) {
        const int ic = (int)(k / (K * K)), rem = (int)(k % (K * K));
        const int kh = rem / K, kw = rem % K;
        float *c = col + k * NP;
        for (int oy = 0; oy < OH; oy++) {
            const int iy = oy * S + kh - P;
            for (int ox = 0; ox < OW; ox++) {
                const int ix = ox * S + kw - P;
                c[(int64_t)oy * OW + ox] = (iy >= 0 && iy < IH && ix >= 0 && ix < IW)
                                               ? x[((int64_t)ic * IH + iy) * IW + ix]
                                               : 0.0f;
            }
        }
    }

    enum { PB = 256, OB = 8 };
    const int64_t npb = (NP + PB - 1) / PB, nob = (OC + OB - 1) / OB;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 1)
    for (int64_t blk = 0; blk < npb * nob; blk++) {
        const int64_t p0 = (blk % npb) * PB, o0 = (blk / npb) * OB;
        const int np = (int)(NP - p0 < PB ? NP - p0 : PB);
        const int no = (int)(OC - o0 < OB ? OC - o0 : OB);
        float acc[OB][PB];
        memset(acc, 0, sizeof(acc));
        for (int64_t k = 0; k < KT; k++) {
            const float *c = col + k * NP + p0;
            for (int o = 0; o < no; o++) {
                const float wv = w[(o0 + o) * KT + k];
                float *a = acc[o];
                for (int p = 0; p < np; p++) a[p] += wv * c[p];
            }
        }
        for (int o = 0; o < no; o++) {
            const float b = bias ? bias[o0 + o] : 0.0f;
            float *dst = out + (o0 + o) * NP + p0;
            for (int p = 0; p < np; p++) dst[p] = act_f(acc[o][p] + b, act);
        }
    }
    free(col);
}

void orc_conv2d_f64(const float *x, int IC, int IH, int IW, const float *w, int OC, int K, int S,
                    int P, const float *bias, int act, double *out) {
    const int OH = (IH + 2 * P - K) / S + 1, OW = (IW + 2 * P - K) / S + 1;
#pragma omp parallel for schedule(static)
    for (int oc = 0; oc < OC; oc++)
        for (int oy = 0; oy < OH; oy++)
            for (int ox = 0; ox < OW; ox++) {
                double s = 0.0;
                for (int ic = 0; ic < IC; ic++)
                    for (int kh = 0; kh < K; kh++) {
                        const int iy = oy * S + kh - P;
                        if (iy < 0 || iy >= IH) continue;
                        for (int kw = 0; kw < K; kw++) {
                            const int ix = ox * S + kw - P;
                            if (ix < 0 || ix >= IW) continue;
                            s += (double)w[(((int64_t)oc * IC + ic) * K + kh) * K + kw] *
                                 (double)x[((int64_t)ic * IH + iy) * IW + ix];
                        }
                    }
                if (bias) s += (double)bias[oc];
                if (act == 1) s = s > 0.0 ? s : 0.0;
                if (act == 2) s = s / (1.0 + exp(-s));
                out[((int64_t)oc * OH + oy) * OW + ox] = s;
            }
}

void orc_bias_act(const float *in, const float *bias, int64_t n, int64_t plane, int act, float *out) {
    for (int64_t i = 0; i < n; i++) out[i] = act_f(in[i] + bias[i / plane], act);
}

/* ------------------------------------------------------------------------ */
/* Winograd F(4,3) with Toom-Cook points {0, 1, -1, 2, -1/2, inf}:           */
/*   Y = At [ (G g G^T) (.) (Bt d Bt^T) ] At^T                               */
static const float kBt[6][6] = {
    {1.0f, 1.5f, -2.0f, -1.5f, 1.0f, 0.0f},   {0.0f, -1.0f, -2.5f, -0.5f, 1.0f, 0.0f},
    {0.0f, 1.0f, 0.5f, -2.5f, 1.0f, 0.0f},    {0.0f, -0.5f, -1.0f, 0.5f, 1.0f, 0.0f},
    {0.0f, 2.0f, -1.0f, -2.0f, 1.0f, 0.0f},   {0.0f, 1.0f, 1.5f, -2.0f, -1.5f, 1.0f},
};
static const float kAt[4][6] = {
    {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 0.0f},
    {0.0f, 1.0f, -1.0f, 2.0f, -0.5f, 0.0f},
    {0.0f, 1.0f, 1.0f, 4.0f, 0.25f, 0.0f},
    {0.0f, 1.0f, -1.0f, 8.0f, -0.125f, 1.0f},
};
static const double kG[6][3] = {
    {1.0, 0.0, 0.0},
    {-1.0 / 3.0, -1.0 / 3.0, -1.0 / 3.0},
    {1.0 / 3.0, -1.0 / 3.0, 1.0 / 3.0},
    {1.0 / 15.0, 2.0 / 15.0, 4.0 / 15.0},
    {-16.0 / 15.0, 8.0 / 15.0, -4.0 / 15.0},
    {0.0, 0.0, 1.0},
};

void orc_wg4_matrices(double *Bt, double *G, double *At) {
    for (int i = 0; i < 36; i++) Bt[i] = kBt[i / 6][i % 6];
    for (int i = 0; i < 18; i++) G[i] = kG[i / 3][i % 3];
    for (int i = 0; i < 24; i++) At[i] = kAt[i / 6][i % 6];
}

/* repack_convs (src/ppdoclayout.cpp:262-283): wr[kh*K+kw][ic][oc];
 * filter transform (:321-337) with this project's G, float64 accumulation. */
void orc_repack(const float *w, int OC, int IC, int K, float *wr, float *wg4) {
    for (int oc = 0; oc < OC; oc++)
        for (int ic = 0; ic < IC; ic++)
            for (int t = 0; t < K * K; t++)
                wr[((int64_t)t * IC + ic) * OC + oc] = w[((int64_t)oc * IC + ic) * K * K + t];
    if (!wg4 || K != 3) return;
    for (int ic = 0; ic < IC; ic++)
        for (int oc = 0; oc < OC; oc++) {
            const float *g = w + ((int64_t)oc * IC + ic) * 9;
            double gg[6][3];
            for (int u = 0; u < 6; u++)
                for (int b = 0; b < 3; b++) {
                    double s = 0.0;
                    for (int a = 0; a < 3; a++) s += kG[u][a] * (double)g[a * 3 + b];
                    gg[u][b] = s;
                }
            for (int u = 0; u < 6; u++)
                for (int v = 0; v < 6; v++) {
                    double s = 0.0;
                    for (int b = 0; b < 3; b++) s += gg[u][b] * kG[v][b];
                    wg4[((int64_t)(u * 6 + v) * IC + ic) * OC + oc] = (float)s;
                }
        }
}

/* Op 10 (patches/ggml-ppdl.patch:496-547): per (ic, tile) the 6x6 patch at
 * (4ty, 4tx) of the padded frame; d~ = Bt d Bt^T as a fixed fmaf chain over
 * the nonzero entries, ascending index (the HIP kernel runs the same chain). */
void orc_wg4_input(const float *x, int IW, int IH, int IC, int TW, int TH, int pad, float *dt) {
    const int64_t T = (int64_t)TW * TH;
#pragma omp parallel for schedule(static)
    for (int ic = 0; ic < IC; ic++)
        for (int64_t tile = 0; tile < T; tile++) {
            const int ty = (int)(tile / TW), tx = (int)(tile % TW);
            float d[6][6], t1[6][6];
            for (int a = 0; a < 6; a++)
                for (int b = 0; b < 6; b++) {
                    const int iy = 4 * ty - pad + a, ix = 4 * tx - pad + b;
                    d[a][b] = (iy >= 0 && iy < IH && ix >= 0 && ix < IW)
                                  ? x[((int64_t)ic * IH + iy) * IW + ix]
                                  : 0.0f;
                }
            for (int u = 0; u < 6; u++)
                for (int b = 0; b < 6; b++) {
                    float s = 0.0f;
                    for (int a = 0; a < 6; a++)
                        if (kBt[u][a] != 0.0f) s = fmaf(kBt[u][a], d[a][b], s);
                    t1[u][b] = s;
                }
            for (int u = 0; u < 6; u++)
                for (int v = 0; v < 6; v++) {
                    float s = 0.0f;
                    for (int b = 0; b < 6; b++)
                        if (kBt[v][b] != 0.0f) s = fmaf(t1[u][b], kBt[v][b], s);
                    dt[((int64_t)(u * 6 + v) * IC + ic) * T + tile] = s;
                }
        }
}

/* Op 12 (:787-802): yt[p][oc][t] = sum_ic dt[p][ic][t] * wg4[p][ic][oc]. */
void orc_wg4_madd(const float *dt, const float *wg4, int T, int IC, int OC, float *yt, int nthreads) {
    const int nt = nthr(nthreads);
#pragma omp parallel for num_threads(nt) schedule(static) collapse(2)
    for (int p = 0; p < 36; p++)
        for (int oc = 0; oc < OC; oc++) {
            float *y = yt + ((int64_t)p * OC + oc) * T;
            for (int t = 0; t < T; t++) y[t] = 0.0f;
            for (int ic = 0; ic < IC; ic++) {
                const float wv = wg4[((int64_t)p * IC + ic) * OC + oc];
                const float *d = dt + ((int64_t)p * IC + ic) * T;
                for (int t = 0; t < T; t++) y[t] += d[t] * wv;
            }
        }
}

/* Op 11 (:549-610): Y = At m At^T + bias, act, bounds-checked CHW store. */
void orc_wg4_output(const float *yt, const float *bias, int TW, int TH, int OC, int OW, int OH,
                    int act, float *out) {
    const int64_t T = (int64_t)TW * TH;
#pragma omp parallel for schedule(static)
    for (int oc = 0; oc < OC; oc++)
        for (int64_t tile = 0; tile < T; tile++) {
            const int ty = (int)(tile / TW), tx = (int)(tile % TW);
            float m[6][6], t1[4][6];
            for (int p = 0; p < 36; p++) m[p / 6][p % 6] = yt[((int64_t)p * OC + oc) * T + tile];
            for (int i = 0; i < 4; i++)
                for (int v = 0; v < 6; v++) {
                    float s = 0.0f;
                    for (int u = 0; u < 6; u++)
                        if (kAt[i][u] != 0.0f) s = fmaf(kAt[i][u], m[u][v], s);
                    t1[i][v] = s;
                }
            for (int i = 0; i < 4; i++) {
                const int py = 4 * ty + i;
                for (int j = 0; j < 4; j++) {
                    const int px = 4 * tx + j;
                    float s = 0.0f;
                    for (int v = 0; v < 6; v++)
                        if (kAt[j][v] != 0.0f) s = fmaf(t1[i][v], kAt[j][v], s);
                    if (py < OH && px < OW)
                        out[((int64_t)oc * OH + py) * OW + px] = act_f(s + bias[oc], act);
                }
            }
        }
}

/* ------------------------------------------------------------------------ */
void orc_im2col(const float *x, int64_t IW, int64_t IH, int64_t OW, int64_t OH, int64_t KW,
                int64_t KH, int64_t IC, int64_t N, int64_t ch_stride, int64_t img_stride, int s0,
                int s1, int p0, int p1, int d0, int d1, float *dst) {
    const int64_t KT = IC * KH * KW;
    for (int64_t n = 0; n < N; n++)
        for (int64_t oh = 0; oh < OH; oh++)
            for (int64_t ow = 0; ow < OW; ow++) {
                const int64_t pix = (n * OH + oh) * OW + ow;
                for (int64_t ic = 0; ic < IC; ic++)
                    for (int64_t kh = 0; kh < KH; kh++)
                        for (int64_t kw = 0; kw < KW; kw++) {
                            const int64_t iy = oh * s1 + kh * d1 - p1, ix = ow * s0 + kw * d0 - p0;
                            const int64_t k = (ic * KH + kh) * KW + kw;
                            dst[pix * KT + k] = (iy >= 0 && iy < IH && ix >= 0 && ix < IW)
                                                    ? x[ic * ch_stride + n * img_stride + iy * IW + ix]
                                                    : 0.0f;
                        }
            }
}

/* ------------------------------------------------------------------------ */
/* op_msdeform (src/ppdoclayout.cpp:148-198): per query and head, softmax over */
/* the 12 (level, point) logits, then grid_sample-style bilinear sampling with */
/* zero padding (align_corners = false), accumulated level -> point -> corner */
/* with one fused multiply-add per tap (the accumulation contract of          */
/* patches/ggml-ppdl.patch:112-115).  The clamp of fx/fy only keeps the       */
/* float->int conversion defined; it never changes which corners are read.   */
static const int kLvlW[3] = {100, 50, 25};
static const int kLvlStart[3] = {0, 10000, 12500};

void orc_msdeform(const float *val, const float *off, const float *awr, const float *ref, int nq,
                  float *out, int nthreads) {
    const int nt = nthr(nthreads);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int q = 0; q < nq; q++) {
        const float *rq = ref + (int64_t)q * 4;
        float *oq = out + (int64_t)q * 256;
        for (int h = 0; h < 8; h++) {
            const float *a = awr + (int64_t)q * 96 + h * 12;
            float amax = a[0], w[12], wsum = 0.0f;
            for (int i = 1; i < 12; i++) amax = amax < a[i] ? a[i] : amax;
            for (int i = 0; i < 12; i++) {
                w[i] = expf(a[i] - amax);
                wsum += w[i];
            }
            for (int i = 0; i < 12; i++) w[i] /= wsum;
            float acc[32];
            for (int c = 0; c < 32; c++) acc[c] = 0.0f;
            for (int l = 0; l < 3; l++) {
                const int W = kLvlW[l], H = kLvlW[l], st = kLvlStart[l];
                for (int p = 0; p < 4; p++) {
                    const float ox = off[(int64_t)q * 192 + ((h * 3 + l) * 4 + p) * 2 + 0];
                    const float oy = off[(int64_t)q * 192 + ((h * 3 + l) * 4 + p) * 2 + 1];
                    const float lx = rq[0] + ox / 4.0f * rq[2] * 0.5f;
                    const float ly = rq[1] + oy / 4.0f * rq[3] * 0.5f;
                    float fx = lx * (float)W - 0.5f, fy = ly * (float)H - 0.5f;
                    fx = fminf(fmaxf(fx, -2.0f), (float)W + 1.0f);
                    fy = fminf(fmaxf(fy, -2.0f), (float)H + 1.0f);
                    const int x0 = (int)floorf(fx), y0 = (int)floorf(fy);
                    const float tx = fx - (float)x0, ty = fy - (float)y0;
                    const float wt = w[l * 4 + p];
                    const float cw[4] = {(1 - tx) * (1 - ty), tx * (1 - ty), (1 - tx) * ty, tx * ty};
                    const int xs[4] = {x0, x0 + 1, x0, x0 + 1};
                    const int ys[4] = {y0, y0, y0 + 1, y0 + 1};
                    for (int k = 0; k < 4; k++) {
                        const int xx = xs[k], yy = ys[k];
                        if (xx < 0 || xx >= W || yy < 0 || yy >= H || cw[k] == 0.0f) continue;
                        const float *v = val + (int64_t)(st + yy * W + xx) * 256 + h * 32;
                        const float ww = wt * cw[k];
                        for (int c = 0; c < 32; c++) acc[c] = fmaf(ww, v[c], acc[c]);
                    }
                }
            }
            for (int c = 0; c < 32; c++) oq[h * 32 + c] = acc[c];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* op_mask_box (src/ppdoclayout.cpp:100-140). */
static float invsig(float x) {
    x = fminf(fmaxf(x, 0.0f), 1.0f);
    const float x1 = fmaxf(x, 1e-5f), x2 = fmaxf(1.0f - x, 1e-5f);
    return logf(x1 / x2);
}

void orc_mask_box(const float *ml, int nq, float *out) {
    for (int q = 0; q < nq; q++) {
        const float *m = ml + (int64_t)q * 40000;
        int xmin = 200, xmax = -1, ymin = 200, ymax = -1;
        for (int y = 0; y < 200; y++)
            for (int x = 0; x < 200; x++)
                if (m[y * 200 + x] > 0.0f) {
                    if (x < xmin) xmin = x;
                    if (x > xmax) xmax = x;
                    if (y < ymin) ymin = y;
                    if (y > ymax) ymax = y;
                }
        float bx0, by0, bx1, by1;
        if (xmax < 0) {
            bx0 = by0 = bx1 = by1 = 0.0f;
        } else {
            bx0 = (float)xmin;
            by0 = (float)ymin;
            bx1 = (float)xmax + 1.0f;
            by1 = (float)ymax + 1.0f;
        }
        bx0 /= 200.0f;
        bx1 /= 200.0f;
        by0 /= 200.0f;
        by1 /= 200.0f;
        const float cx = (bx0 + bx1) * 0.5f, cy = (by0 + by1) * 0.5f;
        const float bw = bx1 - bx0, bh = by1 - by0;
        out[q * 4 + 0] = invsig(cx);
        out[q * 4 + 1] = invsig(cy);
        out[q * 4 + 2] = invsig(bw);
        out[q * 4 + 3] = invsig(bh);
    }
}

/* ------------------------------------------------------------------------ */
/* op_topk300 (src/ppdoclayout.cpp:75-96): order by max-class logit            */
/* descending, ties by index ascending.                                       */
typedef struct {
    float m;
    int idx;
} tk_item;

static int tk_cmp(const void *pa, const void *pb) {
    const tk_item *a = (const tk_item *)pa, *b = (const tk_item *)pb;
    if (a->m != b->m) return a->m > b->m ? -1 : 1;
    return a->idx < b->idx ? -1 : (a->idx > b->idx);
}

void orc_topk(const float *logits, int ntok, int nc, int nq, int32_t *out) {
    tk_item *it = (tk_item *)malloc((size_t)ntok * sizeof(tk_item));
    for (int t = 0; t < ntok; t++) {
        const float *p = logits + (int64_t)t * nc;
        float m = p[0];
        for (int c = 1; c < nc; c++) m = m < p[c] ? p[c] : m;
        it[t].m = m;
        it[t].idx = t;
    }
    qsort(it, (size_t)ntok, sizeof(tk_item), tk_cmp);
    for (int i = 0; i < nq; i++) out[i] = it[i].idx;
    free(it);
}
