/* oracle.h — CPU restatement of PP-DocLayoutV3's tagged-op hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP kernels are
 * compared against (tests/, __graft_entry__.smoke()) and the timed CPU
 * baseline of bench.py.  It is never linked into, loaded by or called from the
 * product library, and the product never falls back to it.
 *
 * Layouts follow the reference (ggml ne order, fastest axis first):
 * images are CHW, conv weights OIHW, token tensors token-major.
 *
 * Pinning (what checks each function beyond restating it) is listed per
 * function; the tests under tests/ carry those checks.
 */
#ifndef PPDL_ORACLE_H
#define PPDL_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reference CPU conv path: F32 im2col (k = ic*K*K + kh*K + kw) + FP32 dot
 * product in k order + bias + act (src/ppdoclayout.cpp:535-542, act per
 * :379-385).  out: OC x OH x OW.  Pinned by: float64 direct conv, torch
 * conv2d fixtures, delta-kernel / identity / zero-input invariants. */
void orc_conv2d_ref(const float *x, int IC, int IH, int IW, const float *w, int OC, int K, int S,
                    int P, const float *bias, int act, float *out, int nthreads);

/* Float64 direct 2-D cross-correlation + bias + act: the closed-form truth. */
void orc_conv2d_f64(const float *x, int IC, int IH, int IW, const float *w, int OC, int K, int S,
                    int P, const float *bias, int act, double *out);

/* Op 5: out[i] = act(in[i] + bias[i / plane]) (patches/ggml-ppdl.patch:417-432). */
void orc_bias_act(const float *in, const float *bias, int64_t n, int64_t plane, int act, float *out);

/* Weight repack (src/ppdoclayout.cpp:262-283 for wr; :321-337 for the
 * 36-plane filter transform, here with this project's G and float64
 * accumulation).  wg4 may be NULL. */
void orc_repack(const float *w, int OC, int IC, int K, float *wr, float *wg4);

/* F(4,3) matrices (float64, row-major Bt 6x6, G 6x3, At 4x6), derived from
 * Toom-Cook points {0, 1, -1, 2, -1/2, inf}. */
void orc_wg4_matrices(double *Bt, double *G, double *At);

/* Op 10 / 15 input transform (patches/ggml-ppdl.patch:496-547): pad = 0 reads
 * a pre-padded image, pad = 1 applies the conv's zero pad of 1. */
void orc_wg4_input(const float *x, int IW, int IH, int IC, int TW, int TH, int pad, float *dt);

/* Op 12: 36 independent FP32 GEMMs, k (= ic) order (:787-802). */
void orc_wg4_madd(const float *dt, const float *wg4, int T, int IC, int OC, float *yt, int nthreads);

/* Op 11 output transform + bias + act, cropped CHW store (:549-610). */
void orc_wg4_output(const float *yt, const float *bias, int TW, int TH, int OC, int OW, int OH,
                    int act, float *out);

/* ggml F32 im2col layout: dst[pix][k] (:845-883); ch_stride / img_stride as
 * in include/ppdl_hip_ops.h. */
void orc_im2col(const float *x, int64_t IW, int64_t IH, int64_t OW, int64_t OH, int64_t KW,
                int64_t KH, int64_t IC, int64_t N, int64_t ch_stride, int64_t img_stride, int s0,
                int s1, int p0, int p1, int d0, int d1, float *dst);

/* Op 2, MSDeformAttn sampling (src/ppdoclayout.cpp:148-198).  Pinned by:
 * per-level grid_sample fixtures, all-out-of-bounds -> 0, equal logits ->
 * weight 1/12, texel-centre sampling -> exact value copy. */
void orc_msdeform(const float *val, const float *off, const float *awr, const float *ref, int nq,
                  float *out, int nthreads);

/* Op 1, mask -> inverse-sigmoid box (src/ppdoclayout.cpp:100-140). */
void orc_mask_box(const float *ml, int nq, float *out);

/* Op 13, top-nq token indices by max-class logit, ties to the lower index
 * (src/ppdoclayout.cpp:75-96). */
void orc_topk(const float *logits, int ntok, int nc, int nq, int32_t *out);

#ifdef __cplusplus
}
#endif

#endif
