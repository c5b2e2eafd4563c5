// C-ABI dispatcher of the tagged-op library (include/ppdl_hip_ops.h).
//
// Plays the role of ggml_cuda_compute_forward_ppdl / ggml_cuda_supports_ppdl_op
// (patches/ggml-ppdl.patch:612-817, :908-917): reads the op id from
// op_params[13], checks the node's views against the op's contract on the
// host, then enqueues the kernels on the caller's stream.  Nothing is
// enqueued when validation fails, so a PPDL_EINVAL leaves the stream as it was.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/ppdl_hip_ops.h"
#include "ppdl_internal.h"

using namespace ppdl;

namespace {

bool contig_f32(const ppdl_tview *t) {
    if (!t || !t->data || t->type != PPDL_TYPE_F32) return false;
    if (t->nb[0] != 4) return false;
    for (int i = 0; i < 4; i++)
        if (t->ne[i] < 1) return false;
    for (int i = 1; i < 4; i++)
        if (t->nb[i] != t->nb[i - 1] * t->ne[i - 1]) return false;
    return true;
}

// F32 CHW map ne(W, H, C, 1) with packed rows and planes at any stride
// nb[2] >= 4*W*H (a multiple of 4 bytes): a contiguous map or a view whose
// channel planes are padded
bool chw_f32(const ppdl_tview *t) {
    if (!t || !t->data || t->type != PPDL_TYPE_F32 || t->nb[0] != 4) return false;
    for (int i = 0; i < 4; i++)
        if (t->ne[i] < 1) return false;
    if (t->ne[3] != 1 || t->nb[1] != 4 * t->ne[0] || t->nb[2] < t->nb[1] * t->ne[1] || t->nb[2] % 4 != 0) return false;
    return (t->nb[2] / 4) * t->ne[2] <= ((int64_t)1 << 40);
}

bool contig_i32(const ppdl_tview *t) {
    if (!t || !t->data || t->type != PPDL_TYPE_I32 || t->nb[0] != 4) return false;
    for (int i = 0; i < 4; i++)
        if (t->ne[i] < 1) return false;
    for (int i = 1; i < 4; i++)
        if (t->nb[i] != t->nb[i - 1] * t->ne[i - 1]) return false;
    return true;
}

bool shape_is(const ppdl_tview *t, int64_t a, int64_t b, int64_t c, int64_t d) {
    return t->ne[0] == a && t->ne[1] == b && t->ne[2] == c && t->ne[3] == d;
}

int64_t nelem(const ppdl_tview *t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

bool aligned16(const void *p) { return (((uintptr_t)p) & 15) == 0; }

int status_of(hipError_t e) { return e == hipSuccess ? PPDL_OK : PPDL_ELAUNCH; }

constexpr int64_t kMaxI32 = 0x7fffffff;

// Index of the optional split-K workspace src of a GEMM op, or -1.  Op 14
// with a fused add (params[15] != 0) carries the add operand at src[3].
int ws_index(const int32_t *p) {
    switch (p[13]) {
        case PPDL_OP_CONV:
        case PPDL_OP_CONV_IM2COL: return 3;
        case PPDL_OP_CONV1X1_BA: return p[15] ? 4 : 3;
        case PPDL_OP_WG4_MADD: return 2;
        case PPDL_OP_TOPK: return 1;
        default: return -1;
    }
}

// F32 rows: unit element stride, any row stride >= the row (a multiple of 4
// bytes, below 2^31 elements), a single plane
bool rows_f32(const ppdl_tview *t) {
    if (!t || !t->data || t->type != PPDL_TYPE_F32 || t->nb[0] != 4) return false;
    for (int i = 0; i < 4; i++)
        if (t->ne[i] < 1) return false;
    if (t->nb[1] < t->ne[0] * 4 || t->nb[1] % 4 != 0 || t->nb[1] / 4 > kMaxI32) return false;
    return t->ne[2] == 1 && t->ne[3] == 1;
}

// F32 Winograd planes ne(T, C, 36, 1): rows of T tiles with a row stride
// nb[1] >= 4T (a multiple of 4 bytes), planes packed after the C rows
bool planes_f32(const ppdl_tview *t, int64_t T, int64_t C) {
    if (!t || !t->data || t->type != PPDL_TYPE_F32 || t->nb[0] != 4) return false;
    if (t->ne[0] != T || t->ne[1] != C || t->ne[2] != 36 || t->ne[3] != 1) return false;
    if (t->nb[1] < T * 4 || t->nb[1] % 4 != 0 || t->nb[2] != t->nb[1] * C || t->nb[3] != t->nb[2] * 36) return false;
    return t->nb[3] / 4 <= kMaxI32;
}

bool ws_valid(const ppdl_tview *t) {
    if (!t->data || (t->type != PPDL_TYPE_F32 && t->type != PPDL_TYPE_I32) || t->nb[0] != 4) return false;
    for (int i = 1; i < 4; i++)
        if (t->ne[i] < 1 || t->nb[i] != t->nb[i - 1] * t->ne[i - 1]) return false;
    return t->ne[0] >= 1 && aligned16(t->data);
}

GemmWorkspace ws_of(const int32_t *p, const ppdl_tview *src, int nsrc) {
    const int i = ws_index(p);
    if (i < 0 || nsrc <= i) return GemmWorkspace{nullptr, 0};
    return GemmWorkspace{src[i].data, nelem(&src[i]) * 4};
}

// ---- per-op validation (shared by supports() and run()) ----
// Returns PPDL_OK when the node satisfies the op's contract, PPDL_EINVAL when
// it does not, PPDL_UNSUPPORTED for an op id this library does not execute.

int check_conv1x1(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, int nsrc,
                  bool fused) {
    if (nsrc < (fused ? 3 : 2)) return PPDL_EINVAL;
    const ppdl_tview *x = &src[0], *w = &src[1];
    // x and dst: CHW maps whose channel planes may be padded (nb[2] >= 4*W*H)
    if (!chw_f32(dst) || !chw_f32(x) || !contig_f32(w)) return PPDL_EINVAL;
    const int64_t W = x->ne[0], H = x->ne[1], IC = x->ne[2], OC = dst->ne[2];
    if (!shape_is(dst, W, H, OC, 1) || !shape_is(w, OC, IC, 1, 1)) return PPDL_EINVAL;
    if (W * H > kMaxI32 || IC > kMaxI32 || OC > kMaxI32) return PPDL_EINVAL;
    // the GEMM indexes planes with 32-bit element offsets
    if ((x->nb[2] / 4) * IC > kMaxI32 || (dst->nb[2] / 4) * OC > kMaxI32) return PPDL_EINVAL;
    if (fused) {
        if (!contig_f32(&src[2]) || nelem(&src[2]) != OC) return PPDL_EINVAL;
        if (p[14] < 0 || p[14] > 2 || p[15] < 0 || p[15] > 2) return PPDL_EINVAL;
        // the added map is laid out as dst
        if (p[15] && (nsrc < 4 || !chw_f32(&src[3]) || !shape_is(&src[3], W, H, OC, 1) || src[3].nb[2] != dst->nb[2]))
            return PPDL_EINVAL;
    }
    return PPDL_OK;
}

int check_op(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, int nsrc) {
    switch (p[13]) {
        case PPDL_OP_WG4_INPUT: case PPDL_OP_WG4_OUTPUT: case PPDL_OP_WG4_MADD: case PPDL_OP_WG4_INPUT_PAD:
        case PPDL_OP_WG4_CONV:
            // .wg4 made with another F(4,3) matrix set would pass every shape check
            if ((uint32_t)p[11] != (uint32_t)PPDL_WG4_SET) return PPDL_EINVAL;
            break;
        default:
            break;
    }
    const int wi = ws_index(p);
    if (wi >= 0 && nsrc > wi && !ws_valid(&src[wi])) return PPDL_EINVAL;
    switch (p[13]) {
        case PPDL_OP_CONV: {
            const int K = p[14] & 0xFF, pad = (p[14] >> 8) & 0xFF;
            if (K != 1) return PPDL_UNSUPPORTED;  // legacy k3 tap-GEMM path is not carried
            if (pad != 0 || p[15] != 0) return PPDL_EINVAL;
            return check_conv1x1(p, dst, src, nsrc, false);
        }
        case PPDL_OP_CONV1X1_BA:
            return check_conv1x1(p, dst, src, nsrc, true);
        case PPDL_OP_BIASACT: {
            if (nsrc < 2 || !contig_f32(dst) || !contig_f32(&src[0]) || !contig_f32(&src[1]))
                return PPDL_EINVAL;
            for (int i = 0; i < 4; i++)
                if (src[0].ne[i] != dst->ne[i]) return PPDL_EINVAL;
            if (nelem(&src[1]) < dst->ne[2] * dst->ne[3]) return PPDL_EINVAL;
            if (p[14] < 0 || p[14] > 2) return PPDL_EINVAL;
            return PPDL_OK;
        }
        case PPDL_OP_WG4_INPUT:
        case PPDL_OP_WG4_INPUT_PAD: {
            if (nsrc < 1 || !contig_f32(&src[0])) return PPDL_EINVAL;
            const ppdl_tview *x = &src[0];
            const int64_t T = p[14], TH = p[15];
            if (T < 1 || TH < 1 || T % TH != 0) return PPDL_EINVAL;
            const int64_t TW = T / TH, IC = x->ne[2];
            if (x->ne[3] != 1 || !planes_f32(dst, T, IC)) return PPDL_EINVAL;
            if (T * IC > kMaxI32) return PPDL_EINVAL;
            if (p[13] == PPDL_OP_WG4_INPUT) {
                // the padded frame must hold every 6x6 patch
                if (4 * TW + 2 > x->ne[0] || 4 * TH + 2 > x->ne[1]) return PPDL_EINVAL;
            } else {
                if (TW != (x->ne[0] + 3) / 4 || TH != (x->ne[1] + 3) / 4) return PPDL_EINVAL;
            }
            return PPDL_OK;
        }
        case PPDL_OP_WG4_MADD: {
            if (nsrc < 2 || !contig_f32(&src[1])) return PPDL_EINVAL;
            const int64_t T = src[0].ne[0], IC = src[0].ne[1], OC = src[1].ne[0];
            if (!planes_f32(&src[0], T, IC) || !shape_is(&src[1], OC, IC, 36, 1) || !planes_f32(dst, T, OC))
                return PPDL_EINVAL;
            if (T > kMaxI32 || IC > kMaxI32 || OC > kMaxI32) return PPDL_EINVAL;
            return PPDL_OK;
        }
        case PPDL_OP_WG4_OUTPUT: {
            if (nsrc < 2 || !contig_f32(dst) || !contig_f32(&src[1])) return PPDL_EINVAL;
            const int64_t OW = dst->ne[0], OH = dst->ne[1], OC = dst->ne[2];
            const int64_t TW = (OW + 3) / 4, TH = (OH + 3) / 4;
            if (dst->ne[3] != 1 || !planes_f32(&src[0], TW * TH, OC)) return PPDL_EINVAL;
            if (p[15] != TW || nelem(&src[1]) != OC || p[14] < 0 || p[14] > 2) return PPDL_EINVAL;
            // optional third source: a map of dst's shape added after the activation
            if (nsrc >= 3 && (!contig_f32(&src[2]) || src[2].ne[0] != OW || src[2].ne[1] != OH ||
                              src[2].ne[2] != OC || src[2].ne[3] != 1))
                return PPDL_EINVAL;
            return PPDL_OK;
        }
        case PPDL_OP_CONV_IM2COL: {
            if (nsrc < 3) return PPDL_EINVAL;
            const ppdl_tview *x = &src[0], *w = &src[1], *b = &src[2];
            if (!contig_f32(dst) || !contig_f32(x) || !contig_f32(w) || !contig_f32(b)) return PPDL_EINVAL;
            const int K = p[14] & 0xFF, S = (p[14] >> 8) & 0xFF, P = (p[14] >> 16) & 0xFF;
            const int act = (p[14] >> 24) & 0xFF, PE = p[15];
            if (K < 1 || S < 1 || act > 2 || PE < 0 || PE > 255) return PPDL_EINVAL;
            const int64_t IW = x->ne[0], IH = x->ne[1], IC = x->ne[2], OC = dst->ne[2];
            if (IW + 2 * P + PE < K || IH + 2 * P + PE < K) return PPDL_EINVAL;
            const int64_t OW = (IW + 2 * P + PE - K) / S + 1, OH = (IH + 2 * P + PE - K) / S + 1;
            if (x->ne[3] != 1 || !shape_is(dst, OW, OH, OC, 1) || !shape_is(w, OC, IC, (int64_t)K * K, 1) ||
                nelem(b) != OC)
                return PPDL_EINVAL;
            if (OW * OH > kMaxI32 || IC * K * K > kMaxI32 || IH * IW > kMaxI32) return PPDL_EINVAL;
            return PPDL_OK;
        }
        case PPDL_OP_WG4_CONV: {
            if (nsrc < 3) return PPDL_EINVAL;
            const ppdl_tview *x = &src[0], *w = &src[1], *b = &src[2];
            if (!contig_f32(dst) || !contig_f32(x) || !contig_f32(w) || !contig_f32(b)) return PPDL_EINVAL;
            const int64_t W = x->ne[0], H = x->ne[1], IC = x->ne[2], OC = dst->ne[2];
            if (x->ne[3] != 1 || !shape_is(dst, W, H, OC, 1) || !shape_is(w, OC, IC, 36, 1) || nelem(b) != OC)
                return PPDL_EINVAL;
            if (p[14] < 0 || p[14] > 2 || p[15] != 0) return PPDL_EINVAL;
            const int64_t T = ((W + 3) / 4) * ((H + 3) / 4);
            if (W * H * IC > kMaxI32 || 36 * IC * OC > kMaxI32 || T * ((OC + 15) / 16) > kMaxI32) return PPDL_EINVAL;
            return PPDL_OK;
        }
        case PPDL_OP_MSDEF: {
            if (nsrc < 4 || !contig_f32(dst)) return PPDL_EINVAL;
            // value, offsets and weights may be row-strided views (slices of
            // wider projections)
            for (int i = 0; i < 3; i++)
                if (!rows_f32(&src[i])) return PPDL_EINVAL;
            if (!contig_f32(&src[3])) return PPDL_EINVAL;
            const int64_t NQ = dst->ne[1];
            if (!shape_is(dst, kDM, NQ, 1, 1) || !shape_is(&src[0], kDM, kNTOK, 1, 1) ||
                !shape_is(&src[1], kNH * kNLVL * kNPTS * 2, NQ, 1, 1) ||
                !shape_is(&src[2], kNH * kNLVL * kNPTS, NQ, 1, 1) || !shape_is(&src[3], 4, NQ, 1, 1))
                return PPDL_EINVAL;
            if (NQ > 65535) return PPDL_EINVAL;
            return PPDL_OK;
        }
        case PPDL_OP_MASKBOX: {
            if (nsrc < 1 || !contig_f32(dst) || !contig_f32(&src[0])) return PPDL_EINVAL;
            const int64_t NQ = dst->ne[1];
            if (!shape_is(dst, 4, NQ, 1, 1) || !shape_is(&src[0], kMaskPix, NQ, 1, 1)) return PPDL_EINVAL;
            if (!aligned16(src[0].data) || NQ > 65535) return PPDL_EINVAL;
            return PPDL_OK;
        }
        case PPDL_OP_TOPK: {
            if (nsrc < 1 || !contig_i32(dst) || !contig_f32(&src[0])) return PPDL_EINVAL;
            const int64_t NC = src[0].ne[0], NT = src[0].ne[1], NQ = dst->ne[0];
            if (src[0].ne[2] != 1 || src[0].ne[3] != 1 || !shape_is(dst, NQ, 1, 1, 1)) return PPDL_EINVAL;
            if (NT > 13312 || NQ > 512 || NQ > NT || NC > 4096) return PPDL_EINVAL;
            return PPDL_OK;
        }
        default:
            return PPDL_UNSUPPORTED;
    }
}

// GEMM description of a validated conv/madd node.  Returns false for ops that
// are not GEMMs.  *im2col selects the implicit-im2col B operand.
bool args_of_node(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, GemmArgs *g, bool *im2col) {
    *g = GemmArgs{};
    *im2col = false;
    switch (p[13]) {
        case PPDL_OP_CONV:
        case PPDL_OP_CONV1X1_BA: {
            const ppdl_tview *x = &src[0], *w = &src[1];
            const bool fused = p[13] == PPDL_OP_CONV1X1_BA;
            g->A = (const float *)w->data;
            g->lda = dst->ne[2];
            g->B = (const float *)x->data;
            g->ldb = x->nb[2] / 4;  // channel-plane strides (packed: W*H)
            g->C = (float *)dst->data;
            g->ldc = dst->nb[2] / 4;
            g->bias = fused ? (const float *)src[2].data : nullptr;
            g->M = (int)dst->ne[2];
            g->N = (int)(x->ne[0] * x->ne[1]);
            g->K = (int)x->ne[2];
            g->batch = 1;
            g->act = fused ? p[14] : 0;
            if (fused && p[15]) {
                g->add_mode = p[15];
                g->add = (const float *)src[3].data;
            }
            return true;
        }
        case PPDL_OP_WG4_MADD: {
            const int64_t T = src[0].ne[0], IC = src[0].ne[1], OC = src[1].ne[0];
            g->A = (const float *)src[1].data;
            g->lda = OC;
            g->sA = IC * OC;
            g->B = (const float *)src[0].data;
            g->ldb = src[0].nb[1] / 4;
            g->sB = IC * g->ldb;
            g->C = (float *)dst->data;
            g->ldc = dst->nb[1] / 4;
            g->sC = OC * g->ldc;
            g->M = (int)OC;
            g->N = (int)T;
            g->K = (int)IC;
            g->batch = 36;
            return true;
        }
        case PPDL_OP_CONV_IM2COL: {
            const ppdl_tview *x = &src[0];
            const int K = p[14] & 0xFF, S = (p[14] >> 8) & 0xFF, P = (p[14] >> 16) & 0xFF;
            g->A = (const float *)src[1].data;
            g->lda = dst->ne[2];
            g->B = (const float *)x->data;
            g->C = (float *)dst->data;
            g->ldc = dst->ne[0] * dst->ne[1];
            g->bias = (const float *)src[2].data;
            g->M = (int)dst->ne[2];
            g->N = (int)(dst->ne[0] * dst->ne[1]);
            g->K = (int)(x->ne[2] * K * K);
            g->batch = 1;
            g->act = (p[14] >> 24) & 0xFF;
            g->IC = (int)x->ne[2];
            g->IH = (int)x->ne[1];
            g->IW = (int)x->ne[0];
            g->OW = (int)dst->ne[0];
            g->KW = K;
            g->S = S;
            g->P = P;
            *im2col = true;
            return true;
        }
        default:
            return false;
    }
}

}  // namespace

bool ppdl::gemm_args_of(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, GemmArgs *g, bool *im2col) {
    return args_of_node(p, dst, src, g, im2col);
}

extern "C" PPDL_HIP_API int64_t ppdl_hip_workspace_bytes(const int32_t op_params[16], const ppdl_tview *dst,
                                                         const ppdl_tview *src, int nsrc) {
    if (!op_params || (uint32_t)op_params[12] != (uint32_t)PPDL_MAGIC || !dst || nsrc < 0 ||
        (nsrc > 0 && !src))
        return -1;
    const int wi = ws_index(op_params);
    const int n = (wi >= 0 && nsrc > wi) ? wi : nsrc;  // ignore a workspace already attached
    if (check_op(op_params, dst, src, n) != PPDL_OK) return -1;
    if (op_params[13] == PPDL_OP_TOPK) return src[0].ne[1] * 8;  // one 64-bit key per token
    GemmArgs g;
    bool im2col;
    if (!args_of_node(op_params, dst, src, &g, &im2col)) return 0;
    return gemm_ws_bytes_for(g, im2col);
}

extern "C" PPDL_HIP_API int ppdl_hip_kernel_name(const int32_t op_params[16], const ppdl_tview *dst,
                                                 const ppdl_tview *src, int nsrc, char *buf, int cap) {
    if (!buf || cap < 1 || check_node(op_params, dst, src, nsrc) != PPDL_OK) return -1;
    GemmArgs g;
    bool im2col;
    std::string name;
    if (args_of_node(op_params, dst, src, &g, &im2col)) name = gemm_kernel_name(g, ws_of(op_params, src, nsrc).bytes, im2col);
    if (op_params[13] == PPDL_OP_WG4_CONV)
        name = wg4_conv_kernel_name((int)src[0].ne[2], (int)src[0].ne[1], (int)src[0].ne[0], (int)dst->ne[2]);
    snprintf(buf, (size_t)cap, "%s", name.c_str());
    return (int)name.size();
}

extern "C" PPDL_HIP_API int ppdl_hip_supports(const int32_t op_params[16], const ppdl_tview *dst,
                                              const ppdl_tview *src, int nsrc) {
    if (!op_params || (uint32_t)op_params[12] != (uint32_t)PPDL_MAGIC) return 0;
    if (!dst) {
        // id-only query, as the reference's gate: op 3 is carried for K=1 only
        switch (op_params[13]) {
            case PPDL_OP_CONV: return (op_params[14] & 0xFF) == 1;
            case PPDL_OP_MASKBOX: case PPDL_OP_MSDEF: case PPDL_OP_BIASACT: case PPDL_OP_WG4_INPUT:
            case PPDL_OP_WG4_OUTPUT: case PPDL_OP_WG4_MADD: case PPDL_OP_TOPK: case PPDL_OP_CONV1X1_BA:
            case PPDL_OP_WG4_INPUT_PAD: case PPDL_OP_CONV_IM2COL: case PPDL_OP_WG4_CONV: return 1;
            default: return 0;
        }
    }
    return check_op(op_params, dst, src, nsrc) == PPDL_OK ? 1 : 0;
}

int ppdl::run_node(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, int nsrc,
                   const GemmWorkspace *ws_in, hipStream_t s) {
    GemmArgs g;
    bool im2col;
    const GemmWorkspace ws = ws_in ? *ws_in : ws_of(p, src, nsrc);
    if (args_of_node(p, dst, src, &g, &im2col)) return status_of(im2col ? gemm_im2col(g, ws, s) : gemm_dense(g, ws, s));

    switch (p[13]) {
        case PPDL_OP_BIASACT: {
            const int64_t n = nelem(dst), plane = dst->ne[0] * dst->ne[1];
            return status_of(bias_act((const float *)src[0].data, (const float *)src[1].data,
                                      (float *)dst->data, n, plane, p[14], s));
        }
        case PPDL_OP_WG4_INPUT:
        case PPDL_OP_WG4_INPUT_PAD: {
            const ppdl_tview *x = &src[0];
            const int T = p[14], TH = p[15], TW = T / TH;
            return status_of(wg4_input((const float *)x->data, (float *)dst->data, (int)x->ne[0],
                                       (int)x->ne[1], (int)x->ne[2], TW, TH,
                                       p[13] == PPDL_OP_WG4_INPUT_PAD ? 1 : 0, (int)(dst->nb[1] / 4), s));
        }
        case PPDL_OP_WG4_OUTPUT: {
            const int OW = (int)dst->ne[0], OH = (int)dst->ne[1], OC = (int)dst->ne[2];
            return status_of(wg4_output((const float *)src[0].data, (const float *)src[1].data,
                                        nsrc >= 3 ? (const float *)src[2].data : nullptr,
                                        (float *)dst->data, (OW + 3) / 4, (OH + 3) / 4, OC, OW, OH,
                                        p[14], (int)(src[0].nb[1] / 4), s));
        }
        case PPDL_OP_WG4_CONV:
            return status_of(wg4_conv((const float *)src[0].data, (const float *)src[1].data, (const float *)src[2].data,
                                      (float *)dst->data, (int)src[0].ne[2], (int)src[0].ne[1], (int)src[0].ne[0],
                                      (int)dst->ne[2], p[14], s));
        case PPDL_OP_MSDEF:
            return status_of(msdeform((const float *)src[0].data, (int)(src[0].nb[1] / 4), (const float *)src[1].data,
                                      (int)(src[1].nb[1] / 4), (const float *)src[2].data, (int)(src[2].nb[1] / 4),
                                      (const float *)src[3].data, (float *)dst->data, (int)dst->ne[1], s));
        case PPDL_OP_MASKBOX:
            return status_of(mask_box((const float *)src[0].data, (float *)dst->data, (int)dst->ne[1], s));
        case PPDL_OP_TOPK:
            return status_of(topk((const float *)src[0].data, (int32_t *)dst->data, (int)src[0].ne[1],
                                  (int)src[0].ne[0], (int)dst->ne[0], ws.base, ws.bytes, s));
        default:
            return PPDL_UNSUPPORTED;
    }
}

int ppdl::check_node(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, int nsrc) {
    if (!p || (uint32_t)p[12] != (uint32_t)PPDL_MAGIC) return PPDL_UNSUPPORTED;
    if (!dst || (nsrc > 0 && !src) || nsrc < 0) return PPDL_EINVAL;
    return check_op(p, dst, src, nsrc);
}

int ppdl::workspace_src_index(const int32_t *p) { return ws_index(p); }

extern "C" PPDL_HIP_API int ppdl_hip_run(const int32_t op_params[16], const ppdl_tview *dst,
                                         const ppdl_tview *src, int nsrc, void *stream) {
    const int rc = check_node(op_params, dst, src, nsrc);
    if (rc != PPDL_OK) return rc;
    return run_node(op_params, dst, src, nsrc, nullptr, (hipStream_t)stream);
}

extern "C" PPDL_HIP_API int ppdl_hip_im2col_f32(const float *x, float *dst, int64_t IW, int64_t IH,
                                                int64_t OW, int64_t OH, int64_t KW, int64_t KH,
                                                int64_t IC, int64_t N, int64_t IC_IH_IW, int64_t IH_IW,
                                                int s0, int s1, int p0, int p1, int d0, int d1,
                                                void *stream) {
    if (!x || !dst) return 0;
    if (IW < 1 || IH < 1 || OW < 1 || OH < 1 || KW < 1 || KH < 1 || IC < 1 || N < 1) return 0;
    if (s0 < 1 || s1 < 1 || d0 < 1 || d1 < 1 || p0 < 0 || p1 < 0) return 0;
    if (N * OH * OW / 64 >= (int64_t)1 << 31 || IC * KH * KW / 64 >= 65535) return 0;
    return im2col_ggml(x, dst, IW, IH, OW, OH, KW, KH, IC, N, IC_IH_IW, IH_IW, s0, s1, p0, p1, d0, d1,
                       (hipStream_t)stream) == hipSuccess
               ? 1
               : 0;
}

extern "C" PPDL_HIP_API int ppdl_hip_repack_conv(const float *w, int64_t OC, int64_t IC, int64_t K,
                                                 float *wr, float *wg4) {
    if (!w || !wr || OC < 1 || IC < 1 || K < 1) return PPDL_EINVAL;
    if (wg4 && K != 3) return PPDL_EINVAL;
    for (int64_t oc = 0; oc < OC; oc++)
        for (int64_t ic = 0; ic < IC; ic++)
            for (int64_t t = 0; t < K * K; t++) wr[(t * IC + ic) * OC + oc] = w[(oc * IC + ic) * K * K + t];
    if (wg4) {
        // g~ = G g G^T per (ic, oc), float64 accumulation, one rounding to fp32
        for (int64_t ic = 0; ic < IC; ic++)
            for (int64_t oc = 0; oc < OC; oc++) {
                const float *g = w + (oc * IC + ic) * 9;
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
    return PPDL_OK;
}

extern "C" PPDL_HIP_API void ppdl_hip_wg4_matrices(double Bt[36], double G[18], double At[24]) {
    for (int i = 0; i < 6; i++)
        for (int j = 0; j < 6; j++)
            if (Bt) Bt[i * 6 + j] = kBt[i][j];
    for (int i = 0; i < 6; i++)
        for (int j = 0; j < 3; j++)
            if (G) G[i * 3 + j] = kG[i][j];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 6; j++)
            if (At) At[i * 6 + j] = kAt[i][j];
}
