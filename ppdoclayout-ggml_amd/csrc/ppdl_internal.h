// Internal declarations shared by the HIP kernels and the C-ABI dispatcher.
#pragma once

#include <hip/hip_runtime.h>
#include <string>
#include <stdint.h>

#include "../../include/ppdl_hip_ops.h"

namespace ppdl {

// ---- model geometry fixed by PP-DocLayoutV3 (src/ppdoclayout.cpp:31-44) ----
constexpr int kDM = 256;           // d_model
constexpr int kNH = 8;             // attention heads
constexpr int kHD = 32;            // head dim
constexpr int kNLVL = 3;           // feature levels
constexpr int kNPTS = 4;           // sampling points per level
constexpr int kNTOK = 13125;       // 100^2 + 50^2 + 25^2 value tokens
constexpr int kMaskHW = 200;       // mask side
constexpr int kMaskPix = kMaskHW * kMaskHW;

// ---- Winograd F(4,3), Toom-Cook points {0, 1, -1, 2, -1/2, inf} ----
// Convention: Y = At [ (G g G^T) (.) (Bt d Bt^T) ] At^T over 6x6 input tiles
// with stride 4.  Bt and At hold dyadic rationals (exact in FP32); G holds
// thirds and fifteenths and is applied in float64 at repack time only.
// Chosen over {0,+-1,+-2} for a ~2.5x smaller FP32 error on 256-channel convs.
constexpr float kBt[6][6] = {
    {1.0f, 1.5f, -2.0f, -1.5f, 1.0f, 0.0f},
    {0.0f, -1.0f, -2.5f, -0.5f, 1.0f, 0.0f},
    {0.0f, 1.0f, 0.5f, -2.5f, 1.0f, 0.0f},
    {0.0f, -0.5f, -1.0f, 0.5f, 1.0f, 0.0f},
    {0.0f, 2.0f, -1.0f, -2.0f, 1.0f, 0.0f},
    {0.0f, 1.0f, 1.5f, -2.0f, -1.5f, 1.0f},
};
constexpr float kAt[4][6] = {
    {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 0.0f},
    {0.0f, 1.0f, -1.0f, 2.0f, -0.5f, 0.0f},
    {0.0f, 1.0f, 1.0f, 4.0f, 0.25f, 0.0f},
    {0.0f, 1.0f, -1.0f, 8.0f, -0.125f, 1.0f},
};
constexpr double kG[6][3] = {
    {1.0, 0.0, 0.0},
    {-1.0 / 3.0, -1.0 / 3.0, -1.0 / 3.0},
    {1.0 / 3.0, -1.0 / 3.0, 1.0 / 3.0},
    {1.0 / 15.0, 2.0 / 15.0, 4.0 / 15.0},
    {-16.0 / 15.0, 8.0 / 15.0, -4.0 / 15.0},
    {0.0, 0.0, 1.0},
};

// ---- GEMM core: C[m][n] = epi( sum_k A(m,k) * B(k,n) ) ----
// A is stored k-major (element (m,k) at A[k*lda + m], a_rowmajor = 0) or
// row-major (A[m*lda + k], a_rowmajor = 1: token-major activations); B is a
// dense k-major matrix or an implicit im2col view of a CHW image.
// Epilogue: v = acc + bias[m or n]; v += add (add_mode 1); v = act(v);
// v += add (add_mode 2) or v = sigmoid(v + inv_sigmoid(add)) (add_mode 3, box
// refinement; add may be C itself); store at C[m*ldc + n], or C[n*ldc + m]
// when c_trans (a CHW conv result written token-major).  `add` uses C's
// layout.  Prologue (row-major A, small-GEMM kernel only): for output columns
// n < a_add_n the A operand is A + a_add (same lda), e.g. tokens + position
// embedding in front of the q|k columns of a fused q|k|v projection.
struct GemmArgs {
    const float *A;
    int64_t lda, sA;  // sA: batch stride (elements)
    const float *B;
    int64_t ldb, sB;
    float *C;
    int64_t ldc, sC;
    const float *bias;  // per-m (bias_n = 0) or per-n (bias_n = 1) bias, or nullptr
    int M, N, K, batch, act;
    // implicit im2col geometry: B[k][n] = x[ic][oy*S-P+kh][ox*S-P+kw] with
    // zeros outside [0,IH) x [0,IW) (the image may be padded beyond IH/IW by
    // choosing OW/OH), k = (kh*KW + kw)*IC + ic, n = oy*OW + ox
    int IC, IH, IW, OW, KW, S, P;
    int a_rowmajor, bias_n, c_trans, add_mode;
    // set by the dispatcher: B rows readable as whole float4s up to this
    // column (N itself, or N rounded up to 4 when ldb leaves room), 0 if not
    int n_vec;
    const float *add;
    const float *a_add;  // nullptr: none; a_add_n is then ignored
    int a_add_n;         // a multiple of 32
    // A computed in the loader (small-GEMM kernel only): with a_w4 set, the A
    // operand is relu(X W4 + b4) for the 4-column row-major X in A / lda,
    // W4 = a_w4[4][K] (row j at a_w4 + j*K) and b4 = a_b4[K]; K % 4 == 0.
    // It fuses a 4-in ReLU linear (the decoder's query-position MLP input)
    // into the GEMM that consumes it.
    const float *a_w4;
    const float *a_b4;
    // Sign-bit output (k_gemm / k_gemm_dma epilogues, no split-K, N % 32 ==
    // 0): with bits set the results are not stored; bit n % 32 of word
    // bits[m * (N / 32) + n / 32] is (acc > 0), before any bias or act.
    uint32_t *bits;
    // Row-norm prologue (small-GEMM kernel, row-major A, K = 256 or 512):
    // with ln_g set, the A operand is LN(A) * ln_g + ln_b per row (layer
    // norm, eps 1e-5) before any a_add, and when ln_out is set the normed
    // rows are also stored there ([M][K], token-major).
    const float *ln_g;
    const float *ln_b;
    float *ln_out;
    // Box-refinement prologue (with a_w4, small-GEMM kernel): with box_h set,
    // the 4-column X of row m is refine(box_b + box_h[m] . box_w, A[m]) (the
    // previous layer's box head: box_h [M][box_k] row-major with row stride
    // box_ldh, box_w [box_k][4], box_k == 256), and the blocks of the first
    // column tile store those rows to box_out ([M][4]).
    const float *box_h;
    const float *box_w;
    const float *box_b;
    float *box_out;
    int box_ldh, box_k;
};

// act codes of the GEMM epilogue and the elementwise kernels
enum { kActNone = 0, kActRelu = 1, kActSilu = 2, kActGelu = 3, kActSigmoid = 4 };

// Split-K workspace: fp32 partials, splits x batch x M x N, fully rewritten by
// every launch that uses it (no initial contents required).
struct GemmWorkspace {
    void *base;
    int64_t bytes;
};
struct GemmPlan {
    int cfg;     // block-shape index
    int splits;  // split-K factor (1 = none)
};

GemmPlan gemm_plan(const GemmArgs &g, int64_t ws_bytes, bool im2col);
int64_t gemm_ws_bytes(int M, int N, int batch, int cfg, int splits);
int64_t gemm_ws_bytes_for(const GemmArgs &g, bool im2col);  // workspace the unconstrained plan uses
hipError_t gemm_dense(const GemmArgs &g, const GemmWorkspace &ws, hipStream_t s);
// the kernel(s) the plan for g launches, named as the device symbols
std::string gemm_kernel_name(const GemmArgs &g, int64_t ws_bytes, bool im2col);
// GEMM description of a validated conv / madd tagged node (ppdl_ops.cpp)
bool gemm_args_of(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, GemmArgs *g, bool *im2col);
// Tagged-node validation (magic, pointers, the op's contract): PPDL_OK,
// PPDL_EINVAL or PPDL_UNSUPPORTED, touching no device (ppdl_ops.cpp)
int check_node(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, int nsrc);
// Enqueue a node that check_node accepted.  ws, when not null, is the
// workspace the node's kernels use instead of an attached workspace src.
int run_node(const int32_t *p, const ppdl_tview *dst, const ppdl_tview *src, int nsrc, const GemmWorkspace *ws,
             hipStream_t s);
// src index of the op's optional workspace, or -1 for ops that take none
int workspace_src_index(const int32_t *p);
hipError_t gemm_im2col(const GemmArgs &g, const GemmWorkspace &ws, hipStream_t s);
// Shape-fitted 16x16-MFMA GEMM for dense k-major A and B (gemm_lt.hip): no
// workspace.  gemm_lt_pick returns a menu index or -1 (g.n_vec must be set;
// `wanted`: the caller's planner prefers this kernel for the shape).
bool gemm_lt_ok(const GemmArgs &g);
int gemm_lt_pick(const GemmArgs &g, int cus, bool wanted);
int gemm_lt_num_cfgs();
hipError_t gemm_lt(const GemmArgs &g, int cfg, hipStream_t s);
std::string gemm_lt_name(int cfg);

// ---- Winograd transforms ----
// pad: 0 when x is already padded (op 10), 1 when the conv's pad is fused.
// dt / yt planes: [36][C][ldt] with the T = TW*TH tiles first in each row
hipError_t wg4_input(const float *x, float *dt, int IW, int IH, int IC, int TW, int TH, int pad, int ldt,
                     hipStream_t s);
// conv i's output transform (+ bias + act, y stored [C][OH][OW]) and conv
// i+1's input transform (pad 1) of y into dt [36][C][ldt_in], one launch
hipError_t wg4_chain(const float *yt, const float *bias, float *y, float *dt, int C, int OW, int OH, int act,
                     int ldt_out, int ldt_in, hipStream_t s);
bool wg4_chain_fits(int OW);  // the band of a map OW wide fits the kernel's LDS
// add (optional, out's shape): added after the activation
hipError_t wg4_output(const float *yt, const float *bias, const float *add, float *out, int TW, int TH, int OC,
                      int OW, int OH, int act, int ldt, hipStream_t s);
// the whole k3 s1 p1 conv in one kernel (op 17): x [IC][H][W], wg4
// [36][IC][OC], out [OC][H][W] = act(conv + bias)
hipError_t wg4_conv(const float *x, const float *wg4, const float *bias, float *out, int IC, int H, int W, int OC,
                    int act, hipStream_t s);
std::string wg4_conv_kernel_name(int IC, int H, int W, int OC);  // the instance the launch uses

// ---- elementwise / data movement ----
hipError_t bias_act(const float *in, const float *bias, float *out, int64_t n, int64_t plane,
                    int act, hipStream_t s);
hipError_t im2col_ggml(const float *x, float *dst, int64_t IW, int64_t IH, int64_t OW, int64_t OH,
                       int64_t KW, int64_t KH, int64_t IC, int64_t N, int64_t ch_stride,
                       int64_t img_stride, int s0, int s1, int p0, int p1, int d0, int d1,
                       hipStream_t s);

// ---- decoder ops ----
// val: 13125 token rows of 256 channels, row stride ldv (>= 256) floats
hipError_t msdeform(const float *val, int ldv, const float *off, int ldo, const float *awr, int ldw,
                    const float *ref, float *out, int nq, hipStream_t s);
hipError_t mask_box(const float *ml, float *out, int nq, hipStream_t s);
// the same boxes from the masks' sign bits [nq][40000 / 32] (bit p % 32 of
// word p / 32: logit of pixel p > 0), bit-identical to mask_box
hipError_t mask_box_bits(const uint32_t *bits, float *out, int nq, hipStream_t s);
// ws (optional, >= 8 * ntok bytes): per-token keys, computed grid-wide first
hipError_t topk(const float *logits, int32_t *out, int ntok, int nc, int nq, void *ws, int64_t ws_bytes,
                hipStream_t s);

}  // namespace ppdl
