/* ppdl_hip_ops.h — C-ABI of the MI355X (gfx950) tagged-op library.
 *
 * This is the device-side boundary of PP-DocLayoutV3's tagged custom ops.  A
 * ggml-based host tags GGML_OP_CUSTOM tensors with op_params[12] = PPDL_MAGIC
 * and op_params[13] = op id (src/ppdoclayout.cpp:48-53); a patched backend
 * hands each tagged node to this library as plain views.  Nothing in these
 * signatures is a ggml, HIP or torch type: a tensor is a `ppdl_tview`, a
 * stream is an opaque `void *` (a hipStream_t; NULL = the null stream).
 *
 * Every entry point is asynchronous on the given stream, allocates nothing,
 * never synchronises the host and changes no device-wide state, so any
 * sequence of calls can be captured into a hipGraph.  Weights are
 * caller-owned device buffers already repacked with ppdl_hip_repack_conv.
 *
 * Tensor convention (ggml's): ne[0] is the fastest-varying axis, nb[] are byte
 * strides.  An image is ne = (W, H, C, 1), i.e. CHW memory.
 */
#ifndef PPDL_HIP_OPS_H
#define PPDL_HIP_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PPDL_HIP_API __attribute__((visibility("default")))

#define PPDL_MAGIC 0x5050444C /* "PPDL", op_params[12] */

/* F(4,3) matrix-set tag, op_params[11] of ops 10, 11, 12, 15 and 17 (an
 * extension: the reference leaves slot 11 zero).  These ops use this
 * library's own Winograd matrices (ppdl_hip_wg4_matrices), so their .wg4
 * weights must come from ppdl_hip_repack_conv; the reference's host repack
 * (src/ppdoclayout.cpp:313-337) builds .wg4 with other matrices, and
 * mixing the two gives wrong convolutions without any error.  A host sets
 * this tag where it switches its repack to ppdl_hip_repack_conv; without it
 * the ops return PPDL_EINVAL. */
#define PPDL_WG4_SET 0x57473433 /* "WG43" */

/* Op ids (op_params[13]).  Ids 1..13 keep the reference's numbering and
 * parameter encoding (patches/ggml-ppdl.patch:120-132); ids >= 14 are fused
 * extensions emitted only by this project's own host. */
enum ppdl_op_id {
    PPDL_OP_MASKBOX       = 1,  /* mask logits -> inverse-sigmoid cxcywh box    */
    PPDL_OP_MSDEF         = 2,  /* multi-scale deformable-attention sampling    */
    PPDL_OP_CONV          = 3,  /* 1x1 conv as one GEMM, CHW out (K=1 only)     */
    PPDL_OP_BIASACT       = 5,  /* dst = act(src0 + bias[plane])                */
    PPDL_OP_WG4_INPUT     = 10, /* Winograd F(4,3) input transform (pre-padded) */
    PPDL_OP_WG4_OUTPUT    = 11, /* F(4,3) output transform + bias + act, CHW    */
    PPDL_OP_WG4_MADD      = 12, /* F(4,3) 36-plane batched GEMM                 */
    PPDL_OP_TOPK          = 13, /* top-300 tokens by max-class logit            */
    PPDL_OP_CONV1X1_BA    = 14, /* ext: op 3 + op 5 fused (GEMM+bias+act)       */
    PPDL_OP_WG4_INPUT_PAD = 15, /* ext: op 10 reading the UNPADDED input        */
    PPDL_OP_CONV_IM2COL   = 16, /* ext: implicit-im2col GEMM + bias + act       */
    PPDL_OP_WG4_CONV      = 17  /* ext: ops 15 -> 12 -> 11 in one kernel        */
};

/* Activation codes (op 5 params[14], op 11 params[14]); same values as the
 * reference's act_t (src/ppdoclayout.cpp:361). */
enum ppdl_act { PPDL_ACT_NONE = 0, PPDL_ACT_RELU = 1, PPDL_ACT_SILU = 2 };

/* Element types: same numbering as ggml_type so a ggml tensor's type passes
 * through unchanged. */
enum ppdl_type { PPDL_TYPE_F32 = 0, PPDL_TYPE_I32 = 26 };

/* Return codes of ppdl_hip_run. */
enum ppdl_status {
    PPDL_OK          = 0, /* enqueued                                           */
    PPDL_UNSUPPORTED = 1, /* op id/magic not handled here: the caller falls back */
    PPDL_EINVAL      = 2, /* shapes/strides/params violate the op's contract    */
    PPDL_ELAUNCH     = 3  /* the HIP launch itself failed                       */
};

/* A ggml-compatible tensor view.  `data` is a device pointer for every op. */
typedef struct {
    void   *data;
    int64_t ne[4];
    int64_t nb[4];
    int32_t type;
} ppdl_tview;

/* Placement gate: 1 if ppdl_hip_run executes this node on the GPU, else 0.
 * Replaces ggml_cuda_supports_ppdl_op (patches/ggml-ppdl.patch:908-917).
 * Host-only: touches no device.  dst/src may be NULL, in which case only the
 * magic and op id are checked (as the reference does). */
PPDL_HIP_API int ppdl_hip_supports(const int32_t op_params[16], const ppdl_tview *dst,
                                   const ppdl_tview *src, int nsrc);

/* Execute one tagged node on `stream`.  Replaces ggml_cuda_compute_forward_ppdl
 * (patches/ggml-ppdl.patch:612-817): the reference returns false for an unknown
 * id and GGML_ASSERTs on contract violations; this returns PPDL_UNSUPPORTED and
 * PPDL_EINVAL instead (validation happens before anything is enqueued).
 *
 * Per-op contract (srcs in order, all F32 contiguous unless stated):
 *  2  MSDEF     src: value ne(256,13125), offsets ne(192,NQ), attn logits
 *               ne(96,NQ), ref cxcywh ne(4,NQ); dst ne(256,NQ).  value,
 *               offsets and logits may be row-strided (nb[1] >= 4*ne[0]).
 *  3  CONV      src: x ne(W,H,IC), wr ne(OC,IC,1), bias ne(OC) (unused);
 *               params[14] = K | pad<<8 with K=1, pad=0; params[15] = 0
 *               (CHW out); dst ne(W,H,OC) = sum_ic x*wr, no bias.  x and
 *               dst may have padded channel planes (nb[1] = 4W, nb[2] >=
 *               4WH, a multiple of 4): an extension, the reference passes
 *               contiguous maps.
 *  5  BIASACT   src: in (any 4-d, contiguous), bias ne(ne2 of dst);
 *               params[14] = act; dst = act(in + bias[i / (ne0*ne1)]).
 *  10 WG4_INPUT src: padded x ne(IWp,IHp,IC) with IWp >= 4*TW+2,
 *               IHp >= 4*TH+2; params[14] = T (tiles), [15] = TH, TW = T/TH;
 *               dst ne(T,IC,36): dst[p][ic][t] = (Bt d B)[p] of the 6x6 patch.
 *  11 WG4_OUTPUT src: yt ne(T,OC,36), bias ne(OC); params[14] = act,
 *               [15] = TW; dst ne(W,H,OC) with T = ceil(W/4)*ceil(H/4).
 *               Optional src[2]: a contiguous map of dst's shape added after
 *               the activation (no counterpart in the reference's op, which
 *               takes two sources; the CSP layers end with it).
 *  12 WG4_MADD  src: dt ne(T,IC,36), wg4 ne(OC,IC,36); dst yt ne(T,OC,36):
 *               yt[p][oc][t] = sum_ic dt[p][ic][t] * wg4[p][ic][oc].
 *  1  MASKBOX   src: mask logits ne(40000,NQ); dst ne(4,NQ).
 *  13 TOPK      src: class logits ne(NC,NTOK), NTOK <= 13312; dst I32 ne(NQ):
 *               token indices by max-class logit, descending, ties to the
 *               lower index.
 *  14 CONV1X1_BA as op 3 plus bias/act: params[14] = act; params[15] = add
 *               mode: 0 none, 1 dst = act(conv + bias + src[3]), 2 dst =
 *               act(conv + bias) + src[3]; src[3] has dst's shape and
 *               strides.
 *  15 WG4_INPUT_PAD as op 10 but src is the unpadded x ne(W,H,IC) and the
 *               conv's zero pad of 1 is applied while reading.
 *  16 CONV_IM2COL src: x ne(IW,IH,IC), wr ne(OC,IC,K*K), bias ne(OC);
 *               params[14] = K | S<<8 | P<<16 | act<<24; params[15] = PE, an
 *               extra zero pad after the last column and row (the
 *               reference's ggml_pad before its k2 convs); dst ne(OW,OH,OC),
 *               OW = (IW+2P+PE-K)/S+1.
 *  17 WG4_CONV  the k3 s1 p1 conv of ops 15 -> 12 -> 11 as one kernel, no
 *               dt / yt planes: src x ne(W,H,IC), wg4 ne(OC,IC,36), bias
 *               ne(OC); params[14] = act, [15] = 0; dst ne(W,H,OC).
 *
 * Split-K workspace (ops 3, 12, 14, 16): one optional extra src after the
 * op's own (src[3] for 3/14/16, src[4] for 14 with an add, src[2] for 12),
 * a 16-byte aligned contiguous
 * buffer of ppdl_hip_workspace_bytes() bytes; its contents are scratch (no
 * initialisation needed).  Without it, or when it is smaller, the GEMM runs
 * with fewer or no K splits: results differ only by fp32 summation order, and
 * a given plan always sums in the same order.  Ops sharing one workspace must
 * not run concurrently.
 *
 * Op 13 takes the same kind of optional workspace as src[1] (8 bytes per
 * token): with it the per-token keys are computed by a grid-wide kernel
 * before the one-block selection; without it the selection block computes
 * them itself (slower, same result).
 */
PPDL_HIP_API int ppdl_hip_run(const int32_t op_params[16], const ppdl_tview *dst,
                              const ppdl_tview *src, int nsrc, void *stream);

/* Size of the device scratch array behind ppdl_hip_run_noalloc (16 MiB per
 * GPU, held from the first call on that GPU until the process ends). */
#define PPDL_HIP_NOALLOC_SCRATCH_BYTES (16LL << 20)

/* ppdl_hip_run without a workspace argument and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under hipGraph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  src holds the op's own sources only; the workspace
 * ppdl_hip_run would take as an extra src comes from a file-scope device
 * array of PPDL_HIP_NOALLOC_SCRATCH_BYTES, so results equal ppdl_hip_run's
 * with a full workspace.  Nodes whose workspace (ppdl_hip_workspace_bytes)
 * exceeds the array are rejected with PPDL_EINVAL and a message on stderr.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, concurrent graph replays) race on it. */
PPDL_HIP_API int ppdl_hip_run_noalloc(const int32_t op_params[16], const ppdl_tview *dst,
                                      const ppdl_tview *src, int nsrc, void *stream);

/* Workspace bytes the node would use (GEMM ops: its split-K plan, 0 = needs
 * none; op 13: 8 per token), or -1 if the node is invalid.  Host-only; no counterpart in the reference, whose
 * GEMMs run in cuBLAS with the backend's own workspace. */
PPDL_HIP_API int64_t ppdl_hip_workspace_bytes(const int32_t op_params[16], const ppdl_tview *dst,
                                              const ppdl_tview *src, int nsrc);

/* Name of the device kernel(s) ppdl_hip_run would launch for this node (with
 * the workspace src it carries, if any), e.g. "k_gemm_dma<64, 64, 2, false,
 * 2, 2, true>"; empty for ops that are not GEMMs.  Writes at most cap bytes
 * including the terminator and returns the full length, or -1 if the node is
 * invalid.  Launches nothing (it may read the current device's CU count).  No
 * counterpart in the reference: a diagnostic for tests and profiles. */
PPDL_HIP_API int ppdl_hip_kernel_name(const int32_t op_params[16], const ppdl_tview *dst,
                                      const ppdl_tview *src, int nsrc, char *buf, int cap);

/* F32 im2col in ggml's layout: dst[pix][k], pix = (n*OH + oh)*OW + ow,
 * k = ic*KH*KW + kh*KW + kw, zero where the tap falls outside the input.
 * Replaces ggml_cuda_ppdl_im2col_f32 (patches/ggml-ppdl.patch:885-906) with the
 * same argument list; as in the reference's index formula (:880) and its
 * layout test (:891), IC_IH_IW is the element stride between input channels
 * and IH_IW the stride between batch images.  Returns 1 when handled, 0 when
 * the arguments are out of range (the caller then uses its own kernel). */
PPDL_HIP_API int ppdl_hip_im2col_f32(const float *x, float *dst,
                                     int64_t IW, int64_t IH, int64_t OW, int64_t OH,
                                     int64_t KW, int64_t KH, int64_t IC, int64_t N,
                                     int64_t IC_IH_IW, int64_t IH_IW,
                                     int s0, int s1, int p0, int p1, int d0, int d1,
                                     void *stream);

/* Host-side weight repack at load time.  Replaces the loops of repack_convs
 * (src/ppdoclayout.cpp:262-337).  w_oihw: OC x IC x K x K (PyTorch OIHW, ggml
 * ne(K,K,IC,OC)), host memory.  wr (OC*IC*K*K floats): wr[t][ic][oc] with
 * t = kh*K + kw.  wg4 (36*IC*OC floats, K == 3 only, may be NULL):
 * wg4[u*6+v][ic][oc] = sum_ab G[u][a] G[v][b] w[oc][ic][a][b], accumulated in
 * float64 with this library's F(4,3) filter matrix G.  Returns 0 or PPDL_EINVAL. */
PPDL_HIP_API int ppdl_hip_repack_conv(const float *w_oihw, int64_t OC, int64_t IC, int64_t K,
                                      float *wr, float *wg4);

/* The F(4,3) matrices this library's ops 10/11/12/15 and the repack use, as
 * float64, row-major: Bt 6x6 (input: d~ = Bt d Bt^T), G 6x3 (filter:
 * g~ = G g G^T), At 4x6 (output: Y = At m At^T).  Host-only. */
PPDL_HIP_API void ppdl_hip_wg4_matrices(double Bt[36], double G[18], double At[24]);

#ifdef __cplusplus
}
#endif

#endif /* PPDL_HIP_OPS_H */
