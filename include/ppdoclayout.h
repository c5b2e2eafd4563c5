/* ppdoclayout.h — PP-DocLayoutV3 inference on MI355X.
 *
 * Same API as the reference's include/ppdoclayout.h (ppdl_init, ppdl_init_ex,
 * ppdl_infer, ppdl_dump, ppdl_dump_raw, ppdl_free; result layout and return
 * codes unchanged), with the GPU backend executed by this library's HIP
 * kernels and hipGraph replay.  Declarations marked "extension" have no
 * counterpart in the reference.
 */
#ifndef PPDOCLAYOUT_H
#define PPDOCLAYOUT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PPDL_API __attribute__((visibility("default")))

#define PPDL_IMG_SIZE   800  /* fixed input resolution (square)         */
#define PPDL_NUM_DETS   300  /* rows in every result                    */
#define PPDL_DET_FIELDS 7    /* label,score,x1,y1,x2,y2,order per row   */
#define PPDL_MASK_HW    200  /* per-detection mask is 200x200           */

#define PPDL_BACKEND_CPU  0  /* not provided by this library: init returns NULL */
#define PPDL_BACKEND_CUDA 1  /* the GPU backend; on this build the same as HIP  */
#define PPDL_BACKEND_HIP  2  /* MI355X (gfx950)                                  */

typedef struct ppdl_ctx ppdl_ctx;

/* Pointers stay valid until the next ppdl_infer or ppdl_free on the same ctx.
 * (include/ppdoclayout.h:28-35 of the reference) */
typedef struct {
    const float   * dets;     /* [PPDL_NUM_DETS * PPDL_DET_FIELDS], score-descending */
    int32_t         num_dets; /* always PPDL_NUM_DETS */
    const int32_t * masks;    /* [PPDL_NUM_DETS * PPDL_MASK_HW * PPDL_MASK_HW] 0/1,
                                 row i corresponds to dets row i */
    double          infer_ms; /* graph compute time of this call */
} ppdl_result;

/* Load a GGUF model (F32, BN folded) and build the compute graph.  Returns
 * NULL on failure (details on stderr). */
PPDL_API ppdl_ctx * ppdl_init(const char * model_path, int backend);

/* Same, with intermediate-tensor dumping enabled (see ppdl_dump). */
PPDL_API ppdl_ctx * ppdl_init_ex(const char * model_path, int backend, int enable_dumps);

/* Run inference. image_chw: float32 CHW 3x800x800, RGB, /255-normalised.
 * ori_h/ori_w: original image size for box coordinate restore.  Returns 0 on
 * success, 1 on bad arguments, 2 on a compute failure. */
PPDL_API int ppdl_infer(ppdl_ctx * ctx, const float * image_chw,
                        int ori_h, int ori_w, ppdl_result * result);

/* Write intermediate tensors of the last infer to dir (requires
 * ppdl_init_ex with enable_dumps).  Returns 0 on success. */
PPDL_API int ppdl_dump(ppdl_ctx * ctx, const char * dir);

/* Write raw graph outputs of the last infer with path prefix: <pfx>logits.bin
 * (300x25 f32), <pfx>boxes.bin (300x4 sigmoid cxcywh f32), <pfx>order.bin
 * (300x300 f32), <pfx>sel.bin (300 i32).  Returns 0 on success. */
PPDL_API int ppdl_dump_raw(ppdl_ctx * ctx, const char * pfx);

PPDL_API void ppdl_free(ppdl_ctx * ctx);

/* ---- extensions ---- */

/* Raw outputs of the last ppdl_infer / ppdl_compute, copied to host memory:
 * which = 0 logits (300x25), 1 boxes (300x4), 2 order (300x300),
 * 3 mask logits (300x40000), 4 top-300 encoder token indices (i32, 300),
 * 5 initial reference boxes before sigmoid (300x4).  n = capacity in
 * elements.  Returns the element count written, or -1. */
PPDL_API int64_t ppdl_get_raw(ppdl_ctx * ctx, int which, void * dst, int64_t n);

/* Upload an image (host CHW 3x800x800) and run the graph once, without
 * downloading or postprocessing.  Returns 0 / 1 / 2 like ppdl_infer. */
PPDL_API int ppdl_compute(ppdl_ctx * ctx, const float * image_chw);

/* Replay the graph `iters` times on the resident input and return the mean
 * device time per replay in ms (HIP events on the replay stream), or < 0. */
PPDL_API double ppdl_time_graph(ppdl_ctx * ctx, int iters);

/* Number of kernel nodes one graph replay executes (0 if not built). */
PPDL_API int ppdl_graph_nodes(ppdl_ctx * ctx);

/* Per-node device time of the graph: each node (one layer's kernels) is
 * captured `iters` times into a graph of its own, replayed between two HIP
 * events on the graph's stream (in-graph launch cost, no host launch cost). */
typedef struct {
    char    name[64];    /* layer / node name                                   */
    char    kernel[64];  /* GEMM nodes: the device kernel(s) the plan launches   */
    int32_t cls;         /* 0 other, 1 conv GEMM, 2 linear (token-major) GEMM    */
    int32_t kernels;     /* kernel launches per run of the node                  */
    double  flops;       /* GEMM nodes: algorithmic FLOP per run (Winograd: the
                            36-plane GEMM), else 0                               */
    double  bytes;       /* GEMM nodes: compulsory HBM bytes per run (A, B and C
                            once each), else 0                                   */
    double  us;          /* mean device time per run, microseconds              */
} ppdl_node_stat;

/* Fills out[0..n) for the first min(cap, nodes) nodes; returns n or -1.
 * iters > 0: each node alone, captured iters times into a graph of its own.
 * iters < 0: the whole graph captured once with a wall-clock stamp kernel
 * after every node and replayed -iters times; `us` is then the node's mean
 * share of a replay in context, less the interval of an empty stamp pair.
 * Intermediate buffers are left in an arbitrary state (the next ppdl_infer or
 * ppdl_compute recomputes them). */
PPDL_API int ppdl_profile_nodes(ppdl_ctx * ctx, int iters, ppdl_node_stat * out, int cap);

#ifdef __cplusplus
}
#endif

#endif /* PPDOCLAYOUT_H */
