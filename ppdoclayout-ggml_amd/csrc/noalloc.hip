// ppdl_hip_run_noalloc: ppdl_hip_run for callers that cannot allocate device
// memory (code under hipGraph capture, tight serving loops, harnesses that
// forbid hipMalloc).  The workspace a node would take as an extra src (split-K
// partials of the GEMM ops, the per-token keys of op 13) comes from `scratch`,
// a file-scope device array of kScratchBytes that every GPU the library runs
// on holds until the process ends.  Nothing here calls hipMalloc / hipFree.
//
// The array's name is a host-side stand-in in host code: its device address is
// looked up once per device with hipGetSymbolAddress (with that device
// current) and only that address is handed to kernels.
//
// Contents: the split-K partials and top-k keys are fully written by the
// kernels of the same call before they are read, so nothing is cleared and no
// contents carry over between calls.  All calls on one GPU share its array:
// calls that overlap on one GPU (different streams, or graphs replayed
// concurrently) race on it.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "../../include/ppdl_hip_ops.h"
#include "ppdl_internal.h"

namespace {

constexpr int64_t kScratchBytes = PPDL_HIP_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
void *g_addr[kMaxDevices] = {};

// Device address of the current device's copy of `scratch`, or nullptr.
void *scratch_of_current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_addr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "ppdl_hip_run_noalloc: hipGetSymbolAddress failed on device %d: %s\n", dev,
                    hipGetErrorString(e));
            return nullptr;
        }
        g_addr[dev] = p;
    }
    return g_addr[dev];
}

}  // namespace

extern "C" PPDL_HIP_API int ppdl_hip_run_noalloc(const int32_t op_params[16], const ppdl_tview *dst,
                                                 const ppdl_tview *src, int nsrc, void *stream) {
    const int rc = ppdl::check_node(op_params, dst, src, nsrc);
    if (rc != PPDL_OK) return rc;
    const int wi = ppdl::workspace_src_index(op_params);
    if (wi >= 0 && nsrc > wi) {
        fprintf(stderr, "ppdl_hip_run_noalloc: op %d takes no workspace src here (src[%d] given)\n",
                (int)op_params[13], wi);
        return PPDL_EINVAL;
    }
    const int64_t need = ppdl_hip_workspace_bytes(op_params, dst, src, nsrc);
    if (need < 0) return PPDL_EINVAL;
    if (need > kScratchBytes) {
        fprintf(stderr,
                "ppdl_hip_run_noalloc: op %d needs %lld workspace bytes, more than the %lld-byte scratch "
                "array; use ppdl_hip_run with a caller workspace\n",
                (int)op_params[13], (long long)need, (long long)kScratchBytes);
        return PPDL_EINVAL;
    }
    ppdl::GemmWorkspace ws{nullptr, 0};
    if (need > 0) {
        ws.base = scratch_of_current_device();
        if (!ws.base) return PPDL_ELAUNCH;
        ws.bytes = kScratchBytes;
    }
    return ppdl::run_node(op_params, dst, src, nsrc, &ws, (hipStream_t)stream);
}
