"""ctypes binding of libppdl_hip.so, the tagged-op C-ABI (include/ppdl_hip_ops.h).

Tensors cross the boundary as `ppdl_tview` structs (ggml convention: ne[0] is
the fastest axis, nb[] byte strides).  `view()` builds one from a contiguous
torch tensor; torch is only the allocator and stream provider here.  There is
no CPU fallback: if the library is missing, loading raises.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libppdl_hip.so")

PPDL_MAGIC = 0x5050444C
WG4_SET = 0x57473433  # op_params[11] of the F(4,3) ops: .wg4 from this library's repack

OP_MASKBOX = 1
OP_MSDEF = 2
OP_CONV = 3
OP_BIASACT = 5
OP_WG4_INPUT = 10
OP_WG4_OUTPUT = 11
OP_WG4_MADD = 12
OP_TOPK = 13
OP_CONV1X1_BA = 14
OP_WG4_INPUT_PAD = 15
OP_CONV_IM2COL = 16
OP_WG4_CONV = 17

ACT_NONE, ACT_RELU, ACT_SILU = 0, 1, 2

TYPE_F32 = 0
TYPE_I32 = 26

OK, UNSUPPORTED, EINVAL, ELAUNCH = 0, 1, 2, 3

# every symbol include/ppdl_hip_ops.h declares
EXPORTS = (
    "ppdl_hip_supports",
    "ppdl_hip_run",
    "ppdl_hip_im2col_f32",
    "ppdl_hip_repack_conv",
    "ppdl_hip_wg4_matrices",
    "ppdl_hip_workspace_bytes",
    "ppdl_hip_run_noalloc",
    "ppdl_hip_kernel_name",
)

NOALLOC_SCRATCH_BYTES = 16 << 20  # PPDL_HIP_NOALLOC_SCRATCH_BYTES


class TView(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_int64 * 4),
        ("type", ctypes.c_int32),
    ]


class PpdlError(RuntimeError):
    pass


_lib = None


def build():
    """Compile lib/libppdl_hip.so for gfx950 (make -C ppdoclayout-ggml_amd)."""
    import subprocess

    subprocess.run(["make", "-s", "-j8", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PpdlError(f"{LIB_PATH} is missing: build it with `make -C {_HERE}`")
        L = ctypes.CDLL(LIB_PATH)
        i32p = ctypes.POINTER(ctypes.c_int32)
        tvp = ctypes.POINTER(TView)
        L.ppdl_hip_supports.argtypes = [i32p, tvp, tvp, ctypes.c_int]
        L.ppdl_hip_supports.restype = ctypes.c_int
        L.ppdl_hip_run.argtypes = [i32p, tvp, tvp, ctypes.c_int, ctypes.c_void_p]
        L.ppdl_hip_run.restype = ctypes.c_int
        L.ppdl_hip_run_noalloc.argtypes = [i32p, tvp, tvp, ctypes.c_int, ctypes.c_void_p]
        L.ppdl_hip_run_noalloc.restype = ctypes.c_int
        L.ppdl_hip_kernel_name.argtypes = [i32p, tvp, tvp, ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
        L.ppdl_hip_kernel_name.restype = ctypes.c_int
        L.ppdl_hip_im2col_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 10 + [
            ctypes.c_int
        ] * 6 + [ctypes.c_void_p]
        L.ppdl_hip_im2col_f32.restype = ctypes.c_int
        f32p = ctypes.POINTER(ctypes.c_float)
        L.ppdl_hip_repack_conv.argtypes = [f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, f32p, f32p]
        L.ppdl_hip_repack_conv.restype = ctypes.c_int
        f64p = ctypes.POINTER(ctypes.c_double)
        L.ppdl_hip_wg4_matrices.argtypes = [f64p, f64p, f64p]
        L.ppdl_hip_wg4_matrices.restype = None
        L.ppdl_hip_workspace_bytes.argtypes = [i32p, tvp, tvp, ctypes.c_int]
        L.ppdl_hip_workspace_bytes.restype = ctypes.c_int64
        _lib = L
    return _lib


def params(op, p14=0, p15=0, wg4_set=True):
    """op_params[16] with the tag in slots 12/13 (src/ppdoclayout.cpp:48-53)
    and, unless wg4_set is False, the F(4,3) matrix-set tag in slot 11 (this
    binding's .wg4 weights come from repack_conv)."""
    p = (ctypes.c_int32 * 16)()
    if wg4_set:
        p[11] = ctypes.c_int32(WG4_SET).value
    p[12] = ctypes.c_int32(PPDL_MAGIC).value
    p[13] = op
    p[14] = ctypes.c_int32(p14).value
    p[15] = ctypes.c_int32(p15).value
    return p


def view(t):
    """ppdl_tview of a contiguous torch tensor (shape reversed into ne)."""
    import torch

    if not t.is_contiguous():
        raise PpdlError("view() needs a contiguous tensor")
    if t.dim() > 4:
        raise PpdlError("at most 4 dims")
    if t.dtype == torch.float32:
        ty = TYPE_F32
    elif t.dtype == torch.int32:
        ty = TYPE_I32
    else:
        raise PpdlError(f"unsupported dtype {t.dtype}")
    ne = list(reversed(t.shape)) + [1] * (4 - t.dim())
    v = TView()
    v.data = t.data_ptr()
    nb = 4
    for i in range(4):
        v.ne[i] = ne[i]
        v.nb[i] = nb
        nb *= ne[i]
    v.type = ty
    return v


def raw_view(ptr, ne, ty=TYPE_F32):
    """ppdl_tview of a raw device pointer with contiguous ggml dims `ne`."""
    v = TView()
    v.data = ptr
    ne = list(ne) + [1] * (4 - len(ne))
    nb = 4
    for i in range(4):
        v.ne[i] = ne[i]
        v.nb[i] = nb
        nb *= ne[i]
    v.type = ty
    return v


def chw_view(t, W, H):
    """ppdl_tview ne(W, H, C) of a contiguous (C, ld) tensor whose rows are
    channel planes of W*H values padded to ld (plane stride nb[2] = 4*ld)."""
    v = view(t)
    C, ld = t.shape
    if ld < W * H:
        raise PpdlError("plane stride below W*H")
    v.ne[0], v.ne[1], v.ne[2], v.ne[3] = W, H, C, 1
    v.nb[0], v.nb[1], v.nb[2] = 4, 4 * W, 4 * ld
    v.nb[3] = v.nb[2] * C
    return v


def _views(dst, srcs):
    d = dst if isinstance(dst, TView) else view(dst)
    s = [x if isinstance(x, TView) else view(x) for x in srcs]
    arr = (TView * max(1, len(s)))(*s)
    return d, arr, len(s)


def current_stream():
    import torch

    return torch.cuda.current_stream().cuda_stream


def run(op, dst, srcs, p14=0, p15=0, stream=None):
    """Enqueue one tagged op; returns the ppdl_status code."""
    d, arr, n = _views(dst, srcs)
    s = current_stream() if stream is None else stream
    return lib().ppdl_hip_run(params(op, p14, p15), ctypes.byref(d), arr, n, ctypes.c_void_p(s))


def run_noalloc(op, dst, srcs, p14=0, p15=0, stream=None):
    """Enqueue one tagged op through ppdl_hip_run_noalloc (the op's own srcs
    only; its workspace comes from the library's device scratch array)."""
    d, arr, n = _views(dst, srcs)
    s = current_stream() if stream is None else stream
    return lib().ppdl_hip_run_noalloc(params(op, p14, p15), ctypes.byref(d), arr, n, ctypes.c_void_p(s))


def run_checked(op, dst, srcs, p14=0, p15=0, stream=None):
    rc = run(op, dst, srcs, p14, p15, stream)
    if rc != OK:
        raise PpdlError(f"ppdl_hip_run(op={op}) returned {rc}")


def supports(op, p14=0, p15=0, dst=None, srcs=()):
    L = lib()
    if dst is None:
        return L.ppdl_hip_supports(params(op, p14, p15), None, None, 0)
    d, arr, n = _views(dst, srcs)
    return L.ppdl_hip_supports(params(op, p14, p15), ctypes.byref(d), arr, n)


def workspace_bytes(op, dst, srcs, p14=0, p15=0):
    """Split-K workspace bytes the node's GEMM plan uses (0: none, -1: invalid node)."""
    d, arr, n = _views(dst, srcs)
    return lib().ppdl_hip_workspace_bytes(params(op, p14, p15), ctypes.byref(d), arr, n)


def kernel_name(op, dst, srcs, p14=0, p15=0):
    """Device kernel(s) ppdl_hip_run would launch for the node ('' for non-GEMM ops)."""
    d, arr, n = _views(dst, srcs)
    buf = ctypes.create_string_buffer(256)
    rc = lib().ppdl_hip_kernel_name(params(op, p14, p15), ctypes.byref(d), arr, n, buf, 256)
    if rc < 0:
        raise PpdlError(f"ppdl_hip_kernel_name(op={op}): invalid node")
    return buf.value.decode()


def make_workspace(nbytes):
    """A zero-filled device workspace of at least nbytes (torch int32)."""
    import torch

    return torch.zeros(max(1, (nbytes + 3) // 4), dtype=torch.int32, device="cuda")


def im2col_f32(x, dst, IW, IH, OW, OH, KW, KH, IC, N, ch_stride, img_stride, s0, s1, p0, p1, d0, d1,
               stream=None):
    s = current_stream() if stream is None else stream
    xp = x if isinstance(x, int) else x.data_ptr()
    dp = dst if isinstance(dst, int) else dst.data_ptr()
    return lib().ppdl_hip_im2col_f32(xp, dp, IW, IH, OW, OH, KW, KH, IC, N, ch_stride, img_stride,
                                     s0, s1, p0, p1, d0, d1, ctypes.c_void_p(s))


def repack_conv(w):
    """Host repack of an OIHW weight: (wr [K*K][IC][OC], wg4 [36][IC][OC] | None)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    OC, IC, K, _ = w.shape
    wr = np.empty((K * K, IC, OC), np.float32)
    wg4 = np.empty((36, IC, OC), np.float32) if K == 3 else None
    f32p = ctypes.POINTER(ctypes.c_float)
    rc = lib().ppdl_hip_repack_conv(
        w.ctypes.data_as(f32p), OC, IC, K, wr.ctypes.data_as(f32p),
        None if wg4 is None else wg4.ctypes.data_as(f32p))
    if rc != OK:
        raise PpdlError(f"ppdl_hip_repack_conv returned {rc}")
    return wr, wg4


def wg4_matrices():
    f64p = ctypes.POINTER(ctypes.c_double)
    Bt, G, At = np.empty(36), np.empty(18), np.empty(24)
    lib().ppdl_hip_wg4_matrices(Bt.ctypes.data_as(f64p), G.ctypes.data_as(f64p), At.ctypes.data_as(f64p))
    return Bt.reshape(6, 6), G.reshape(6, 3), At.reshape(4, 6)
