"""ctypes binding of the PP-DocLayoutV3 runtime (include/ppdoclayout.h).

Mirrors the reference's C API (include/ppdoclayout.h of the reference:
ppdl_init / ppdl_init_ex / ppdl_infer / ppdl_dump / ppdl_dump_raw / ppdl_free)
plus this library's extensions (raw outputs, compute-only, graph timing).
Everything runs in libppdl_hip.so on the GPU; there is no CPU backend, and a
missing library raises.
"""
import ctypes

import numpy as np

import ppdl_hip

IMG = 800
NQ = 300
NC = 25
MASK_HW = 200
BACKEND_CPU, BACKEND_CUDA, BACKEND_HIP = 0, 1, 2

RAW_LOGITS, RAW_BOXES, RAW_ORDER, RAW_MASKS, RAW_TOPK, RAW_INIT_REF = range(6)
_RAW_SHAPE = {
    RAW_LOGITS: ((NQ, NC), np.float32),
    RAW_BOXES: ((NQ, 4), np.float32),
    RAW_ORDER: ((NQ, NQ), np.float32),  # [i][j] = q_i . k_j / 8
    RAW_MASKS: ((NQ, MASK_HW * MASK_HW), np.float32),
    RAW_TOPK: ((NQ,), np.int32),
    RAW_INIT_REF: ((NQ, 4), np.float32),
}

# every symbol include/ppdoclayout.h declares
EXPORTS = (
    "ppdl_init",
    "ppdl_init_ex",
    "ppdl_infer",
    "ppdl_dump",
    "ppdl_dump_raw",
    "ppdl_free",
    "ppdl_get_raw",
    "ppdl_compute",
    "ppdl_time_graph",
    "ppdl_graph_nodes",
    "ppdl_profile_nodes",
)


class Result(ctypes.Structure):
    _fields_ = [
        ("dets", ctypes.POINTER(ctypes.c_float)),
        ("num_dets", ctypes.c_int32),
        ("masks", ctypes.POINTER(ctypes.c_int32)),
        ("infer_ms", ctypes.c_double),
    ]


class NodeStat(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 64),
        ("kernel", ctypes.c_char * 64),
        ("cls", ctypes.c_int32),
        ("kernels", ctypes.c_int32),
        ("flops", ctypes.c_double),
        ("bytes", ctypes.c_double),
        ("us", ctypes.c_double),
    ]


NODE_OTHER, NODE_CONV_GEMM, NODE_LINEAR_GEMM = 0, 1, 2

_bound = None


def lib():
    global _bound
    L = ppdl_hip.lib()
    if _bound is None:
        vp, cp, i32 = ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int
        L.ppdl_init.argtypes = [cp, i32]
        L.ppdl_init.restype = vp
        L.ppdl_init_ex.argtypes = [cp, i32, i32]
        L.ppdl_init_ex.restype = vp
        L.ppdl_infer.argtypes = [vp, vp, i32, i32, ctypes.POINTER(Result)]
        L.ppdl_infer.restype = i32
        L.ppdl_dump.argtypes = [vp, cp]
        L.ppdl_dump.restype = i32
        L.ppdl_dump_raw.argtypes = [vp, cp]
        L.ppdl_dump_raw.restype = i32
        L.ppdl_free.argtypes = [vp]
        L.ppdl_free.restype = None
        L.ppdl_get_raw.argtypes = [vp, i32, vp, ctypes.c_int64]
        L.ppdl_get_raw.restype = ctypes.c_int64
        L.ppdl_compute.argtypes = [vp, vp]
        L.ppdl_compute.restype = i32
        L.ppdl_time_graph.argtypes = [vp, i32]
        L.ppdl_time_graph.restype = ctypes.c_double
        L.ppdl_graph_nodes.argtypes = [vp]
        L.ppdl_graph_nodes.restype = i32
        L.ppdl_profile_nodes.argtypes = [vp, i32, ctypes.POINTER(NodeStat), i32]
        L.ppdl_profile_nodes.restype = i32
        _bound = L
    return _bound


def _image(img):
    a = np.ascontiguousarray(img, dtype=np.float32)
    if a.shape != (3, IMG, IMG):
        raise ValueError("image must be float32 CHW 3x%dx%d, got %s" % (IMG, IMG, a.shape))
    return a


class PPDocLayout:
    """One loaded model with its captured graph (ppdl_ctx)."""

    def __init__(self, model_path, backend=BACKEND_HIP, dumps=False):
        self._L = lib()
        self._ctx = self._L.ppdl_init_ex(str(model_path).encode(), backend, 1 if dumps else 0)
        if not self._ctx:
            raise ppdl_hip.PpdlError("ppdl_init failed for %s (see stderr)" % model_path)

    def close(self):
        if self._ctx:
            self._L.ppdl_free(self._ctx)
            self._ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def infer(self, image, ori_h=IMG, ori_w=IMG):
        """-> (dets float32 (300, 7): label, score, x1, y1, x2, y2, order;
        masks int32 (300, 200, 200); graph time in ms)."""
        a = _image(image)
        r = Result()
        rc = self._L.ppdl_infer(self._ctx, a.ctypes.data, int(ori_h), int(ori_w), ctypes.byref(r))
        if rc != 0:
            raise ppdl_hip.PpdlError("ppdl_infer returned %d" % rc)
        n = r.num_dets
        dets = np.ctypeslib.as_array(r.dets, shape=(n * 7,)).reshape(n, 7).copy()
        masks = np.ctypeslib.as_array(r.masks, shape=(n * MASK_HW * MASK_HW,)).reshape(n, MASK_HW, MASK_HW).copy()
        return dets, masks, r.infer_ms

    def compute(self, image):
        rc = self._L.ppdl_compute(self._ctx, _image(image).ctypes.data)
        if rc != 0:
            raise ppdl_hip.PpdlError("ppdl_compute returned %d" % rc)

    def raw(self, which):
        shape, dt = _RAW_SHAPE[which]
        out = np.empty(shape, dt)
        n = self._L.ppdl_get_raw(self._ctx, which, out.ctypes.data, out.size)
        if n != out.size:
            raise ppdl_hip.PpdlError("ppdl_get_raw(%d) returned %d" % (which, n))
        return out

    def profile_nodes(self, iters):
        """[dict(name, kernel, cls, kernels, flops, bytes, us)] per graph node."""
        cap = 4096
        arr = (NodeStat * cap)()
        n = self._L.ppdl_profile_nodes(self._ctx, int(iters), arr, cap)
        if n < 0:
            raise ppdl_hip.PpdlError("ppdl_profile_nodes failed")
        return [dict(name=a.name.decode(), kernel=a.kernel.decode(), cls=a.cls, kernels=a.kernels, flops=a.flops,
                     bytes=a.bytes, us=a.us) for a in arr[:n]]

    def time_graph(self, iters):
        ms = self._L.ppdl_time_graph(self._ctx, int(iters))
        if ms < 0:
            raise ppdl_hip.PpdlError("ppdl_time_graph failed")
        return ms

    def graph_nodes(self):
        return self._L.ppdl_graph_nodes(self._ctx)

    def dump(self, directory):
        return self._L.ppdl_dump(self._ctx, str(directory).encode())

    def dump_raw(self, prefix):
        return self._L.ppdl_dump_raw(self._ctx, str(prefix).encode())


def read_dump(directory):
    """name -> array of a ppdl_dump directory (shapes.txt + <name>.bin; ne
    order reversed into numpy shapes)."""
    import os

    out = {}
    with open(os.path.join(directory, "shapes.txt")) as f:
        for line in f:
            name, ty, *ne = line.split()
            ne = [int(x) for x in ne]
            while len(ne) > 1 and ne[-1] == 1:
                ne.pop()
            a = np.fromfile(os.path.join(directory, name + ".bin"), np.int32 if ty == "i32" else np.float32)
            out[name] = a.reshape(tuple(reversed(ne)))
    return out
