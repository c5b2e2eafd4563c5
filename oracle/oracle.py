"""ctypes front-end of liboracle.so — the CPU restatement of the tagged-op path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, where it is the checker (or the timed CPU
reference), never the thing shipped.  All arrays are numpy, C-contiguous.
Layouts: images (C, H, W); conv weights (OC, IC, K, K); token tensors
(tokens, channels).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i = ctypes.c_int
_i64 = ctypes.c_int64


def build():
    """Compile liboracle.so (make -C oracle)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_conv2d_ref.argtypes = [_f32p, _i, _i, _i, _f32p, _i, _i, _i, _i, _f32p, _i, _f32p, _i]
        L.orc_conv2d_f64.argtypes = [_f32p, _i, _i, _i, _f32p, _i, _i, _i, _i, _f32p, _i, _f64p]
        L.orc_bias_act.argtypes = [_f32p, _f32p, _i64, _i64, _i, _f32p]
        L.orc_repack.argtypes = [_f32p, _i, _i, _i, _f32p, _f32p]
        L.orc_wg4_matrices.argtypes = [_f64p, _f64p, _f64p]
        L.orc_wg4_input.argtypes = [_f32p, _i, _i, _i, _i, _i, _i, _f32p]
        L.orc_wg4_madd.argtypes = [_f32p, _f32p, _i, _i, _i, _f32p, _i]
        L.orc_wg4_output.argtypes = [_f32p, _f32p, _i, _i, _i, _i, _i, _i, _f32p]
        L.orc_im2col.argtypes = [_f32p] + [_i64] * 10 + [_i] * 6 + [_f32p]
        L.orc_msdeform.argtypes = [_f32p, _f32p, _f32p, _f32p, _i, _f32p, _i]
        L.orc_mask_box.argtypes = [_f32p, _i, _f32p]
        L.orc_topk.argtypes = [_f32p, _i, _i, _i, _i32p]
        _lib = L
    return _lib


def _p(a, t=_f32p):
    return None if a is None else a.ctypes.data_as(t)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def conv_out_hw(IH, IW, K, S, P):
    return (IH + 2 * P - K) // S + 1, (IW + 2 * P - K) // S + 1


def conv2d_ref(x, w, bias, stride=1, pad=0, act=0, nthreads=0):
    """Reference CPU conv path: im2col F32 + k-ordered FP32 dot + bias + act."""
    x, w = _f32(x), _f32(w)
    bias = None if bias is None else _f32(bias)
    IC, IH, IW = x.shape
    OC, IC2, K, K2 = w.shape
    assert IC == IC2 and K == K2
    OH, OW = conv_out_hw(IH, IW, K, stride, pad)
    out = np.empty((OC, OH, OW), np.float32)
    lib().orc_conv2d_ref(_p(x), IC, IH, IW, _p(w), OC, K, stride, pad, _p(bias), act, _p(out), nthreads)
    return out


def conv2d_f64(x, w, bias, stride=1, pad=0, act=0):
    """Float64 direct cross-correlation (+bias, act): the closed-form truth."""
    x, w = _f32(x), _f32(w)
    bias = None if bias is None else _f32(bias)
    IC, IH, IW = x.shape
    OC, _, K, _ = w.shape
    OH, OW = conv_out_hw(IH, IW, K, stride, pad)
    out = np.empty((OC, OH, OW), np.float64)
    lib().orc_conv2d_f64(_p(x), IC, IH, IW, _p(w), OC, K, stride, pad, _p(bias), act, _p(out, _f64p))
    return out


def bias_act(x, bias, act):
    """Op 5 on an (C, H, W) tensor."""
    x, bias = _f32(x), _f32(bias)
    out = np.empty_like(x)
    plane = x.shape[-1] * x.shape[-2]
    lib().orc_bias_act(_p(x), _p(bias), x.size, plane, act, _p(out))
    return out


def repack(w):
    """(wr [K*K][IC][OC], wg4 [36][IC][OC] or None) for an OIHW weight."""
    w = _f32(w)
    OC, IC, K, _ = w.shape
    wr = np.empty((K * K, IC, OC), np.float32)
    wg4 = np.empty((36, IC, OC), np.float32) if K == 3 else None
    lib().orc_repack(_p(w), OC, IC, K, _p(wr), _p(wg4))
    return wr, wg4


def wg4_matrices():
    Bt, G, At = np.empty(36), np.empty(18), np.empty(24)
    lib().orc_wg4_matrices(_p(Bt, _f64p), _p(G, _f64p), _p(At, _f64p))
    return Bt.reshape(6, 6), G.reshape(6, 3), At.reshape(4, 6)


def wg4_tiles(H, W):
    """(TW, TH) of the F(4,3) tile grid covering an H x W output."""
    return (W + 3) // 4, (H + 3) // 4


def wg4_input(x, TW, TH, pad):
    x = _f32(x)
    IC, IH, IW = x.shape
    dt = np.empty((36, IC, TW * TH), np.float32)
    lib().orc_wg4_input(_p(x), IW, IH, IC, TW, TH, pad, _p(dt))
    return dt


def wg4_madd(dt, wg4, nthreads=0):
    dt, wg4 = _f32(dt), _f32(wg4)
    _, IC, T = dt.shape
    OC = wg4.shape[2]
    yt = np.empty((36, OC, T), np.float32)
    lib().orc_wg4_madd(_p(dt), _p(wg4), T, IC, OC, _p(yt), nthreads)
    return yt


def wg4_output(yt, bias, TW, TH, OH, OW, act):
    yt, bias = _f32(yt), _f32(bias)
    OC = yt.shape[1]
    out = np.empty((OC, OH, OW), np.float32)
    lib().orc_wg4_output(_p(yt), _p(bias), TW, TH, OC, OW, OH, act, _p(out))
    return out


def winograd_conv(x, w, bias, act):
    """k3 s1 p1 conv through the oracle's F(4,3) pipeline (pad fused)."""
    IC, H, W = x.shape
    TW, TH = wg4_tiles(H, W)
    _, wg4 = repack(w)
    dt = wg4_input(x, TW, TH, 1)
    yt = wg4_madd(dt, wg4)
    return wg4_output(yt, bias, TW, TH, H, W, act)


def im2col(x, K, S, P, OH, OW, KH=None, d=1):
    """ggml F32 im2col of one CHW image: (OH*OW, IC*KH*KW)."""
    x = _f32(x)
    IC, IH, IW = x.shape
    KH = K if KH is None else KH
    dst = np.empty((OH * OW, IC * KH * K), np.float32)
    lib().orc_im2col(_p(x), IW, IH, OW, OH, K, KH, IC, 1, IH * IW, IC * IH * IW, S, S, P, P, d, d, _p(dst))
    return dst


def msdeform(val, off, awr, ref, nthreads=0):
    """Op 2: val (13125, 256), off (NQ, 192), awr (NQ, 96), ref (NQ, 4) -> (NQ, 256)."""
    val, off, awr, ref = _f32(val), _f32(off), _f32(awr), _f32(ref)
    nq = ref.shape[0]
    out = np.empty((nq, 256), np.float32)
    lib().orc_msdeform(_p(val), _p(off), _p(awr), _p(ref), nq, _p(out), nthreads)
    return out


def mask_box(ml):
    """Op 1: ml (NQ, 40000) -> (NQ, 4)."""
    ml = _f32(ml)
    nq = ml.shape[0]
    out = np.empty((nq, 4), np.float32)
    lib().orc_mask_box(_p(ml), nq, _p(out))
    return out


def topk(logits, nq):
    """Op 13: logits (NTOK, NC) -> int32 (nq,)."""
    logits = _f32(logits)
    ntok, nc = logits.shape
    out = np.empty((nq,), np.int32)
    lib().orc_topk(_p(logits), ntok, nc, nq, _p(out, _i32p))
    return out
