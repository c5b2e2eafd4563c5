"""Host-side checks of the C-ABI library (no GPU needed, nothing is launched).

The library must load, export every symbol include/*.h declares, reject
malformed nodes before touching a device, and its host-only helpers (weight
repack, Winograd matrices) must agree with the oracle.
"""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        names |= set(re.findall(r"PPDL_\w*API\s+[\w\s\*]*?\b(ppdl_\w+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = declared_symbols()
    assert {"ppdl_hip_supports", "ppdl_hip_run", "ppdl_hip_im2col_f32", "ppdl_hip_repack_conv",
            "ppdl_hip_wg4_matrices"} <= names


def test_library_exports_every_declared_symbol(hip):
    lib = ctypes.CDLL(hip.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert set(hip.EXPORTS) <= declared_symbols()


def test_supports_id_only(hip):
    for op in (hip.OP_MSDEF, hip.OP_BIASACT, hip.OP_WG4_INPUT, hip.OP_WG4_OUTPUT, hip.OP_WG4_MADD,
               hip.OP_MASKBOX, hip.OP_TOPK, hip.OP_CONV1X1_BA, hip.OP_WG4_INPUT_PAD, hip.OP_CONV_IM2COL,
               hip.OP_WG4_CONV):
        assert hip.supports(op) == 1, op
    assert hip.supports(hip.OP_CONV, 1) == 1      # K=1 carried
    assert hip.supports(hip.OP_CONV, 3 | (1 << 8)) == 0  # legacy k3 tap-GEMM: not carried
    for op in (4, 6, 7, 8, 9, 0, 99):
        assert hip.supports(op) == 0, op
    p = hip.params(hip.OP_MSDEF)
    p[12] = 0x1234
    assert hip.lib().ppdl_hip_supports(p, None, None, 0) == 0


FAKE = 0x1000  # never dereferenced: validation rejects these nodes first


def test_run_rejects_bad_nodes_without_launching(hip):
    v = lambda ne, ty=hip.TYPE_F32: hip.raw_view(FAKE, ne, ty)  # noqa: E731
    # wrong magic / unknown id -> unsupported
    d = v([4, 4, 8])
    arr = (hip.TView * 1)(v([4, 4, 8]))
    p = hip.params(hip.OP_BIASACT)
    p[12] = 7
    assert hip.lib().ppdl_hip_run(p, ctypes.byref(d), arr, 1, None) == hip.UNSUPPORTED
    assert hip.run(42, v([4]), [v([4])], stream=0) == hip.UNSUPPORTED
    # 1x1 conv with mismatched IC
    assert hip.run(hip.OP_CONV1X1_BA, v([10, 10, 8]), [v([10, 10, 16]), v([8, 12, 1]), v([8])],
                   0, stream=0) == hip.EINVAL
    # bad activation code
    assert hip.run(hip.OP_CONV1X1_BA, v([10, 10, 8]), [v([10, 10, 16]), v([8, 16, 1]), v([8])],
                   7, stream=0) == hip.EINVAL
    # op 3 with pad != 0
    assert hip.run(hip.OP_CONV, v([10, 10, 8]), [v([10, 10, 16]), v([8, 16, 1]), v([8])],
                   1 | (1 << 8), stream=0) == hip.EINVAL
    # winograd input: padded frame too small for the tile grid
    assert hip.run(hip.OP_WG4_INPUT, v([25, 16, 36]), [v([21, 21, 16])], 25, 5, stream=0) == hip.EINVAL
    # winograd input: T not divisible by TH
    assert hip.run(hip.OP_WG4_INPUT, v([25, 16, 36]), [v([22, 22, 16])], 25, 4, stream=0) == hip.EINVAL
    # winograd madd: IC mismatch
    assert hip.run(hip.OP_WG4_MADD, v([25, 8, 36]), [v([25, 16, 36]), v([8, 12, 36])], stream=0) == hip.EINVAL
    # winograd output: wrong TW param
    assert hip.run(hip.OP_WG4_OUTPUT, v([20, 20, 8]), [v([25, 8, 36]), v([8])], 0, 4, stream=0) == hip.EINVAL
    # fused winograd conv: weight planes, bias length, act, params[15]
    good17 = [v([20, 20, 8]), v([16, 8, 36]), v([16])]
    assert hip.supports(hip.OP_WG4_CONV, 1, 0, v([20, 20, 16]), good17) == 1
    assert hip.run(hip.OP_WG4_CONV, v([20, 20, 16]), [v([20, 20, 8]), v([16, 8, 16]), v([16])], 1, stream=0) == hip.EINVAL
    assert hip.run(hip.OP_WG4_CONV, v([20, 20, 16]), [v([20, 20, 8]), v([16, 8, 36]), v([15])], 1, stream=0) == hip.EINVAL
    assert hip.run(hip.OP_WG4_CONV, v([20, 20, 16]), good17, 3, stream=0) == hip.EINVAL
    assert hip.run(hip.OP_WG4_CONV, v([20, 20, 16]), good17, 1, 1, stream=0) == hip.EINVAL
    assert hip.run(hip.OP_WG4_CONV, v([20, 19, 16]), good17, 1, stream=0) == hip.EINVAL
    assert hip.workspace_bytes(hip.OP_WG4_CONV, v([20, 20, 16]), good17, 1) == 0
    # im2col conv: dst shape inconsistent with K/S/P
    assert hip.run(hip.OP_CONV_IM2COL, v([50, 50, 8]), [v([100, 100, 4]), v([8, 4, 9]), v([8])],
                   3 | (1 << 8) | (1 << 16), stream=0) == hip.EINVAL
    # msdeform: wrong token count
    assert hip.run(hip.OP_MSDEF, v([256, 300]), [v([256, 13000]), v([192, 300]), v([96, 300]), v([4, 300])],
                   stream=0) == hip.EINVAL
    # topk: dst must be I32, and nq <= 512
    assert hip.run(hip.OP_TOPK, v([300]), [v([25, 13125])], stream=0) == hip.EINVAL
    assert hip.run(hip.OP_TOPK, v([600], hip.TYPE_I32), [v([25, 13125])], stream=0) == hip.EINVAL
    # non-contiguous stride
    bad = v([10, 10, 8])
    bad.nb[1] = 44
    assert hip.run(hip.OP_BIASACT, bad, [v([10, 10, 8]), v([8])], stream=0) == hip.EINVAL
    # null data
    assert hip.run(hip.OP_BIASACT, hip.raw_view(0, [4]), [v([4]), v([1])], stream=0) == hip.EINVAL


def test_wg4_ops_require_the_matrix_set_tag(hip):
    """Ops 10/11/12/15/17 return EINVAL unless op_params[11] carries
    PPDL_WG4_SET (the caller's .wg4 came from this library's repack); the
    other ops ignore slot 11."""
    import ctypes
    v = lambda ne: hip.raw_view(FAKE, ne)  # noqa: E731
    cases = [
        (hip.OP_WG4_INPUT, v([25, 16, 36]), [v([22, 22, 16])], 25, 5),
        (hip.OP_WG4_INPUT_PAD, v([25, 16, 36]), [v([20, 20, 16])], 25, 5),
        (hip.OP_WG4_MADD, v([25, 8, 36]), [v([25, 16, 36]), v([8, 16, 36])], 0, 0),
        (hip.OP_WG4_OUTPUT, v([20, 20, 8]), [v([25, 8, 36]), v([8])], 0, 5),
        (hip.OP_WG4_CONV, v([20, 20, 16]), [v([20, 20, 8]), v([16, 8, 36]), v([16])], 1, 0),
    ]
    L = hip.lib()
    for op, d, srcs, p14, p15 in cases:
        dd, arr, n = hip._views(d, srcs)
        assert L.ppdl_hip_supports(hip.params(op, p14, p15), ctypes.byref(dd), arr, n) == 1, op
        assert L.ppdl_hip_supports(hip.params(op, p14, p15, wg4_set=False), ctypes.byref(dd), arr, n) == 0, op
        assert L.ppdl_hip_run(hip.params(op, p14, p15, wg4_set=False), ctypes.byref(dd), arr, n, None) == hip.EINVAL
    # a non-Winograd op is indifferent to the tag
    dd, arr, n = hip._views(v([10, 10, 8]), [v([10, 10, 16]), v([8, 16, 1]), v([8])])
    assert L.ppdl_hip_supports(hip.params(hip.OP_CONV1X1_BA, 1, 0, wg4_set=False), ctypes.byref(dd), arr, n) == 1


def test_supports_with_views_uses_the_same_validation(hip):
    v = lambda ne: hip.raw_view(FAKE, ne)  # noqa: E731
    good = (v([10, 10, 8]), [v([10, 10, 16]), v([8, 16, 1]), v([8])])
    assert hip.supports(hip.OP_CONV1X1_BA, 1, 0, *good) == 1
    assert hip.supports(hip.OP_CONV1X1_BA, 1, 0, v([10, 10, 9]), good[1]) == 0


def test_conv1x1_accepts_plane_strided_maps(hip):
    """Ops 3 / 14 take CHW maps whose channel planes are padded (nb[2] >
    4*W*H, rows packed); an added map must share dst's layout."""
    def pv(W, H, C, ld):
        t = hip.raw_view(FAKE, [W, H, C])
        t.nb[2] = 4 * ld
        t.nb[3] = t.nb[2] * C
        return t
    w, b = hip.raw_view(FAKE, [8, 16, 1]), hip.raw_view(FAKE, [8])
    assert hip.supports(hip.OP_CONV1X1_BA, 1, 0, pv(25, 25, 8, 628), [pv(25, 25, 16, 628), w, b]) == 1
    assert hip.supports(hip.OP_CONV, 1, 0, pv(25, 25, 8, 628), [pv(25, 25, 16, 625), w]) == 1
    assert hip.supports(hip.OP_CONV1X1_BA, 1, 2, pv(25, 25, 8, 628), [pv(25, 25, 16, 628), w, b, pv(25, 25, 8, 628)]) == 1
    # the added map laid out differently from dst
    assert hip.supports(hip.OP_CONV1X1_BA, 1, 2, pv(25, 25, 8, 628), [pv(25, 25, 16, 628), w, b, pv(25, 25, 8, 625)]) == 0
    # planes overlapping (stride below W*H), padded rows, odd byte strides
    assert hip.supports(hip.OP_CONV1X1_BA, 1, 0, pv(25, 25, 8, 624), [pv(25, 25, 16, 628), w, b]) == 0
    bad = pv(25, 25, 16, 700)
    bad.nb[1] = 104
    assert hip.supports(hip.OP_CONV1X1_BA, 1, 0, pv(25, 25, 8, 628), [bad, w, b]) == 0
    odd = pv(25, 25, 16, 628)
    odd.nb[2] = 4 * 628 + 2
    assert hip.supports(hip.OP_CONV1X1_BA, 1, 0, pv(25, 25, 8, 628), [odd, w, b]) == 0


def test_im2col_rejects_out_of_range_args(hip):
    assert hip.im2col_f32(FAKE, FAKE, 8, 8, 8, 8, 3, 3, 4, 1, 64, 256, 0, 1, 1, 1, 1, 1, stream=0) == 0
    assert hip.im2col_f32(0, FAKE, 8, 8, 8, 8, 3, 3, 4, 1, 64, 256, 1, 1, 1, 1, 1, 1, stream=0) == 0


def test_repack_matches_oracle(hip, orc):
    rng = np.random.default_rng(1)
    for OC, IC, K in [(7, 5, 3), (16, 8, 1), (4, 3, 2)]:
        w = rng.standard_normal((OC, IC, K, K)).astype(np.float32)
        wr, wg4 = hip.repack_conv(w)
        owr, owg4 = orc.repack(w)
        assert np.array_equal(wr, owr)
        if K == 3:
            assert np.array_equal(wg4, owg4)
        else:
            assert wg4 is None


def test_wg4_matrices_match_oracle(hip, orc):
    for a, b in zip(hip.wg4_matrices(), orc.wg4_matrices()):
        assert np.array_equal(a, b)


def test_repack_rejects_bad_args(hip):
    f32p = ctypes.POINTER(ctypes.c_float)
    w = np.zeros(9, np.float32)
    out = np.zeros(36, np.float32)
    L = hip.lib()
    assert L.ppdl_hip_repack_conv(w.ctypes.data_as(f32p), 1, 1, 0, out.ctypes.data_as(f32p), None) == hip.EINVAL
    assert L.ppdl_hip_repack_conv(w.ctypes.data_as(f32p), 1, 1, 2, out.ctypes.data_as(f32p),
                                  out.ctypes.data_as(f32p)) == hip.EINVAL


@pytest.mark.parametrize("src", sorted(glob.glob(os.path.join(ROOT, "ppdoclayout-ggml_amd", "csrc", "*"))))
def test_no_cuda_compat_layer(src):
    text = open(src).read()
    for banned in ("__HIP_PLATFORM_NVIDIA__", "cuda_runtime", "#ifdef __CUDACC__", "hipify"):
        assert banned not in text, (src, banned)


def test_workspace_query_is_host_only(hip, monkeypatch):
    v = lambda ne: hip.raw_view(FAKE, ne)  # noqa: E731
    # a plan pinned to 4 K splits asks for 4 fp32 partial planes
    monkeypatch.setenv("PPDL_GEMM_TILE", "3,4")
    big = hip.workspace_bytes(hip.OP_CONV1X1_BA, v([25, 25, 1024]), [v([25, 25, 3328]), v([1024, 3328, 1]), v([1024])], 1)
    assert big == 4 * 1024 * 625 * 4
    # a workspace already attached is ignored by the query
    again = hip.workspace_bytes(hip.OP_CONV1X1_BA, v([25, 25, 1024]),
                                [v([25, 25, 3328]), v([1024, 3328, 1]), v([1024]), v([big // 4])], 1)
    assert again == big
    # tiny GEMM (one k tile): no split even when asked
    assert hip.workspace_bytes(hip.OP_CONV1X1_BA, v([4, 4, 8]), [v([4, 4, 8]), v([8, 8, 1]), v([8])], 0) == 0
    # non-GEMM op: none; invalid node: -1
    assert hip.workspace_bytes(hip.OP_BIASACT, v([4, 4, 8]), [v([4, 4, 8]), v([8])], 0) == 0
    assert hip.workspace_bytes(hip.OP_CONV1X1_BA, v([4, 4, 9]), [v([4, 4, 8]), v([8, 8, 1]), v([8])], 0) == -1


def test_noalloc_rejects_on_the_host(hip, monkeypatch):
    """ppdl_hip_run_noalloc validates like ppdl_hip_run, refuses an attached
    workspace src and a plan larger than its scratch array, all before any
    device call (FAKE pointers are never dereferenced)."""
    v = lambda ne: hip.raw_view(FAKE, ne)  # noqa: E731
    L = hip.lib()

    def call(op, dst, srcs, p14=0, p15=0):
        d, arr, n = hip._views(dst, srcs)
        return L.ppdl_hip_run_noalloc(hip.params(op, p14, p15), ctypes.byref(d), arr, n, None)

    srcs = [v([25, 25, 4096]), v([1024, 4096, 1]), v([1024])]
    assert call(hip.OP_CONV1X1_BA, v([25, 25, 1023]), srcs) == hip.EINVAL  # shape mismatch
    assert call(42, v([4]), [v([4])]) == hip.UNSUPPORTED
    assert call(hip.OP_CONV1X1_BA, v([25, 25, 1024]), srcs + [v([1 << 20])]) == hip.EINVAL  # workspace src
    monkeypatch.setenv("PPDL_GEMM_TILE", "3,16")  # 16 x 1024 x 625 fp32 partials: 41 MB
    assert hip.workspace_bytes(hip.OP_CONV1X1_BA, v([25, 25, 1024]), srcs) > hip.NOALLOC_SCRATCH_BYTES
    assert call(hip.OP_CONV1X1_BA, v([25, 25, 1024]), srcs) == hip.EINVAL


def test_misaligned_workspace_rejected(hip):
    v = lambda ne, p=FAKE: hip.raw_view(p, ne)  # noqa: E731
    srcs = [v([25, 25, 64]), v([32, 64, 1]), v([32]), v([1024], FAKE + 4)]
    assert hip.run(hip.OP_CONV1X1_BA, v([25, 25, 32]), srcs, 0, stream=0) == hip.EINVAL


# ---------------------------------------------------------------- CLI (no GPU work)
CLI = os.path.join(ROOT, "ppdoclayout-ggml_amd", "lib", "ppdoclayout")


@pytest.mark.skipif(not os.path.exists(CLI), reason="CLI not built (make -C ppdoclayout-ggml_amd)")
def test_cli_argument_handling(tmp_path):
    import subprocess

    r = subprocess.run([CLI], capture_output=True, text=True)
    assert r.returncode == 1 and "usage:" in r.stderr
    r = subprocess.run([CLI, "-i", "x.bin", "--bogus", "1"], capture_output=True, text=True)
    assert r.returncode == 1 and "unknown arg" in r.stderr
    r = subprocess.run([CLI, "-i", "x.bin", "--backend", "cpu"], capture_output=True, text=True)
    assert r.returncode == 1 and "not available" in r.stderr
    r = subprocess.run([CLI, "-i"], capture_output=True, text=True)
    assert r.returncode == 1 and "missing value" in r.stderr
