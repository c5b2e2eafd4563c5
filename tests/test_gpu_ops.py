"""GPU parity of every tagged op, called through the C-ABI (libppdl_hip.so).

Each test runs the HIP path on seeded inputs and compares it with the CPU
oracle on the same inputs:
  * conv outputs (1x1 GEMM, Winograd F(4,3), implicit-im2col GEMM) and the
    MSDeformAttn sampler: normwise max|y-ref|/max|ref| <= 2e-5 (the per-op
    FP32 budget), plus the float64 truth where the size allows;
  * Winograd input transform, im2col, top-k: bit-exact (same arithmetic or
    pure data movement); output transform bit-exact without SiLU.
Sizes include every benchmark configuration (1x1 512->256 @100^2, the Winograd sweep,
the im2col convs, MSDeformAttn at 300 queries) plus ragged edge shapes.
"""
import os
import sys

import numpy as np
import pytest
import torch
from conftest import normwise, rel1

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLD)
from fixture_inputs import msdef_value_map  # noqa: E402

TOL = 2e-5
SEED = 0x5050444C


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module", autouse=True)
def device():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    torch.cuda.set_device(0)
    yield


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def conv_inputs(rng, IC, H, W, OC, K):
    x = rng.random((IC, H, W)).astype(np.float32)
    w = (rng.standard_normal((OC, IC, K, K)) / np.sqrt(K * K * IC)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, OC).astype(np.float32)
    return x, w, b


# ---------------------------------------------------------------- HIP paths
def with_ws(hip, op, dst, srcs, p14=0, p15=0, use_ws=True):
    """srcs plus the split-K workspace the op's plan asks for (if any)."""
    if not use_ws:
        return list(srcs)
    nb = hip.workspace_bytes(op, dst, srcs, p14, p15)
    assert nb >= 0
    return list(srcs) + ([hip.make_workspace(nb)] if nb > 0 else [])


def hip_conv1x1(hip, x, w, b, act, use_ws=True):
    wr, _ = hip.repack_conv(w)
    OC = w.shape[0]
    xt, wt, bt = dev(x), dev(wr), dev(b)
    out = torch.empty((OC,) + x.shape[1:], device="cuda")
    srcs = with_ws(hip, hip.OP_CONV1X1_BA, out, [xt, wt, bt], act, 0, use_ws)
    hip.run_checked(hip.OP_CONV1X1_BA, out, srcs, act)
    return out, (xt, wt, bt)


def hip_winograd(hip, x, w, b, act, prepadded=False, use_ws=True):
    IC, H, W = x.shape
    OC = w.shape[0]
    TW, TH = (W + 3) // 4, (H + 3) // 4
    T = TW * TH
    _, wg4 = hip.repack_conv(w)
    wt, bt = dev(wg4), dev(b)
    dt = torch.empty((36, IC, T), device="cuda")
    yt = torch.empty((36, OC, T), device="cuda")
    out = torch.empty((OC, H, W), device="cuda")
    if prepadded:
        xp = np.zeros((IC, 4 * TH + 2, 4 * TW + 2), np.float32)
        xp[:, 1:H + 1, 1:W + 1] = x
        hip.run_checked(hip.OP_WG4_INPUT, dt, [dev(xp)], T, TH)
    else:
        hip.run_checked(hip.OP_WG4_INPUT_PAD, dt, [dev(x)], T, TH)
    hip.run_checked(hip.OP_WG4_MADD, yt, with_ws(hip, hip.OP_WG4_MADD, yt, [dt, wt], use_ws=use_ws))
    hip.run_checked(hip.OP_WG4_OUTPUT, out, [yt, bt], act, TW)
    return out, dt, yt, wg4


def planes_view(hip, t, T, C):
    """ppdl_tview ne(T, C, 36) over a torch (36, C, ldt) buffer: rows padded."""
    ldt = t.shape[2]
    v = hip.TView()
    v.data = t.data_ptr()
    for i, (n, b) in enumerate(zip((T, C, 36, 1), (4, ldt * 4, ldt * 4 * C, ldt * 4 * C * 36))):
        v.ne[i], v.nb[i] = n, b
    v.type = hip.TYPE_F32
    return v


def hip_winograd_padded(hip, x, w, b, act, ldt):
    """ops 15 -> 12 -> 11 with dt / yt plane rows padded to ldt (padding NaN)."""
    IC, H, W = x.shape
    OC = w.shape[0]
    TW, TH = (W + 3) // 4, (H + 3) // 4
    T = TW * TH
    _, wg4 = hip.repack_conv(w)
    dt = torch.full((36, IC, ldt), float("nan"), device="cuda")
    yt = torch.full((36, OC, ldt), float("nan"), device="cuda")
    out = torch.empty((OC, H, W), device="cuda")
    vdt, vyt = planes_view(hip, dt, T, IC), planes_view(hip, yt, T, OC)
    hip.run_checked(hip.OP_WG4_INPUT_PAD, vdt, [dev(x)], T, TH)
    srcs = [vdt, dev(wg4)]
    nb = hip.workspace_bytes(hip.OP_WG4_MADD, vyt, srcs)
    if nb > 0:
        srcs.append(hip.make_workspace(nb))
    hip.run_checked(hip.OP_WG4_MADD, vyt, srcs)
    hip.run_checked(hip.OP_WG4_OUTPUT, out, [vyt, dev(b)], act, TW)
    return out, dt


def hip_conv_im2col(hip, x, w, b, K, S, P, act, use_ws=True):
    wr, _ = hip.repack_conv(w)
    IC, IH, IW = x.shape
    OC = w.shape[0]
    OH, OW = (IH + 2 * P - K) // S + 1, (IW + 2 * P - K) // S + 1
    out = torch.empty((OC, OH, OW), device="cuda")
    p14 = K | (S << 8) | (P << 16) | (act << 24)
    srcs = with_ws(hip, hip.OP_CONV_IM2COL, out, [dev(x), dev(wr), dev(b)], p14, 0, use_ws)
    hip.run_checked(hip.OP_CONV_IM2COL, out, srcs, p14)
    return out


# ---------------------------------------------------------------- 1x1 conv
def test_conv1x1_512_256_100(hip, orc):
    say("1x1 512->256 @100x100 relu")
    rng = np.random.default_rng(SEED + 1)
    x, w, b = conv_inputs(rng, 512, 100, 100, 256, 1)
    out, (xt, wt, bt) = hip_conv1x1(hip, x, w, b, 1)
    y = host(out)
    ref = orc.conv2d_ref(x, w, b, 1, 0, 1)
    assert normwise(y, ref) < TOL, normwise(y, ref)
    # op 3 (GEMM) then op 5 (bias+act) reproduces the fused op bit for bit
    # when both run the same GEMM plan (same split-K summation order)
    g = torch.empty_like(out)
    r = torch.empty_like(out)
    hip.run_checked(hip.OP_CONV, g, with_ws(hip, hip.OP_CONV, g, [xt, wt, bt], 1), 1)
    hip.run_checked(hip.OP_BIASACT, r, [g, bt], 1)
    assert np.array_equal(host(r), y)
    # op 3 alone is the bias-free GEMM
    assert normwise(host(g), orc.conv2d_ref(x, w, None, 1, 0, 0)) < TOL


@pytest.mark.parametrize("IC,H,W,OC", [
    (1, 1, 1, 1), (3, 7, 5, 2), (17, 13, 11, 33), (64, 25, 25, 200), (48, 40, 40, 24),
    (336, 25, 25, 64), (2176, 7, 9, 40), (32, 200, 200, 48), (5, 3, 300, 130),
])
@pytest.mark.parametrize("act", [0, 1, 2])
def test_conv1x1_shapes(hip, orc, IC, H, W, OC, act):
    say(f"1x1 {IC}->{OC} @{H}x{W} act{act}")
    rng = np.random.default_rng(IC * 7 + H * 3 + W + OC + act)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 1)
    out, _ = hip_conv1x1(hip, x, w, b, act)
    y = host(out)
    assert normwise(y, orc.conv2d_ref(x, w, b, 1, 0, act)) < TOL
    assert normwise(y, orc.conv2d_f64(x, w, b, 1, 0, act)) < TOL


@pytest.mark.parametrize("IC,H,W,OC,ld", [(3328, 25, 25, 1024, 628), (1024, 25, 25, 2048, 628), (40, 5, 7, 12, 37),
                                          (384, 25, 25, 384, 640)])
def test_conv1x1_plane_strided(hip, orc, IC, H, W, OC, ld):
    """Op 14 on maps whose channel planes are ld floats apart (the 25x25
    maps of stage 3 use 628 so that GEMM B rows are whole float4s): the
    result equals the packed-map conv, with and without an added map, and
    the padding columns of dst stay untouched.  With ld % 4 == 0 the
    stage-3 aggregation GEMMs take the direct-to-LDS loader."""
    say(f"1x1 plane-strided {IC}->{OC} @{H}x{W} ld {ld}")
    rng = np.random.default_rng(IC + OC + ld)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 1)
    wr, _ = hip.repack_conv(w)
    P = H * W
    xs = torch.full((IC, ld), float("nan"), device="cuda")
    xs[:, :P] = dev(x.reshape(IC, P))
    add = rng.standard_normal((OC, P)).astype(np.float32)
    adds = torch.full((OC, ld), float("nan"), device="cuda")
    adds[:, :P] = dev(add)
    ref = orc.conv2d_ref(x, w, b, 1, 0, 1).reshape(OC, P)
    for mode in (0, 2):
        out = torch.full((OC, ld), float("nan"), device="cuda")
        srcs = [hip.chw_view(xs, W, H), dev(wr), dev(b)] + ([hip.chw_view(adds, W, H)] if mode else [])
        d = hip.chw_view(out, W, H)
        srcs = with_ws(hip, hip.OP_CONV1X1_BA, d, srcs, 1, mode, True)
        if ld % 4 == 0 and IC >= 1024:  # the stage-3 aggregations: a float4 B loader
            assert hip.kernel_name(hip.OP_CONV1X1_BA, d, srcs, 1, mode).startswith(("k_gemm_dma", "k_gemm_lt"))
        hip.run_checked(hip.OP_CONV1X1_BA, d, srcs, 1, mode)
        y = host(out)
        assert np.isnan(y[:, P:]).all()
        assert normwise(y[:, :P], ref + add if mode else ref) < TOL


def lt_menu(hip, op, dst, srcs, p14=0, p15=0):
    """Indices of the 16x16-MFMA GEMM menu, read back through the kernel
    names that PPDL_LT=<index> selects (an index past the menu falls back)."""
    idx = []
    for i in range(64):
        os.environ["PPDL_LT"] = str(i)
        try:
            if not hip.kernel_name(op, dst, srcs, p14, p15).startswith("k_gemm_lt"):
                break
        finally:
            os.environ.pop("PPDL_LT", None)
        idx.append(i)
    return idx


LT_SHAPES = [  # (IC, H, W, OC, plane stride or 0, act, add mode)
    (132, 9, 12, 52, 0, 2, 2),      # K not a multiple of the k tile, M and N not of the block
    (40, 5, 7, 12, 36, 1, 0),       # 35 pixels in planes 36 floats apart
    (1664, 50, 50, 512, 0, 1, 0),   # stage-2 aggregation: many k tiles, both loop halves
    (1024, 25, 25, 384, 628, 1, 2),  # stage-3 map with padded planes
]


@pytest.mark.parametrize("shape", LT_SHAPES)
def test_gemm_lt_menu_matches_oracle(hip, orc, shape, monkeypatch):
    """Every entry of the shape-fitted 16x16-MFMA GEMM menu, pinned with
    PPDL_LT=<index>, on 1x1 convs whose edges are ragged in M, N and K,
    with padded channel planes, bias + act and a residual add: the result
    matches the float64 oracle, padding columns stay untouched and repeated
    launches are bitwise identical."""
    IC, H, W, OC, ld, act, mode = shape
    P = H * W
    ld = ld or P
    say(f"gemm_lt menu 1x1 {IC}->{OC} @{H}x{W} ld {ld}")
    rng = np.random.default_rng(IC * 7 + OC)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 1)
    wr, _ = hip.repack_conv(w)
    xs = torch.full((IC, ld), float("nan"), device="cuda")
    xs[:, :P] = dev(x.reshape(IC, P))
    add = rng.standard_normal((OC, P)).astype(np.float32)
    adds = torch.full((OC, ld), float("nan"), device="cuda")
    adds[:, :P] = dev(add)
    ref = orc.conv2d_ref(x, w, b, 1, 0, act).reshape(OC, P) + (add if mode == 2 else 0)
    out = torch.full((OC, ld), float("nan"), device="cuda")
    d = hip.chw_view(out, W, H)
    srcs = [hip.chw_view(xs, W, H), dev(wr), dev(b)] + ([hip.chw_view(adds, W, H)] if mode else [])
    menu = lt_menu(hip, hip.OP_CONV1X1_BA, d, srcs, act, mode)
    assert len(menu) >= 8
    for i in menu:
        monkeypatch.setenv("PPDL_LT", str(i))
        runs = []
        for _ in range(2):
            out.fill_(float("nan"))
            hip.run_checked(hip.OP_CONV1X1_BA, d, srcs, act, mode)
            runs.append(host(out).copy())
        y = runs[0]
        assert np.array_equal(runs[0], runs[1], equal_nan=True), f"entry {i}: not deterministic"
        if ld > P:
            assert np.isnan(y[:, P:]).all(), f"entry {i}: wrote padding"
        assert normwise(y[:, :P], ref) < TOL, f"entry {i}"


def test_gemm_lt_menu_on_winograd_planes(hip, orc, monkeypatch):
    """The menu on op 12's batched products: 36 F(4,3) planes of 96 x 169 x
    96 with plane rows padded to 172 floats; the whole conv matches the
    oracle for every entry."""
    IC, H, W, OC = 96, 50, 50, 96
    rng = np.random.default_rng(12)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 3)
    ref = orc.conv2d_ref(x, w, b, 1, 1, 1)
    T = 13 * 13
    _, wg4 = hip.repack_conv(w)
    dt = torch.full((36, IC, 172), float("nan"), device="cuda")
    yt = torch.full((36, OC, 172), float("nan"), device="cuda")
    vdt, vyt = planes_view(hip, dt, T, IC), planes_view(hip, yt, T, OC)
    menu = lt_menu(hip, hip.OP_WG4_MADD, vyt, [vdt, dev(wg4)])
    assert len(menu) >= 8
    for i in menu:
        monkeypatch.setenv("PPDL_LT", str(i))
        say(f"gemm_lt menu F(4,3) planes entry {i}")
        out, _ = hip_winograd_padded(hip, x, w, b, 1, 172)
        assert normwise(host(out), ref) < TOL, f"entry {i}"


@pytest.mark.parametrize("wv", ["", "1", "2", "4", "8", "16"])
@pytest.mark.parametrize("IC,H,W,OC", [
    (1, 1, 1, 1), (3, 7, 5, 2), (17, 13, 11, 33), (256, 15, 20, 256), (1024, 17, 19, 96), (70, 9, 9, 300),
])
def test_small_gemm_kernel(hip, orc, IC, H, W, OC, wv, monkeypatch):
    """The small-GEMM kernel (32x32 tiles, K split over the block's 1 to 16
    waves; "" = the planner's choice from K) forced for every GEMM, on edge
    shapes: K not a multiple of the 32-wide chunk, fewer chunks than waves, M
    and N not multiples of 32."""
    monkeypatch.setenv("PPDL_GEMM_TILE", "6,1")
    monkeypatch.setenv("PPDL_SMALL_WV", wv)
    say(f"small GEMM 1x1 {IC}->{OC} @{H}x{W} waves {wv or 'auto'}")
    rng = np.random.default_rng(IC + 3 * OC + H)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 1)
    out, _ = hip_conv1x1(hip, x, w, b, 2)
    y = host(out)
    assert normwise(y, orc.conv2d_ref(x, w, b, 1, 0, 2)) < TOL
    # Winograd planes through the same kernel (batch 36)
    if IC <= 256 and H >= 5:
        x3, w3, b3 = conv_inputs(rng, IC, H, W, OC, 3)
        wo = hip_winograd(hip, x3, w3, b3, 1)[0]
        assert normwise(host(wo), orc.conv2d_ref(x3, w3, b3, 1, 1, 1)) < TOL


@pytest.mark.parametrize("IC,H,W", [(48, 200, 200), (5, 9, 12), (3, 4, 4), (7, 13, 8)])
def test_wg4_input_vector_loads(hip, orc, IC, H, W):
    """Op 15 on a 16-byte aligned image with W % 4 == 0 loads rows as float4 +
    halo scalars; a 4-byte offset copy of the same image takes the scalar
    path.  The transforms must agree bit for bit."""
    say(f"wg4 input vector vs scalar {IC} @{H}x{W}")
    x = np.random.default_rng(IC + H + W).standard_normal((IC, H, W)).astype(np.float32)
    TW, TH = (W + 3) // 4, (H + 3) // 4
    T = TW * TH
    buf = torch.zeros(IC * H * W + 4, device="cuda")
    outs = []
    for off in (0, 1):  # 0: aligned (vector path), 1: 4-byte offset (scalar path)
        xv = buf[off:off + IC * H * W].view(IC, H, W)
        xv.copy_(dev(x))
        assert (xv.data_ptr() % 16 == 0) == (off == 0)
        dt = torch.full((36, IC, T), float("nan"), device="cuda")
        hip.run_checked(hip.OP_WG4_INPUT_PAD, dt, [xv], T, TH)
        outs.append(host(dt))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0], orc.wg4_input(x, TW, TH, 1))


# ---------------------------------------------------------------- Winograd F(4,3)
@pytest.mark.parametrize("IC,H,W,OC", [(64, 100, 100, 48), (96, 50, 50, 96), (256, 25, 25, 256), (7, 9, 11, 5)])
def test_winograd_padded_planes(hip, orc, IC, H, W, OC):
    """dt / yt plane rows padded past T (NaN-filled padding): the padding is
    never read into a stored output (the result is finite), and the result
    equals the contiguous layout's bit for bit when both layouts run the same
    plane kernel (same summation order); padded rows whose width is whole
    float4s may select the float4-loading kernel instead, which then agrees
    within the tolerance."""
    say(f"F(4,3) padded planes {IC}->{OC} @{H}x{W}")
    rng = np.random.default_rng(IC + H + OC)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 3)
    T = ((W + 3) // 4) * ((H + 3) // 4)
    _, wg4 = hip.repack_conv(w)
    packed = hip.kernel_name(hip.OP_WG4_MADD, torch.empty((36, OC, T), device="cuda"),
                             [torch.empty((36, IC, T), device="cuda"), dev(wg4)])
    ref_out = host(hip_winograd(hip, x, w, b, 2)[0])
    for ldt in ((T + 3) // 4 * 4, T + 17):
        out, dt = hip_winograd_padded(hip, x, w, b, 2, ldt)
        y = host(out)
        assert np.isfinite(y).all()
        vdt = planes_view(hip, torch.empty((36, IC, ldt), device="cuda"), T, IC)
        vyt = planes_view(hip, torch.empty((36, OC, ldt), device="cuda"), T, OC)
        if hip.kernel_name(hip.OP_WG4_MADD, vyt, [vdt, dev(wg4)]) == packed:
            assert np.array_equal(y, ref_out), ldt
        else:
            assert normwise(y, ref_out) < TOL, ldt
        assert normwise(y, orc.conv2d_ref(x, w, b, 1, 1, 2)) < TOL
        if ldt > T:
            assert torch.isnan(dt[:, :, T:]).all().item()  # the input transform leaves the padding alone

WG_CONFIGS = [(256, 100, 100), (256, 50, 50), (256, 25, 25), (48, 200, 200), (96, 100, 100)]


@pytest.mark.parametrize("C,H,W", WG_CONFIGS)
def test_winograd_sweep(hip, orc, C, H, W):
    say(f"winograd {C}->{C} @{H}x{W} silu")
    rng = np.random.default_rng(SEED + 2 + C + H)
    x, w, b = conv_inputs(rng, C, H, W, C, 3)
    out, dt, yt, wg4 = hip_winograd(hip, x, w, b, 2)
    y = host(out)
    ref = orc.conv2d_ref(x, w, b, 1, 1, 2)
    e = normwise(y, ref)
    say(f"  normwise vs reference CPU conv path {e:.2e}")
    assert e < TOL
    TW, TH = (W + 3) // 4, (H + 3) // 4
    # per-op parity
    assert np.array_equal(host(dt), orc.wg4_input(x, TW, TH, 1)), "input transform must be bit-exact"
    yt_h = host(yt)
    assert normwise(yt_h, orc.wg4_madd(host(dt), wg4)) < TOL
    out_ref = orc.wg4_output(yt_h, b, TW, TH, H, W, 2)
    assert rel1(y, out_ref) < 1e-6


@pytest.mark.parametrize("IC,H,W,OC", [(3, 9, 10, 2), (1, 1, 1, 1), (5, 4, 4, 7), (8, 5, 6, 3),
                                       (33, 17, 23, 65), (128, 50, 50, 96), (64, 13, 200, 64)])
@pytest.mark.parametrize("act", [0, 1, 2])
def test_winograd_shapes(hip, orc, IC, H, W, OC, act):
    say(f"winograd {IC}->{OC} @{H}x{W} act{act}")
    rng = np.random.default_rng(IC + H * 5 + W * 7 + OC + act)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 3)
    out, dt, yt, _ = hip_winograd(hip, x, w, b, act)
    y = host(out)
    assert normwise(y, orc.conv2d_f64(x, w, b, 1, 1, act)) < TOL
    TW, TH = (W + 3) // 4, (H + 3) // 4
    out_ref = orc.wg4_output(host(yt), b, TW, TH, H, W, act)
    if act == 2:
        assert rel1(y, out_ref) < 1e-6
    else:
        assert np.array_equal(y, out_ref), "output transform must be bit-exact"
    # op 10 on a pre-padded frame == op 15 with the pad fused
    out2, dt2, _, _ = hip_winograd(hip, x, w, b, act, prepadded=True)
    assert np.array_equal(host(dt2), host(dt))
    assert np.array_equal(host(out2), y)


# ---------------------------------------------------------------- im2col convs
IM2COL_CONFIGS = [  # IC, IH, IW, OC, K, S, P
    (48, 401, 401, 24, 2, 1, 0),    # stem2a-like k2: input padded right/bottom to 401
    (256, 100, 100, 256, 3, 2, 1),
    (256, 50, 50, 256, 3, 2, 1),
    (3, 800, 800, 32, 3, 2, 1),
    (32, 401, 401, 16, 2, 1, 0),    # stem2a: one tap per k tile (IC % 32 == 0)
    (64, 400, 400, 32, 3, 2, 1),    # stem3: one tap per k tile
]


@pytest.mark.parametrize("IC,IH,IW,OC,K,S,P", IM2COL_CONFIGS)
@pytest.mark.parametrize("act", [0, 1, 2])
def test_conv_im2col_bench_shapes(hip, orc, IC, IH, IW, OC, K, S, P, act):
    say(f"im2col conv k{K}s{S}p{P} {IC}->{OC} @{IH}x{IW} act{act}")
    rng = np.random.default_rng(SEED + 3 + IC + IH + act)
    x, w, b = conv_inputs(rng, IC, IH, IW, OC, K)
    y = host(hip_conv_im2col(hip, x, w, b, K, S, P, act))
    e = normwise(y, orc.conv2d_ref(x, w, b, S, P, act))
    say(f"  normwise {e:.2e}")
    assert e < TOL


@pytest.mark.parametrize("IC,IH,IW,OC,K,S,P", [(1, 1, 1, 1, 1, 1, 0), (2, 5, 3, 3, 2, 1, 0), (7, 9, 8, 5, 3, 2, 1),
                                               (16, 33, 31, 70, 3, 2, 1), (4, 6, 6, 9, 5, 1, 2), (3, 2, 2, 4, 3, 1, 1),
                                               # IC >= 32: at most two taps per k tile, ragged M / N,
                                               # borders and (IC % 32 != 0) a ragged last k tile
                                               (32, 33, 31, 40, 3, 2, 1), (64, 17, 19, 20, 2, 1, 0),
                                               (32, 9, 9, 7, 3, 1, 1), (96, 5, 4, 33, 3, 1, 1),
                                               (40, 11, 13, 12, 3, 1, 1), (33, 9, 8, 5, 2, 1, 0),
                                               (48, 21, 22, 36, 3, 2, 1),
                                               # IC == 16: every k tile exactly two taps
                                               (16, 17, 15, 32, 2, 1, 0), (16, 9, 10, 20, 3, 2, 1)])
def test_conv_im2col_shapes(hip, orc, IC, IH, IW, OC, K, S, P):
    say(f"im2col conv edge k{K}s{S}p{P} {IC}->{OC} @{IH}x{IW}")
    rng = np.random.default_rng(IC + IH + IW + OC + K)
    x, w, b = conv_inputs(rng, IC, IH, IW, OC, K)
    y = host(hip_conv_im2col(hip, x, w, b, K, S, P, 1))
    assert normwise(y, orc.conv2d_f64(x, w, b, S, P, 1)) < TOL


@pytest.mark.parametrize("IC,IH,IW,OC,P", [(3, 800, 800, 32, 1), (3, 9, 7, 5, 1), (1, 5, 5, 32, 1), (4, 17, 33, 17, 0),
                                         (2, 3, 3, 1, 1), (3, 2, 1, 32, 1), (4, 6, 11, 30, 1)])
@pytest.mark.parametrize("act", [0, 1])
def test_conv_direct_kernel(hip, orc, IC, IH, IW, OC, P, act, monkeypatch):
    """Op 16 k3 s2 with IC <= 4 and OC <= 32 (the first stem conv) runs the
    direct VALU kernel: against float64, and against the MFMA fragment
    kernel it replaced (PPDL_CONV_DIRECT=0), odd widths included (the last
    pair's second pixel is not stored)."""
    say(f"direct conv k3s2p{P} {IC}->{OC} @{IH}x{IW} act{act}")
    rng = np.random.default_rng(IC * 7 + IH + IW + OC + act)
    x, w, b = conv_inputs(rng, IC, IH, IW, OC, 3)
    wr, _ = hip.repack_conv(w)
    OH, OW = (IH + 2 * P - 3) // 2 + 1, (IW + 2 * P - 3) // 2 + 1
    p14 = 3 | (2 << 8) | (P << 16) | (act << 24)
    outs = []
    for flag, kern in (("1", f"k_conv_k3s2<{IC}>"), ("0", "k_conv_frag<")):
        monkeypatch.setenv("PPDL_CONV_DIRECT", flag)
        out = torch.full((OC, OH, OW), float("nan"), device="cuda")
        srcs = [dev(x), dev(wr), dev(b)]
        assert hip.kernel_name(hip.OP_CONV_IM2COL, out, srcs, p14).startswith(kern)
        hip.run_checked(hip.OP_CONV_IM2COL, out, srcs, p14)
        outs.append(host(out))
    ref = orc.conv2d_f64(x, w, b, 2, P, act)
    assert np.isfinite(outs[0]).all()
    assert normwise(outs[0], ref) < TOL and normwise(outs[1], ref) < TOL


@pytest.mark.parametrize("IC,IH,IW,K,S,P", [(48, 401, 401, 2, 1, 0), (256, 100, 100, 3, 2, 1), (3, 800, 800, 3, 2, 1),
                                            (5, 7, 9, 3, 1, 1), (16, 10, 10, 1, 1, 0), (2, 3, 3, 3, 2, 1)])
def test_im2col_ggml_layout(hip, orc, IC, IH, IW, K, S, P):
    say(f"im2col ggml layout k{K}s{S}p{P} IC{IC} @{IH}x{IW}")
    rng = np.random.default_rng(IC + IH + K)
    x = rng.random((IC, IH, IW)).astype(np.float32)
    OH, OW = (IH + 2 * P - K) // S + 1, (IW + 2 * P - K) // S + 1
    d = torch.empty((OH * OW, IC * K * K), device="cuda")
    assert hip.im2col_f32(dev(x), d, IW, IH, OW, OH, K, K, IC, 1, IH * IW, IC * IH * IW, S, S, P, P, 1, 1) == 1
    assert np.array_equal(host(d), orc.im2col(x, K, S, P, OH, OW))


def test_conv_golden_fixtures_on_gpu(hip, orc):
    import glob
    for path in sorted(glob.glob(os.path.join(GOLD, "conv_*.npz"))):
        f = np.load(path)
        S, P, act = (int(v) for v in f["meta"])
        x, w, b = f["x"], f["w"], f["b"]
        K = w.shape[2]
        say(f"fixture {os.path.basename(path)}")
        if K == 1:
            y = host(hip_conv1x1(hip, x, w, b, act)[0])
        elif K == 3 and S == 1 and P == 1:
            y = host(hip_winograd(hip, x, w, b, act)[0])
        else:
            y = host(hip_conv_im2col(hip, x, w, b, K, S, P, act))
        assert normwise(y, f["y"]) < TOL, path


@pytest.mark.parametrize("IC,H,W,OC,K,S,P,PE", [
    (3, 800, 800, 32, 3, 2, 1, 0),     # stem1
    (32, 400, 400, 16, 2, 1, 0, 1),    # stem2a (zero pad after the last column / row)
    (64, 200, 200, 32, 3, 2, 1, 0),    # stem3: several channel chunks
    (37, 33, 150, 24, 3, 2, 1, 0),     # ragged: channel chunk remainder, partial row segment
    (5, 9, 7, 3, 2, 1, 0, 1),          # tiny
])
def test_conv_patch_kernel(hip, orc, IC, H, W, OC, K, S, P, PE, monkeypatch):
    """Op 16 with <= 32 output channels on the opt-in LDS-patch kernel
    (PPDL_CONV_PATCH=1): against the oracle, and against the default generic
    implicit-im2col loader (PPDL_CONV_PATCH=0)."""
    say(f"patch conv {IC}->{OC} k{K}s{S} @{H}x{W} pe{PE}")
    rng = np.random.default_rng(IC * 31 + OC + H)
    x, w, b = conv_inputs(rng, IC, H, W, OC, K)
    wr, _ = hip.repack_conv(w)
    OH, OW = (H + 2 * P + PE - K) // S + 1, (W + 2 * P + PE - K) // S + 1
    p14 = K | (S << 8) | (P << 16) | (1 << 24)
    outs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("PPDL_CONV_PATCH", flag)
        out = torch.full((OC, OH, OW), float("nan"), device="cuda")
        srcs = with_ws(hip, hip.OP_CONV_IM2COL, out, [dev(x), dev(wr), dev(b)], p14, PE, True)
        hip.run_checked(hip.OP_CONV_IM2COL, out, srcs, p14, PE)
        outs.append(host(out))
    xp = np.pad(x, ((0, 0), (0, PE), (0, PE))) if PE else x
    ref = orc.conv2d_ref(xp, w, b, S, P, 1)
    assert np.isfinite(outs[0]).all()
    assert normwise(outs[0], ref) < TOL
    assert normwise(outs[1], ref) < TOL
    assert normwise(outs[0], outs[1]) < TOL


@pytest.mark.parametrize("IC,H,W,OC,PE", [
    (32, 400, 400, 16, 1),   # stem2a
    (16, 400, 400, 32, 1),   # stem2b
    (16, 12, 16, 20, 1),     # ragged output channels, 4 quads per row
    (32, 5, 4, 32, 1),       # one quad per row, bottom padding row
    (16, 9, 20, 7, 1),       # quads of a wave span several rows
])
@pytest.mark.parametrize("act", [0, 1])
def test_conv_k2q_kernel(hip, orc, IC, H, W, OC, PE, act, monkeypatch):
    """Op 16 k2 s1 with 16 or 32 input channels, <= 32 output channels and
    widths a multiple of 4 (the stem's 2x2 convs) on the quad kernel: against float64 with the bottom /
    right zero padding, and against the fragment kernel (PPDL_CONV_K2Q=0)."""
    say(f"k2q conv {IC}->{OC} @{H}x{W} pe{PE} act{act}")
    rng = np.random.default_rng(IC * 13 + OC + H + W + act)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 2)
    wr, _ = hip.repack_conv(w)
    OH, OW = H + PE - 1, W + PE - 1
    p14 = 2 | (1 << 8) | (0 << 16) | (act << 24)
    outs = []
    for flag, kern in (("1", "k_conv_k2q"), ("0", "k_conv_frag<")):
        monkeypatch.setenv("PPDL_CONV_K2Q", flag)
        out = torch.full((OC, OH, OW), float("nan"), device="cuda")
        srcs = [dev(x), dev(wr), dev(b)]
        assert hip.kernel_name(hip.OP_CONV_IM2COL, out, srcs, p14, PE).startswith(kern)
        hip.run_checked(hip.OP_CONV_IM2COL, out, srcs, p14, PE)
        outs.append(host(out))
    xp = np.pad(x, ((0, 0), (0, PE), (0, PE)))
    ref = orc.conv2d_f64(xp, w, b, 1, 0, act)
    assert np.isfinite(outs[0]).all()
    assert normwise(outs[0], ref) < TOL and normwise(outs[1], ref) < TOL


@pytest.mark.parametrize("H,W,OC", [(400, 400, 32), (12, 16, 20), (9, 8, 32), (10, 24, 7)])
@pytest.mark.parametrize("act", [0, 1])
def test_conv_k3s2q_kernel(hip, orc, H, W, OC, act, monkeypatch):
    """Op 16 k3 s2 p1 with 64 input and <= 32 output channels (the stem's
    64 -> 32 conv) on the quad kernel with its four-way channel split: against
    float64, and against the fragment kernel (PPDL_CONV_K2Q=0)."""
    IC = 64
    say(f"k3s2q conv {IC}->{OC} @{H}x{W} act{act}")
    rng = np.random.default_rng(OC + H + W + act)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 3)
    wr, _ = hip.repack_conv(w)
    OH, OW = (H + 2 - 3) // 2 + 1, (W + 2 - 3) // 2 + 1
    p14 = 3 | (2 << 8) | (1 << 16) | (act << 24)
    outs = []
    for flag, kern in (("1", "k_conv_k3s2q"), ("0", "k_conv_frag<")):
        monkeypatch.setenv("PPDL_CONV_K2Q", flag)
        out = torch.full((OC, OH, OW), float("nan"), device="cuda")
        srcs = [dev(x), dev(wr), dev(b)]
        assert hip.kernel_name(hip.OP_CONV_IM2COL, out, srcs, p14).startswith(kern)
        hip.run_checked(hip.OP_CONV_IM2COL, out, srcs, p14)
        outs.append(host(out))
    ref = orc.conv2d_f64(x, w, b, 2, 1, act)
    assert np.isfinite(outs[0]).all()
    assert normwise(outs[0], ref) < TOL and normwise(outs[1], ref) < TOL


# ---------------------------------------------------------------- fused F(4,3) conv (op 17)
def hip_wg4_conv(hip, x, w, b, act):
    _, wg4 = hip.repack_conv(w)
    out = torch.full((w.shape[0],) + x.shape[1:], float("nan"), device="cuda")
    srcs = [dev(x), dev(wg4), dev(b)]
    hip.run_checked(hip.OP_WG4_CONV, out, srcs, act)
    return out, srcs


@pytest.mark.parametrize("IC,H,W,OC", [
    (256, 100, 100, 256), (256, 50, 50, 256), (256, 25, 25, 256), (48, 200, 200, 48), (96, 100, 100, 96),
    (128, 100, 100, 96), (128, 200, 200, 64), (256, 100, 100, 64),
    (1, 1, 1, 1), (3, 9, 10, 2), (5, 4, 4, 7), (17, 13, 11, 33), (33, 17, 23, 65), (64, 13, 200, 64),
    (6, 3, 17, 20),
])
@pytest.mark.parametrize("act", [0, 2])
def test_wg4_conv_fused(hip, orc, IC, H, W, OC, act):
    """Op 17 (ops 15 -> 12 -> 11 as one kernel) on the Winograd benchmark sweep,
    the network's other F(4,3) shapes and ragged edges (channels not a
    multiple of 4 or 16, widths not a multiple of 4, tile counts not a
    multiple of 16) against the oracle's reference CPU conv, the float64
    truth, and the three-op pipeline."""
    say(f"fused F(4,3) {IC}->{OC} @{H}x{W} act{act}")
    rng = np.random.default_rng(IC * 5 + OC + H * 7 + W + act)
    x, w, b = conv_inputs(rng, IC, H, W, OC, 3)
    out, _ = hip_wg4_conv(hip, x, w, b, act)
    y = host(out)
    assert np.isfinite(y).all()
    e = normwise(y, orc.conv2d_ref(x, w, b, 1, 1, act))
    say(f"  normwise vs oracle {e:.2e}")
    assert e < TOL
    if IC * H * W * OC <= 40_000_000:
        assert normwise(y, orc.conv2d_f64(x, w, b, 1, 1, act)) < TOL
    three, _, _, _ = hip_winograd(hip, x, w, b, act)
    assert normwise(y, host(three)) < TOL


@pytest.mark.parametrize("ot", ["1", "2", "3", "4"])
@pytest.mark.parametrize("IC,H,W,OC", [(17, 13, 11, 33), (96, 20, 24, 50), (256, 25, 25, 64), (4, 8, 8, 16),
                                       (48, 40, 44, 48), (6, 9, 9, 20), (12, 10, 10, 16), (16, 10, 10, 16)])
def test_wg4_conv_block_shapes(hip, orc, IC, H, W, OC, ot, monkeypatch):
    """Every block shape of op 17 (1 to 4 tiles of 16 output channels), with
    channel counts that leave partial tiles, blocks and steps, and step
    counts below, at and above the prefetch depth: within the tolerance,
    launched as named, and the same bits on a second run."""
    monkeypatch.setenv("PPDL_WG_OT", ot)
    say(f"fused F(4,3) {IC}->{OC} @{H}x{W} with {ot} channel tiles per block")
    rng = np.random.default_rng(IC + OC + 7 * int(ot))
    x, w, b = conv_inputs(rng, IC, H, W, OC, 3)
    out, srcs = hip_wg4_conv(hip, x, w, b, 1)
    assert hip.kernel_name(hip.OP_WG4_CONV, out, srcs, 1) == f"k_wg4_conv<{ot}>"
    y = host(out).copy()
    assert normwise(y, orc.conv2d_ref(x, w, b, 1, 1, 1)) < TOL
    out.fill_(float("nan"))
    hip.run_checked(hip.OP_WG4_CONV, out, srcs, 1)
    assert np.array_equal(host(out), y)


# ---------------------------------------------------------------- split-K
SPLIT_SHAPES = [  # long K, few output tiles: the planner splits K
    ("conv1x1", (3328, 25, 25, 1024, 1, 1, 0)),
    ("conv1x1", (1664, 50, 50, 512, 1, 1, 0)),
    ("im2col", (256, 50, 50, 256, 3, 2, 1)),
    ("im2col", (64, 13, 11, 40, 3, 2, 1)),
]


@pytest.mark.parametrize("kind,shape", SPLIT_SHAPES)
@pytest.mark.parametrize("plan", ["3,4", "0,3", "5,2"])
def test_split_k_matches_unsplit_and_is_deterministic(hip, orc, kind, shape, plan, monkeypatch):
    """Split-K pinned to several (block shape, splits) plans; one workspace
    reused for several launches: every launch must write the whole output
    (NaN-filled before each run), identically each time, and agree with the
    unsplit GEMM and the oracle."""
    monkeypatch.setenv("PPDL_GEMM_TILE", plan)
    IC, H, W, OC, K, S, P = shape
    say(f"split-K {kind} {IC}->{OC} @{H}x{W}")
    rng = np.random.default_rng(IC + OC)
    x, w, b = conv_inputs(rng, IC, H, W, OC, K)
    wr, _ = hip.repack_conv(w)
    xt, wt, bt = dev(x), dev(wr), dev(b)
    OH, OW = (H + 2 * P - K) // S + 1, (W + 2 * P - K) // S + 1
    out = torch.empty((OC, OH, OW), device="cuda")
    if kind == "conv1x1":
        op, p14 = hip.OP_CONV1X1_BA, 2
    else:
        op, p14 = hip.OP_CONV_IM2COL, K | (S << 8) | (P << 16) | (2 << 24)
    nb = hip.workspace_bytes(op, out, [xt, wt, bt], p14)
    assert nb > 0, "the planner should split this shape"
    ws = hip.make_workspace(nb)
    runs = []
    for _ in range(3):
        out.fill_(float("nan"))
        hip.run_checked(op, out, [xt, wt, bt, ws], p14)
        runs.append(host(out).copy())
    out.fill_(float("nan"))
    hip.run_checked(op, out, [xt, wt, bt], p14)  # no workspace: the same block shape unsplit
    unsplit = host(out)
    ref = orc.conv2d_ref(x, w, b, S, P, 2)
    assert not np.isnan(runs[0]).any() and not np.isnan(runs[2]).any()
    assert np.array_equal(runs[0], runs[1]) and np.array_equal(runs[1], runs[2]), "split-K must be deterministic"
    assert normwise(runs[0], ref) < TOL
    assert normwise(unsplit, ref) < TOL


def test_workspace_too_small_falls_back(hip, orc, monkeypatch):
    monkeypatch.setenv("PPDL_GEMM_TILE", "3,8")
    rng = np.random.default_rng(6)
    x, w, b = conv_inputs(rng, 1024, 25, 25, 512, 1)
    wr, _ = hip.repack_conv(w)
    xt, wt, bt = dev(x), dev(wr), dev(b)
    out = torch.empty((512, 25, 25), device="cuda")
    nb = hip.workspace_bytes(hip.OP_CONV1X1_BA, out, [xt, wt, bt], 0)
    assert nb > 0
    small = hip.make_workspace(nb // 3)
    out.fill_(float("nan"))
    hip.run_checked(hip.OP_CONV1X1_BA, out, [xt, wt, bt, small], 0)
    assert normwise(host(out), orc.conv2d_ref(x, w, b, 1, 0, 0)) < TOL


# ---------------------------------------------------------------- bias + act
@pytest.mark.parametrize("shape", [(256, 100, 100), (7, 5, 3), (3, 1, 1)])
def test_bias_act(hip, orc, shape):
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(np.float32)
    b = rng.standard_normal(shape[0]).astype(np.float32)
    for act in (0, 1, 2):
        out = torch.empty(shape, device="cuda")
        hip.run_checked(hip.OP_BIASACT, out, [dev(x), dev(b)], act)
        y, ref = host(out), orc.bias_act(x, b, act)
        if act == 2:
            assert rel1(y, ref) < 1e-6
        else:
            assert np.array_equal(y, ref)


# ---------------------------------------------------------------- MSDeformAttn
def msdef_300q(rng, nq=300):
    """Config 4: values N(0,1); ref cx,cy U(0,1), w,h U(0.05,1); a normalised
    displacement d ~ N(0, 0.05) per sample, off = d*8/wh so loc = ref + d,
    then loc clamped to [-0.1, 1.1] (partly and fully out-of-bounds samples);
    attention logits N(0,1)."""
    val = rng.standard_normal((13125, 256)).astype(np.float32)
    ref = np.concatenate([rng.random((nq, 2)), rng.uniform(0.05, 1.0, (nq, 2))], 1).astype(np.float32)
    d = rng.normal(0.0, 0.05, (nq, 8, 3, 4, 2))
    loc = np.clip(ref[:, None, None, None, :2] + d, -0.1, 1.1)
    off = ((loc - ref[:, None, None, None, :2]) * 8.0 / ref[:, None, None, None, 2:]).astype(np.float32)
    awr = rng.standard_normal((nq, 96)).astype(np.float32)
    return val, off.reshape(nq, 192), awr, ref


def hip_msdeform(hip, val, off, awr, ref):
    out = torch.empty((ref.shape[0], 256), device="cuda")
    hip.run_checked(hip.OP_MSDEF, out, [dev(val), dev(off), dev(awr), dev(ref)])
    return host(out)


def col_slice_view(hip, wide, col, ncols):
    """ne(ncols, rows) view of columns [col, col + ncols) of a 2-d tensor."""
    rows, ld = wide.shape
    v = hip.TView()
    v.data = wide.data_ptr() + col * 4
    for i, (n, b) in enumerate(zip((ncols, rows, 1, 1), (4, ld * 4, ld * 4 * rows, ld * 4 * rows))):
        v.ne[i], v.nb[i] = n, b
    v.type = hip.TYPE_F32
    return v


def test_msdeform_row_strided_value(hip, orc):
    """Value map, offsets and attention logits may be row-strided slices of
    wider projections (the runtime's six decoder layers share one 13125 x
    1536 value projection; offsets | logits come from one 288-wide GEMM):
    same result, bit for bit, as the contiguous inputs."""
    val, off, awr, ref = msdef_300q(np.random.default_rng(SEED + 44))
    wide = torch.full((val.shape[0], 1536), float("nan"), device="cuda")
    wide[:, 512:768] = dev(val)
    v = col_slice_view(hip, wide, 512, 256)
    out = torch.empty((ref.shape[0], 256), device="cuda")
    hip.run_checked(hip.OP_MSDEF, out, [v, dev(off), dev(awr), dev(ref)])
    want = hip_msdeform(hip, val, off, awr, ref)
    assert np.array_equal(host(out), want)
    soaw = torch.full((ref.shape[0], 300), float("nan"), device="cuda")
    soaw[:, :192] = dev(off)
    soaw[:, 192:288] = dev(awr)
    out2 = torch.empty((ref.shape[0], 256), device="cuda")
    hip.run_checked(hip.OP_MSDEF, out2, [v, col_slice_view(hip, soaw, 0, 192), col_slice_view(hip, soaw, 192, 96),
                                         dev(ref)])
    assert np.array_equal(host(out2), want)
    bad = hip.TView()
    bad.data, bad.type = v.data, v.type
    for i, (n, b) in enumerate(zip((256, val.shape[0], 1, 1), (4, 255 * 4, 255 * 4 * val.shape[0],
                                                                   255 * 4 * val.shape[0]))):
        bad.ne[i], bad.nb[i] = n, b
    assert hip.run(hip.OP_MSDEF, out, [bad, dev(off), dev(awr), dev(ref)]) == hip.EINVAL  # rows overlap


def test_msdeform_300q(hip, orc):
    say("msdeform 300q x 8h x 3lvl x 4pt")
    val, off, awr, ref = msdef_300q(np.random.default_rng(SEED + 4))
    y = hip_msdeform(hip, val, off, awr, ref)
    oref = orc.msdeform(val, off, awr, ref)
    e = normwise(y, oref)
    say(f"  normwise {e:.2e}, bit-exact fraction {np.mean(y == oref):.3f}")
    assert e < TOL


def test_msdeform_fixture_and_special_cases(hip, orc):
    f = np.load(os.path.join(GOLD, "msdef_nq7.npz"))
    val = msdef_value_map(int(f["val_salt"]))
    assert normwise(hip_msdeform(hip, val, f["off"], f["awr"], f["ref"]), f["y"]) < TOL
    # all samples outside -> exactly 0
    far = np.tile(np.array([[5.0, 5.0, 0.5, 0.5]], np.float32), (3, 1))
    assert not hip_msdeform(hip, val, np.zeros((3, 192), np.float32), np.zeros((3, 96), np.float32), far).any()
    # texel-centre copy
    r = np.array([[37.5 / 100, 12.5 / 100, 0.3, 0.3]], np.float32)
    lg = np.tile(np.array([0] + [-1e4] * 11, np.float32), 8)[None]
    y = hip_msdeform(hip, val, np.zeros((1, 192), np.float32), lg, r)
    assert np.array_equal(y[0], val[12 * 100 + 37])
    # odd query counts
    rng = np.random.default_rng(3)
    for nq in (1, 17):
        v2, o2, a2, r2 = msdef_300q(rng, nq)
        assert normwise(hip_msdeform(hip, v2, o2, a2, r2), orc.msdeform(v2, o2, a2, r2)) < TOL


def test_msdeform_skipped_corners_do_not_reach_the_sum(hip, orc):
    """The reference skips a corner outside the map or with zero bilinear
    weight (src/ppdoclayout.cpp:183), so a non-finite value there never
    reaches the output.  Inf / NaN planted at token 0 (the address skipped
    corners read) and at the zero-weight neighbours of a level-0 texel
    centre: a query sampling only that centre, and a query whose samples all
    fall outside, stay finite and equal the oracle."""
    rng = np.random.default_rng(SEED + 45)
    val = rng.standard_normal((13125, 256)).astype(np.float32)
    val[0] = np.inf
    val[3] = np.inf     # (x 3, y 0): weight 0 beside the centre of texel (2, 0)
    val[102] = np.nan   # (x 2, y 1)
    val[103] = -np.inf  # (x 3, y 1)
    ref = np.array([[2.5 / 100, 0.5 / 100, 0.3, 0.3],  # texel centre (2, 0) of level 0
                    [5.0, 5.0, 0.5, 0.5]], np.float32)  # every sample outside every level
    off = np.zeros((2, 192), np.float32)
    awr = rng.standard_normal((2, 96)).astype(np.float32)
    y = hip_msdeform(hip, val, off, awr, ref)
    oref = orc.msdeform(val, off, awr, ref)
    assert np.isfinite(oref).all()
    assert np.isfinite(y).all()
    assert not y[1].any()
    assert normwise(y, oref) < TOL


# ---------------------------------------------------------------- mask box / top-k
def test_mask_box(hip, orc):
    rng = np.random.default_rng(21)
    ml = rng.standard_normal((300, 40000)).astype(np.float32) - 2.5  # sparse positives
    ml[0] = -1.0               # empty mask
    ml[1] = 1.0                # full mask
    ml[2] = -1.0
    ml[2, 199 * 200 + 199] = 0.5  # single corner pixel
    out = torch.empty((300, 4), device="cuda")
    hip.run_checked(hip.OP_MASKBOX, out, [dev(ml)])
    y, ref = host(out), orc.mask_box(ml)
    assert rel1(y, ref) < 1e-6


@pytest.mark.parametrize("with_ws", [False, True])
def test_topk(hip, orc, with_ws):
    """Both paths: keys computed by the selection block (no workspace) and by
    the grid-wide key kernel (workspace of 8 bytes per token)."""
    rng = np.random.default_rng(22)
    ws = torch.empty((13125 * 2,), dtype=torch.float32, device="cuda") if with_ws else None

    def run(lg, nq):
        out = torch.empty((nq,), dtype=torch.int32, device="cuda")
        hip.run_checked(hip.OP_TOPK, out, [dev(lg)] + ([ws] if with_ws else []))
        return host(out)

    lg = rng.standard_normal((13125, 25)).astype(np.float32)
    lg[10:20] = 9.0          # ties -> lower index first
    lg[7000, 3] = 9.0
    lg[40] = -0.0            # -0 and +0 compare equal
    lg[41] = 0.0
    assert np.array_equal(run(lg, 300), orc.topk(lg, 300))
    # all equal -> 0..299 (the selection runs into the index bytes)
    eq = np.zeros((13125, 25), np.float32)
    assert np.array_equal(run(eq, 300), np.arange(300, dtype=np.int32))
    # a tie group straddling the 300th place
    tie = rng.standard_normal((13125, 25)).astype(np.float32)
    tie[::37] = 5.0
    assert np.array_equal(run(tie, 300), orc.topk(tie, 300))
    small = rng.standard_normal((50, 3)).astype(np.float32)
    assert np.array_equal(run(small, 50), orc.topk(small, 50))
    # scores crowded into one histogram bin (more keys than the direct ranking
    # takes): the radix select
    crowd = (100.0 + 1e-3 * rng.standard_normal((13125, 25))).astype(np.float32)
    assert np.array_equal(run(crowd, 300), orc.topk(crowd, 300))
    # a wide spread: the threshold bin holds few keys
    wide = (rng.standard_normal((13125, 25)) * np.exp(4 * rng.standard_normal((13125, 1)))).astype(np.float32)
    assert np.array_equal(run(wide, 300), orc.topk(wide, 300))


# ---------------------------------------------------------------- tail balancing
@pytest.mark.parametrize("kind,IC,OC,H,W", [
    ("conv1x1", 512, 256, 100, 100),  # 1x1 512->256 @100^2: 628 tiles, 14-15 tail tiles per XCD
    ("conv1x1", 96, 200, 60, 167),    # 4 x 157 tiles, ragged M and N edges inside the tail
    ("madd", 96, 192, 1, 640),        # 36 planes x 3 x 10 tiles: 7 tail tiles per XCD
])
def test_dma_tail_balancing_bit_identical(hip, orc, kind, IC, OC, H, W, monkeypatch):
    """The balanced-tail launch of the 64x64 direct-to-LDS GEMM (each XCD's
    last round as half tiles) against the plain launch (PPDL_DMA_TAIL=0): the
    same k split and sum order, so bit-identical, and both at the oracle's
    tolerance."""
    say(f"tail balancing {kind} {IC}->{OC} @{H}x{W}")
    monkeypatch.setenv("PPDL_LT", "off")  # the 64x64 kernel even if the 16x16 menu were planned
    rng = np.random.default_rng(IC + OC + W)
    outs = []
    def launched(flag, op, dst, srcs, p14=0):
        name = hip.kernel_name(op, dst, srcs, p14)
        say(f"  PPDL_DMA_TAIL={flag}: {name}")
        assert name.startswith("k_gemm_dma<64, 64, 2, false, 2, 2, ")
        assert name.endswith("true>" if flag == "1" else "false>"), name

    if kind == "conv1x1":
        x, w, b = conv_inputs(rng, IC, H, W, OC, 1)
        for flag in ("1", "0"):
            monkeypatch.setenv("PPDL_DMA_TAIL", flag)
            out, srcs = hip_conv1x1(hip, x, w, b, 1)
            launched(flag, hip.OP_CONV1X1_BA, out, list(srcs), 1)
            outs.append(host(out))
        ref = orc.conv2d_ref(x, w, b, 1, 0, 1)
    else:
        T = W
        dt = rng.random((36, IC, T)).astype(np.float32)
        wg = (rng.standard_normal((36, IC, OC)) / np.sqrt(IC)).astype(np.float32)
        for flag in ("1", "0"):
            monkeypatch.setenv("PPDL_DMA_TAIL", flag)
            yt = torch.full((36, OC, T), float("nan"), device="cuda")
            srcs = with_ws(hip, hip.OP_WG4_MADD, yt, [dev(dt), dev(wg)])
            launched(flag, hip.OP_WG4_MADD, yt, srcs)
            hip.run_checked(hip.OP_WG4_MADD, yt, srcs)
            outs.append(host(yt))
        ref = np.einsum("pko,pkt->pot", wg.astype(np.float64), dt.astype(np.float64))
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0], outs[1])
    e = normwise(outs[0], ref)
    say(f"  normwise {e:.2e}")
    assert e < TOL

# ---------------------------------------------------------------- graph capture
def test_ops_replay_under_graph_capture(hip):
    """Every op is capture-safe: a captured sequence replays to the eager
    result, replay after replay, with eager work in between."""
    say("graph capture of winograd + 1x1 + msdeform")
    rng = np.random.default_rng(23)
    x, w, b = conv_inputs(rng, 64, 50, 50, 64, 3)
    _, wg4 = hip.repack_conv(w)
    w1 = (rng.standard_normal((32, 64, 1, 1)) / 8).astype(np.float32)
    wr1, _ = hip.repack_conv(w1)
    xt, wgt, bt, w1t = dev(x), dev(wg4), dev(b), dev(wr1)
    b1 = dev(rng.uniform(-0.1, 0.1, 32).astype(np.float32))
    T = 13 * 13
    dt = torch.empty((36, 64, T), device="cuda")
    yt = torch.empty((36, 64, T), device="cuda")
    mid = torch.empty((64, 50, 50), device="cuda")
    mid2 = torch.empty((64, 50, 50), device="cuda")
    out = torch.empty((32, 50, 50), device="cuda")
    val, off, awr, ref = msdef_300q(rng, 300)
    vt, ot, at, rt = dev(val), dev(off), dev(awr), dev(ref)
    ms = torch.empty((300, 256), device="cuda")

    def seq():
        s = torch.cuda.current_stream().cuda_stream
        hip.run_checked(hip.OP_WG4_INPUT_PAD, dt, [xt], T, 13, stream=s)
        hip.run_checked(hip.OP_WG4_MADD, yt, [dt, wgt], stream=s)
        hip.run_checked(hip.OP_WG4_OUTPUT, mid, [yt, bt], 2, 13, stream=s)
        hip.run_checked(hip.OP_CONV1X1_BA, out, [mid, w1t, b1], 1, stream=s)
        hip.run_checked(hip.OP_WG4_CONV, mid2, [xt, wgt, bt], 2, stream=s)
        hip.run_checked(hip.OP_MSDEF, ms, [vt, ot, at, rt], stream=s)

    seq()
    eager_out, eager_ms, eager_mid2 = host(out).copy(), host(ms).copy(), host(mid2).copy()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            seq()
    torch.cuda.current_stream().wait_stream(side)
    for i in range(3):
        out.zero_()
        ms.zero_()
        mid2.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(out), eager_out), i
        assert np.array_equal(host(ms), eager_ms), i
        assert np.array_equal(host(mid2), eager_mid2), i
        junk = torch.randn(1000, device="cuda").sum()  # eager work between replays
        torch.cuda.synchronize()
        del junk
