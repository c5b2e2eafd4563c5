"""Pins the CPU oracle before it is trusted as the checker of the HIP kernels.

Each oracle function is checked against something other than its own
formula: the golden fixtures (torch float64 conv2d / grid_sample), the
float64 direct conv, exact closed forms of the Winograd construction, and
special cases whose answer is known.  Planted-mistake tests show that these
checks fail on a plausible bug (a flipped sign, a transposed kernel, a
swapped coordinate).
"""
import glob
import os
import sys
from fractions import Fraction as Fr

import numpy as np
import pytest
from conftest import normwise, rel1

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLD)
from fixture_inputs import msdef_value_map  # noqa: E402


def rand_conv(rng, IC, H, W, OC, K):
    x = rng.random((IC, H, W)).astype(np.float32)
    w = (rng.standard_normal((OC, IC, K, K)) / np.sqrt(K * K * IC)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, OC).astype(np.float32)
    return x, w, b


# --------------------------------------------------------------------------- conv
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLD, "conv_*.npz"))),
                         ids=lambda p: os.path.basename(p))
def test_conv_fixtures(orc, path):
    f = np.load(path)
    S, P, act = (int(v) for v in f["meta"])
    y = f["y"]
    assert normwise(orc.conv2d_f64(f["x"], f["w"], f["b"], S, P, act), y) < 1e-12
    assert normwise(orc.conv2d_ref(f["x"], f["w"], f["b"], S, P, act), y) < 2e-6
    if f["w"].shape[2] == 3 and S == 1 and P == 1:
        assert normwise(orc.winograd_conv(f["x"], f["w"], f["b"], act), y) < 2e-5


@pytest.mark.parametrize("K,S,P", [(1, 1, 0), (2, 1, 0), (3, 2, 1), (3, 1, 1), (5, 2, 2)])
@pytest.mark.parametrize("act", [0, 1, 2])
def test_conv_ref_vs_f64(orc, K, S, P, act):
    rng = np.random.default_rng(K * 100 + S * 10 + P + act)
    x, w, b = rand_conv(rng, 13, 17, 19, 11, K)
    assert normwise(orc.conv2d_ref(x, w, b, S, P, act), orc.conv2d_f64(x, w, b, S, P, act)) < 2e-6


def test_conv_invariants(orc):
    rng = np.random.default_rng(5)
    x, w, b = rand_conv(rng, 4, 9, 11, 3, 3)
    # zero input -> act(bias)
    y = orc.conv2d_ref(np.zeros_like(x), w, b, 1, 1, 0)
    assert np.array_equal(y, np.broadcast_to(b[:, None, None], y.shape))
    # delta kernel at the centre tap -> the input channel, exactly
    wd = np.zeros((4, 4, 3, 3), np.float32)
    for c in range(4):
        wd[c, c, 1, 1] = 1.0
    assert np.array_equal(orc.conv2d_ref(x, wd, np.zeros(4, np.float32), 1, 1, 0), x)
    # delta at tap (0,0) -> input shifted down/right by one with zero fill
    wd2 = np.zeros((4, 4, 3, 3), np.float32)
    for c in range(4):
        wd2[c, c, 0, 0] = 1.0
    y2 = orc.conv2d_ref(x, wd2, np.zeros(4, np.float32), 1, 1, 0)
    assert np.array_equal(y2[:, 1:, 1:], x[:, :-1, :-1]) and not y2[:, 0, :].any() and not y2[:, :, 0].any()
    # linearity in x (to rounding)
    x2 = rng.random(x.shape).astype(np.float32)
    lhs = orc.conv2d_ref(x + x2, w, np.zeros(3, np.float32), 1, 1, 0)
    rhs = orc.conv2d_ref(x, w, np.zeros(3, np.float32), 1, 1, 0) + orc.conv2d_ref(x2, w, np.zeros(3, np.float32), 1, 1, 0)
    assert normwise(lhs, rhs) < 1e-6


def test_planted_transposed_kernel_is_caught(orc):
    """A conv that flips the kernel (true convolution instead of correlation)
    must fail the float64-truth check."""
    rng = np.random.default_rng(6)
    x, w, b = rand_conv(rng, 5, 10, 12, 4, 3)
    truth = orc.conv2d_f64(x, w, b, 1, 1, 0)
    wrong = orc.conv2d_ref(x, np.ascontiguousarray(w[:, :, ::-1, ::-1]), b, 1, 1, 0)
    assert normwise(wrong, truth) > 1e-2


# --------------------------------------------------------------------------- bias/act
def test_bias_act(orc):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 6, 7)).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    for act in (0, 1, 2):
        y = orc.bias_act(x, b, act)
        v = x.astype(np.float64) + b[:, None, None]
        ref = v if act == 0 else (np.maximum(v, 0) if act == 1 else v / (1 + np.exp(-v)))
        assert rel1(y, ref) < 1e-6
    assert np.array_equal(orc.bias_act(x, b, 0), (x + b[:, None, None]).astype(np.float32))


# --------------------------------------------------------------------------- winograd
def _exact_mats(orc):
    Bt, G, At = orc.wg4_matrices()
    frac = lambda M, den: [[Fr(v).limit_denominator(den) for v in row] for row in M]  # noqa: E731
    return frac(Bt, 8), frac(G, 15), frac(At, 8)


def _identity_holds(Bt, G, At):
    # At[i][j] G[j][k] Bt[j][t] summed over j must be [t == i + k]: the F(4,3)
    # correlation identity, in exact rational arithmetic
    for i in range(4):
        for k in range(3):
            for t in range(6):
                s = sum(At[i][j] * G[j][k] * Bt[j][t] for j in range(6))
                if s != (1 if t == i + k else 0):
                    return False
    return True


def test_wg4_matrices_exact_identity(orc):
    Bt, G, At = _exact_mats(orc)
    assert _identity_holds(Bt, G, At)
    # the float64 values are exactly these rationals (dyadic for Bt and At)
    Btf, Gf, Atf = orc.wg4_matrices()
    assert all(float(Bt[i][j]) == Btf[i, j] for i in range(6) for j in range(6))
    assert all(float(At[i][j]) == Atf[i, j] for i in range(4) for j in range(6))
    assert np.abs(np.array(G, dtype=np.float64) - Gf).max() < 1e-16


def test_wg4_matrices_from_toom_cook_points(orc):
    """At rows are powers of the points {0, 1, -1, 2, -1/2} (+ the point at
    infinity); G rows are p^k / prod(p - q): the Lagrange construction."""
    pts = [Fr(0), Fr(1), Fr(-1), Fr(2), Fr(-1, 2)]
    Bt, G, At = _exact_mats(orc)
    for i in range(4):
        assert At[i][:5] == [p**i for p in pts]
        assert At[i][5] == (1 if i == 3 else 0)
    for j, p in enumerate(pts):
        N = Fr(1)
        for q in pts:
            if q != p:
                N *= p - q
        assert G[j] == [p**k / N for k in range(3)]
    assert G[5] == [0, 0, 1]


def test_planted_wrong_sign_in_bt_is_caught(orc):
    Bt, G, At = _exact_mats(orc)
    Bt[2][3] = -Bt[2][3]
    assert not _identity_holds(Bt, G, At)


def test_repack_layouts(orc):
    rng = np.random.default_rng(8)
    w = rng.standard_normal((5, 3, 3, 3)).astype(np.float32)
    wr, wg4 = orc.repack(w)
    for t in range(9):
        assert np.array_equal(wr[t], w[:, :, t // 3, t % 3].T)
    Bt, G, At = orc.wg4_matrices()
    ref = np.einsum("ua,oiab,vb->uvio", G, w.astype(np.float64), G).reshape(36, 3, 5)
    assert np.abs(wg4 - ref).max() <= 4 * np.finfo(np.float32).eps * np.abs(ref).max()
    wr1, none = orc.repack(rng.standard_normal((4, 6, 1, 1)).astype(np.float32))
    assert none is None and wr1.shape == (1, 6, 4)


@pytest.mark.parametrize("IC,H,W,OC", [(3, 9, 10, 2), (16, 13, 13, 8), (8, 4, 4, 3), (5, 1, 1, 4), (7, 5, 9, 6)])
@pytest.mark.parametrize("act", [0, 2])
def test_winograd_pipeline_vs_truth(orc, IC, H, W, OC, act):
    rng = np.random.default_rng(IC * H + W)
    x, w, b = rand_conv(rng, IC, H, W, OC, 3)
    y = orc.winograd_conv(x, w, b, act)
    assert normwise(y, orc.conv2d_f64(x, w, b, 1, 1, act)) < 2e-5


def test_winograd_prepadded_equals_fused_pad(orc):
    rng = np.random.default_rng(9)
    x, w, b = rand_conv(rng, 6, 10, 7, 4, 3)
    TW, TH = orc.wg4_tiles(10, 7)
    xp = np.zeros((6, 4 * TH + 2, 4 * TW + 2), np.float32)
    xp[:, 1:11, 1:8] = x
    assert np.array_equal(orc.wg4_input(xp, TW, TH, 0), orc.wg4_input(x, TW, TH, 1))


def test_winograd_256ch_accuracy(orc):
    """256->256 @ 25x25, the deepest F(4,3) conv of the network: the FP32
    pipeline stays well inside the 2e-5 normwise budget."""
    rng = np.random.default_rng(10)
    x, w, b = rand_conv(rng, 256, 25, 25, 256, 3)
    e = normwise(orc.winograd_conv(x, w, b, 0), orc.conv2d_f64(x, w, b, 1, 1, 0))
    assert e < 8e-6, e


# --------------------------------------------------------------------------- im2col
def test_im2col_matches_loop(orc):
    rng = np.random.default_rng(11)
    x = rng.random((3, 7, 8)).astype(np.float32)
    for K, S, P in [(3, 2, 1), (2, 1, 0), (1, 1, 0)]:
        OH, OW = orc.conv_out_hw(7, 8, K, S, P)
        d = orc.im2col(x, K, S, P, OH, OW)
        xp = np.pad(x, ((0, 0), (P, P), (P, P)))
        ref = np.stack([xp[:, kh + S * np.arange(OH)[:, None], kw + S * np.arange(OW)[None, :]]
                        for kh in range(K) for kw in range(K)], 1)  # IC, K*K, OH, OW
        ref = ref.reshape(3 * K * K, OH * OW).T
        assert np.array_equal(d, ref)


# --------------------------------------------------------------------------- msdeform
def _msdef_inputs(rng, nq, spread=2.0):
    val = msdef_value_map(3)
    ref = np.concatenate([rng.random((nq, 2)), rng.uniform(0.05, 1.0, (nq, 2))], 1).astype(np.float32)
    off = (rng.standard_normal((nq, 192)) * spread).astype(np.float32)
    awr = rng.standard_normal((nq, 96)).astype(np.float32)
    return val, off, awr, ref


def test_msdeform_fixture(orc):
    f = np.load(os.path.join(GOLD, "msdef_nq7.npz"))
    val = msdef_value_map(int(f["val_salt"]))
    y = orc.msdeform(val, f["off"], f["awr"], f["ref"])
    # fp32 sample positions lx*W carry ~W*6e-8 px of rounding against the
    # float64 fixture, hence the op tolerance rather than a few ulp
    assert normwise(y, f["y"]) < 2e-5


def test_msdeform_special_cases(orc):
    rng = np.random.default_rng(12)
    val, off, awr, ref = _msdef_inputs(rng, 4)
    # every sample far outside the map -> exactly zero
    far = ref.copy()
    far[:, :2] = 5.0
    assert not orc.msdeform(val, np.zeros_like(off), awr, far).any()
    # zero offsets at a level-0 texel centre (37.5/100 and 12.5/100 are exact
    # in fp32) with all softmax mass on level 0, point 0: an exact value copy
    r = np.array([[37.5 / 100, 12.5 / 100, 0.3, 0.3]], np.float32)
    only0 = orc.msdeform(val, np.zeros((1, 192), np.float32),
                         np.tile(np.array([0] + [-1e4] * 11, np.float32), 8)[None], r)
    assert np.array_equal(only0[0], val[12 * 100 + 37])
    # equal logits: weights 1/12, so a constant value map reproduces itself
    # at any in-range location whose 4 corners all lie inside every level
    cval = np.full_like(val, 0.75)
    mid = np.array([[0.5, 0.5, 0.2, 0.2]], np.float32)
    y = orc.msdeform(cval, np.zeros((1, 192), np.float32), np.zeros((1, 96), np.float32), mid)
    assert np.abs(y - 0.75).max() < 1e-6


def test_planted_swapped_xy_is_caught(orc):
    f = np.load(os.path.join(GOLD, "msdef_nq7.npz"))
    val = msdef_value_map(int(f["val_salt"]))
    off = f["off"].reshape(7, 96, 2)[:, :, ::-1].reshape(7, 192)
    ref = f["ref"][:, [1, 0, 3, 2]]
    assert normwise(orc.msdeform(val, np.ascontiguousarray(off), f["awr"], np.ascontiguousarray(ref)), f["y"]) > 1e-2


# --------------------------------------------------------------------------- mask box / topk
def test_mask_box(orc):
    rng = np.random.default_rng(13)
    ml = -np.ones((3, 200, 200), np.float32)
    ml[0, 10:20, 30:45] = rng.random((10, 15)).astype(np.float32) + 0.1
    ml[1, 199, 0] = 1.0
    out = orc.mask_box(ml.reshape(3, 40000))
    inv = lambda v: np.log(max(min(max(v, 0.0), 1.0), 1e-5) / max(1.0 - min(max(v, 0.0), 1.0), 1e-5))  # noqa: E731
    x0, x1, y0, y1 = 30 / 200, 45 / 200, 10 / 200, 20 / 200
    exp0 = [inv((x0 + x1) / 2), inv((y0 + y1) / 2), inv(x1 - x0), inv(y1 - y0)]
    assert np.abs(out[0] - exp0).max() < 1e-5
    exp1 = [inv(0.5 / 200), inv(199.5 / 200), inv(1 / 200), inv(1 / 200)]
    assert np.abs(out[1] - exp1).max() < 1e-5
    assert np.all(out[2] == np.float32(np.log(np.float32(1e-5))))  # empty mask -> invsig(0)


def test_topk(orc):
    rng = np.random.default_rng(14)
    lg = rng.standard_normal((13125, 25)).astype(np.float32)
    lg[100:110] = 10.0  # ties above every random row max: lower index first
    lg[5000] = 10.0
    idx = orc.topk(lg, 300)
    m = lg.max(1)
    ref = np.lexsort((np.arange(13125), -m))[:300]
    assert np.array_equal(idx, ref)
    assert list(idx[:11]) == list(range(100, 110)) + [5000]
