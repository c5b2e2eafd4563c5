"""CPU checks of the full-network pieces: the GGUF layout, the synthetic
model's tensor table, the stock-op restatements in oracle/ppdl_net.py
(pinned against float64 closed forms, brute force and special cases), the
network composition of oracle/ppdl_net.py against transformers'
PP-DocLayoutV3 run in float64 (tests/golden/net_*.npz, written by
tests/golden/make_net_golden.py), the postprocess, and the runtime
library's file checks (no GPU needed)."""
import ctypes
import os
import struct
import sys

import numpy as np
import pytest

import synth_gguf as S
from conftest import normwise
from oracle import ppdl_net as N

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
if GOLD not in sys.path:
    sys.path.insert(0, GOLD)
import net_inputs as NI  # noqa: E402


# ---------------------------------------------------------------- GGUF layout

def test_gguf_roundtrip_and_layout(tmp_path):
    rng = np.random.default_rng(1)
    t = {"b.bias": rng.standard_normal(7).astype(np.float32),
         "a.weight": rng.standard_normal((5, 3, 3, 3)).astype(np.float32),
         "c.weight": rng.standard_normal((4, 6)).astype(np.float32)}
    p = str(tmp_path / "m.gguf")
    S.write_gguf(p, t)
    raw = open(p, "rb").read()
    assert raw[:4] == b"GGUF" and struct.unpack_from("<I", raw, 4)[0] == 3
    assert struct.unpack_from("<QQ", raw, 8) == (3, 6)
    kv, back = S.read_gguf(p)
    assert kv["ppdlv3.num_queries"] == 300 and kv["ppdlv3.num_classes"] == 25
    assert sorted(back) == sorted(t)
    for k in t:
        assert np.array_equal(back[k], t[k])


def test_gguf_tensor_dims_are_reversed_numpy_shape(tmp_path):
    # ggml ne order: a conv weight OIHW is stored as ne = (K, K, IC, OC)
    p = str(tmp_path / "m.gguf")
    S.write_gguf(p, {"w.weight": np.zeros((8, 4, 3, 2), np.float32)})
    raw = open(p, "rb").read()
    i = raw.index(b"w.weight") + len(b"w.weight")
    nd = struct.unpack_from("<I", raw, i)[0]
    assert nd == 4 and struct.unpack_from("<4Q", raw, i + 4) == (2, 3, 4, 8)


def test_model_tensor_table():
    specs = S.tensor_specs()
    names = [n for n, _, _ in specs]
    assert len(names) == len(set(names))
    assert all(len(n) < 64 for n in names)  # converter limit
    shp = {n: s for n, s, _ in specs}
    # HGNetV2 aggregation widths (in + 6 * mid -> out / 2 -> out)
    assert shp["st3.b0.agg0.weight"] == (1024, 1024 + 6 * 384, 1, 1)
    assert shp["st2.b1.agg0.weight"] == (512, 1024 + 6 * 192, 1, 1)
    assert shp["st0.b0.l0.weight"] == (48, 48, 3, 3)
    assert shp["st2.b0.l0.c2.weight"] == (192, 1, 5, 5)
    assert shp["st1.ds.weight"] == (128, 1, 3, 3)
    assert shp["stem2a.weight"] == (16, 32, 2, 2)
    assert shp["dec5.ca.so.weight"] == (192, 256) and shp["dec5.ca.aw.weight"] == (96, 256)
    assert shp["qpos.0.weight"] == (512, 4) and shp["gp.weight"] == (128, 256)
    assert sum(int(np.prod(s)) for s in shp.values()) > 30_000_000


def test_random_weights_are_seeded():
    a, b = S.random_weights(3), S.random_weights(3)
    assert all(np.array_equal(a[k], b[k]) for k in a)
    assert not np.array_equal(a["stem1.weight"], S.random_weights(4)["stem1.weight"])


# ---------------------------------------------------------------- runtime file checks

def test_runtime_rejects_bad_model_files(tmp_path):
    import ppdoclayout as P

    L = P.lib()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUF" + struct.pack("<I", 3) + b"\xff" * 8)
    assert L.ppdl_init(str(bad).encode(), P.BACKEND_HIP) is None
    wrongver = tmp_path / "v9.gguf"
    wrongver.write_bytes(b"GGUF" + struct.pack("<IQQ", 9, 0, 0))
    assert L.ppdl_init(str(wrongver).encode(), P.BACKEND_HIP) is None
    notg = tmp_path / "x.bin"
    notg.write_bytes(b"NOPE" * 8)
    assert L.ppdl_init(str(notg).encode(), P.BACKEND_HIP) is None
    assert L.ppdl_init(str(tmp_path / "missing.gguf").encode(), P.BACKEND_HIP) is None
    # truncated data section: header promises a tensor the file does not hold
    t = {"w.weight": np.ones((4, 4), np.float32)}
    p = str(tmp_path / "trunc.gguf")
    S.write_gguf(p, t)
    data = open(p, "rb").read()
    open(p, "wb").write(data[:-40])
    assert L.ppdl_init(p.encode(), P.BACKEND_HIP) is None


def test_runtime_null_handles_are_safe():
    import ppdoclayout as P

    L = P.lib()
    assert L.ppdl_graph_nodes(None) == 0
    assert L.ppdl_time_graph(None, 5) < 0
    assert L.ppdl_dump(None, b"/tmp") == 1
    assert L.ppdl_dump_raw(None, b"/tmp/x") == 1
    assert L.ppdl_compute(None, None) == 1
    L.ppdl_free(None)


# ---------------------------------------------------------------- stock-op restatements

def test_layer_norm_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((40, 256)).astype(np.float32) * 3 + 1
    w, b = rng.standard_normal(256).astype(np.float32), rng.standard_normal(256).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5) * w + b
    assert np.abs(N.layer_norm(x, w, b) - ref).max() < 1e-5
    # constant rows normalise to the bias
    c = np.full((2, 256), 7.0, np.float32)
    assert np.allclose(N.layer_norm(c, w, b), b)


def test_softmax_and_attention_vs_float64():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 33)).astype(np.float32) * 4
    s = N.softmax_rows(x)
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    assert np.abs(s - e / e.sum(1, keepdims=True)).max() < 1e-6
    # multi-head attention against a float64 per-head loop
    T = 17
    w = {}
    for p in ("q", "k", "v", "o"):
        w["t.%s.weight" % p] = (rng.standard_normal((256, 256)) / 16).astype(np.float32)
        w["t.%s.bias" % p] = rng.standard_normal(256).astype(np.float32) * 0.1
    net = N.Net(w)
    qk = rng.standard_normal((T, 256)).astype(np.float32)
    v_in = rng.standard_normal((T, 256)).astype(np.float32)
    got = net.mha(qk, v_in, "t")
    W = {k: v.astype(np.float64) for k, v in w.items()}
    q = qk @ W["t.q.weight"].T + W["t.q.bias"]
    k = qk @ W["t.k.weight"].T + W["t.k.bias"]
    v = v_in @ W["t.v.weight"].T + W["t.v.bias"]
    out = np.zeros((T, 256))
    for h in range(8):
        sl = slice(32 * h, 32 * h + 32)
        a = q[:, sl] @ k[:, sl].T / np.sqrt(32.0)
        a = np.exp(a - a.max(1, keepdims=True))
        out[:, sl] = (a / a.sum(1, keepdims=True)) @ v[:, sl]
    ref = out @ W["t.o.weight"].T + W["t.o.bias"]
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5


def test_interpolation_special_cases():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 5, 7)).astype(np.float32)
    # nearest 2x: every source pixel becomes a 2x2 block
    n = N.interp_nearest(x, 10, 14)
    assert np.array_equal(n, x.repeat(2, 1).repeat(2, 2))
    # bilinear keeps constants, reproduces a linear ramp away from the edges
    c = np.full((2, 4, 4), 3.25, np.float32)
    assert np.array_equal(N.interp_bilinear(c, 8, 8), np.full((2, 8, 8), 3.25, np.float32))
    ramp = np.tile(np.arange(6, dtype=np.float32), (1, 6, 1))
    up = N.interp_bilinear(ramp, 12, 12)
    xs = (np.arange(12) + 0.5) / 2 - 0.5
    inner = (xs >= 0) & (xs <= 5)
    assert np.allclose(up[0, 3, inner], xs[inner], atol=1e-6)
    assert up[0, 3, 0] == 0.0 and up[0, 3, -1] == 5.0  # clamped edges
    # half-pixel 2x: output (1,1) mixes source (0,0),(0,1),(1,0),(1,1) 9:3:3:1 / 16
    y = N.interp_bilinear(x, 10, 14)
    ref = (9 * x[:, 0, 0] + 3 * x[:, 0, 1] + 3 * x[:, 1, 0] + x[:, 1, 1]) / 16
    assert np.allclose(y[:, 1, 1], ref, atol=1e-6)


def test_maxpool_and_depthwise_brute_force(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 6, 5)).astype(np.float32)
    p = N.maxpool2_padend(x)
    xp = np.pad(x, ((0, 0), (0, 1), (0, 1)))
    ref = np.array([[[xp[c, i:i + 2, j:j + 2].max() for j in range(5)] for i in range(6)] for c in range(3)])
    assert np.array_equal(p, ref)
    for k, s, pd in ((3, 2, 1), (5, 1, 2)):
        w = rng.standard_normal((3, 1, k, k)).astype(np.float32)
        b = rng.standard_normal(3).astype(np.float32)
        got = N.dwconv(x, w, b, s, pd, N.ACT_NONE)
        for c in range(3):  # one channel = a 1-in 1-out conv, float64 truth
            ref = orc.conv2d_f64(x[c:c + 1], w[c:c + 1], b[c:c + 1], s, pd)
            assert np.abs(got[c] - ref[0]).max() < 1e-5


def test_activations_vs_float64():
    x = np.linspace(-9, 9, 1001).astype(np.float32)
    x64 = x.astype(np.float64)
    assert np.abs(N.silu(x) - x64 / (1 + np.exp(-x64))).max() < 1e-5
    assert np.abs(N.sigmoid(x) - 1 / (1 + np.exp(-x64))).max() < 1e-6
    from scipy.special import erf

    assert np.abs(N.gelu_erf(x) - 0.5 * x64 * (1 + erf(x64 / np.sqrt(2)))).max() < 1e-5
    # inv_sigmoid inverts sigmoid inside the clamp range, saturates at +-log(1e5)
    z = np.linspace(-6, 6, 101).astype(np.float32)
    assert np.abs(N.inv_sigmoid(N.sigmoid(z)) - z).max() < 2e-3
    assert np.isclose(N.inv_sigmoid(np.float32(1.0)), np.log(1e5), rtol=1e-5)
    assert np.isclose(N.inv_sigmoid(np.float32(0.0)), -np.log(1e5), rtol=1e-5)


def test_host_constants():
    pe = N.pos_embed()
    assert pe.shape == (625, 256)
    h, w, i = 3, 7, 5
    om = 1.0 / 10000 ** (i / 64)
    row = pe[h * 25 + w]
    assert np.isclose(row[i], np.sin(h * om)) and np.isclose(row[64 + i], np.cos(h * om))
    assert np.isclose(row[128 + i], np.sin(w * om)) and np.isclose(row[192 + i], np.cos(w * om))
    v = N.valid_mask()
    # (x + 0.5) / n must lie strictly inside (0.01, 0.99): the border ring of
    # the 100x100 and 50x50 levels is invalid, the 25x25 level is all valid
    assert v.shape == (13125,) and int(v.sum()) == 13125 - (4 * 99) - (4 * 49)
    assert v[0] == 0 and v[101] == 1 and v[10000] == 0 and v[10051] == 1 and v[12500:].all()


# ---------------------------------------------------------------- composition vs transformers
# Each fixture holds float64 transformers outputs of the same synthetic model
# (the GGUF weights with their BatchNorm fold undone); the oracle runs in
# float32, so agreement is to float32 accumulation error: 1e-5 normwise.
NET_TOL = 1e-5


@pytest.fixture(scope="module")
def fixture_net():
    return N.Net(S.random_weights(NI.WEIGHT_SEED))


def test_backbone_matches_transformers(fixture_net):
    g = np.load(os.path.join(GOLD, "net_backbone.npz"))
    outs = fixture_net.backbone(NI.backbone_input())
    assert normwise(fixture_net.dumps["stem"], g["stem"]) <= NET_TOL
    for i, o in enumerate(outs):
        assert o.shape == g["st%d" % i].shape
        assert normwise(o, g["st%d" % i]) <= NET_TOL, i


def test_hybrid_encoder_matches_transformers(fixture_net):
    g = np.load(os.path.join(GOLD, "net_encoder.npz"))
    f8, n16, n32, mf = fixture_net.encoder(*NI.encoder_inputs())
    got = {"aifi": fixture_net.dumps["aifi"], "f8": f8, "n16": n16, "n32": n32, "mask_feat": mf}
    for k, v in got.items():
        assert v.shape == g[k].shape, k
        assert normwise(v, g[k]) <= NET_TOL, k


def test_decoder_and_heads_match_transformers(fixture_net):
    g = np.load(os.path.join(GOLD, "net_decode.npz"))
    f8, n16, n32, mf = NI.decode_inputs()
    o = fixture_net.decode(f8, n16, n32, mf)
    d = fixture_net.dumps
    assert np.array_equal(o["topk"], g["topk"])
    # the mask-derived initial boxes cover whole-page, empty and local masks
    ref = g["init_ref_unact"]
    assert (ref[:, 2] < -11).sum() >= 10 and (ref[:, 2] > 11).sum() >= 10 and (np.abs(ref[:, 2]) < 5).sum() >= 50
    assert normwise(o["init_ref"], ref) <= NET_TOL
    for i in range(6):
        assert normwise(d["hidden%d" % i][:32], g["hidden_first32"][i]) <= NET_TOL, i
    assert normwise(o["logits"], g["logits"]) <= NET_TOL
    assert normwise(o["boxes"], g["boxes"]) <= NET_TOL
    # masks = mask queries x prototypes and order = q_i . k_j / sqrt(64),
    # both from the stored head projections
    mq, gp = g["mq"].astype(np.float64), g["gp"].astype(np.float64)
    assert normwise(d["mq"], mq) <= NET_TOL and normwise(d["gp"], gp) <= NET_TOL
    assert normwise(o["masks"], mq @ mf.reshape(32, -1).astype(np.float64)) <= NET_TOL
    assert normwise(o["order"], gp[:, :64] @ gp[:, 64:].T / 8.0) <= NET_TOL


def test_transformers_fixtures_catch_planted_mistakes(fixture_net):
    """The fixtures separate the reference's composition from plausible
    variants: the order head on the normed hidden state (what transformers
    itself does), and a swapped residual / norm order in the AIFI layer."""
    g = np.load(os.path.join(GOLD, "net_decode.npz"))
    o = fixture_net.decode(*NI.decode_inputs())
    x = fixture_net.dumps["hidden5"]
    gp_post = fixture_net.lin(fixture_net.lin(fixture_net.ln(x, "dec_norm"), "order5"), "gp")
    assert normwise(gp_post, g["gp"]) > 1e-2 and normwise(o["order"], g["gp"][:, :64] @ g["gp"][:, 64:].T / 8) <= NET_TOL

    class PreNormAifi(N.Net):
        def aifi(self, s, pos):
            h = self.ln(s, "aifi.ln1")
            s = s + self.mha(h + pos, h, "aifi")
            return s + self.lin(N.gelu_erf(self.lin(self.ln(s, "aifi.ln2"), "aifi.fc1")), "aifi.fc2")

    ge = np.load(os.path.join(GOLD, "net_encoder.npz"))
    bad = PreNormAifi(fixture_net.w)
    bad.encoder(*NI.encoder_inputs())
    assert normwise(bad.dumps["aifi"], ge["aifi"]) > 1e-2


# ---------------------------------------------------------------- postprocess

def test_postprocess_known_answer():
    rng = np.random.default_rng(6)
    logits = rng.standard_normal((300, 25)).astype(np.float32) - 2
    logits[7, 3] = 5.0  # top detection
    logits[11, 4] = 4.0  # second
    logits[11, 9] = 4.0  # tie in score with [11, 4]: lower flat index first
    boxes = rng.uniform(0.2, 0.8, (300, 4)).astype(np.float32)
    # reading order: query i precedes j for i < j  => order[i][j] large for i < j
    iu = np.triu(np.ones((300, 300), np.float32), 1)
    order = 6.0 * iu - 6.0 * iu.T
    masks = rng.standard_normal((300, 40000)).astype(np.float32)
    dets, m, sel = N.postprocess(logits, boxes, order, masks, 1000, 500)
    assert sel[0] == 7 * 25 + 3 and sel[1] == 11 * 25 + 4 and sel[2] == 11 * 25 + 9
    assert dets[0, 0] == 3 and np.isclose(dets[0, 1], 1 / (1 + np.exp(-5.0)))
    # votes[j] = sum_{i != j} sigmoid(order[i][j] - order[j][i]): larger for later
    # queries, so the rank of query q is q
    assert dets[0, 6] == 7 and dets[1, 6] == 11 and dets[2, 6] == 11
    b = boxes[7]
    assert np.isclose(dets[0, 2], (b[0] - b[2] / 2) * 500) and np.isclose(dets[0, 5], (b[1] + b[3] / 2) * 1000)
    assert np.array_equal(m[0], (masks[7] > 0).astype(np.int32))
    assert np.all(np.diff(dets[:, 1]) <= 0)


def test_e2e_gates_detect_planted_differences():
    import e2e_gates as G

    rng = np.random.default_rng(7)
    od = np.zeros((300, 7), np.float32)
    od[:, 0] = rng.integers(0, 25, 300)
    od[:, 1] = np.sort(rng.uniform(0, 1, 300))[::-1]
    od[:, 2:6] = rng.uniform(0, 800, (300, 4))
    od[:, 6] = rng.permutation(300)
    om = rng.integers(0, 2, (300, 40000)).astype(np.int32)
    assert G.passes(G.compare(od, om, od.copy(), om.copy()))
    gd = od.copy()
    gd[3, 1] += 1e-4  # score beyond 3e-5
    assert not G.passes(G.compare(od, om, gd, om))
    gd = od.copy()
    gd[5, 2] += 0.05  # box beyond 0.01 px
    assert not G.passes(G.compare(od, om, gd, om))
    gd = od.copy()
    conf = np.where(od[:, 1] >= 0.3)[0]
    a, b = conf[0], conf[1]
    gd[a, 6], gd[b, 6] = od[b, 6], od[a, 6]  # swapped reading order
    assert not G.compare(od, om, gd, om)["order_rel_ok"]
    gd = od.copy()
    gd[conf[2], 0] = (od[conf[2], 0] + 1) % 25  # label change
    assert not G.passes(G.compare(od, om, gd, om))
