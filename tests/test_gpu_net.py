"""Full PP-DocLayoutV3 network on the GPU (the ppdl_* runtime) against the CPU
restatement of the reference's graph (oracle/ppdl_net.py).

The model is the real architecture with seeded random weights written as a
GGUF exactly as the reference's converter lays one out (no checkpoint can be
fetched here).  Two inputs: a synthetic document page and seeded U(0,1)
pixels (the stated benchmark input).  Checks per input: every dumped
intermediate and raw output within a normwise tolerance, the top-300 encoder
selection identical, the host result equal to the reference's postprocess
restated on the GPU's own raw outputs, the postprocessed detections through
the reference's end-to-end gates (e2e_gates.py), and bit-identical graph
replays.
"""
import os
import sys

import numpy as np
import pytest

from conftest import normwise

pytestmark = pytest.mark.gpu

# Normwise tolerances (max|gpu - cpu| / max|cpu|).  Each op is within 2e-5 of
# the CPU restatement on its own; through ~150 sequential layers the
# differences (summation order, Winograd F(4,3) vs im2col) could compound, so
# the network-level gate is looser than the per-op one.  Measured on MI355X:
# at most 7.4e-6 (enc_masks), most tensors 1e-6 .. 4e-6.
TOL_FEATURE = 5e-5
TOL_OUTPUT = 5e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    import synth_gguf

    path = str(tmp_path_factory.mktemp("model") / "ppdlv3-random-seed0.gguf")
    weights = synth_gguf.write_random_model(path, seed=0)
    return path, weights


@pytest.fixture(scope="module", params=["document_page", "uniform_page"])
def image(request):
    import pages

    say("input:", request.param)
    return getattr(pages, request.param)(0)


@pytest.fixture(scope="module")
def cpu(model, image):
    from oracle import ppdl_net

    net = ppdl_net.Net(model[1])
    out = net.forward(image)
    dets, masks, sel = ppdl_net.postprocess(out["logits"], out["boxes"], out["order"], out["masks"], 1000, 700)
    return out, net.dumps, dets, masks, sel


@pytest.fixture(scope="module")
def gpu(model, image, tmp_path_factory):
    import ppdoclayout as P

    say("ppdl_init_ex", model[0])
    ctx = P.PPDocLayout(model[0], P.BACKEND_HIP, dumps=True)
    say("graph kernel launches:", ctx.graph_nodes())
    dets, masks, ms = ctx.infer(image, 1000, 700)
    say("infer_ms %.3f" % ms)
    d = str(tmp_path_factory.mktemp("dump"))
    assert ctx.dump(d) == 0
    raw = {k: ctx.raw(w) for k, w in (("logits", P.RAW_LOGITS), ("boxes", P.RAW_BOXES), ("order", P.RAW_ORDER),
                                      ("masks", P.RAW_MASKS), ("topk", P.RAW_TOPK), ("init_ref", P.RAW_INIT_REF))}
    yield ctx, raw, P.read_dump(d), dets, masks
    ctx.close()


# Tensors whose rows are the 300 decoder queries (in top-300 order).
QUERY_ROWS = {"target", "enc_masks", "init_ref_unact", "hidden0", "hidden1", "hidden2", "hidden3", "hidden4",
              "hidden5", "logits", "boxes", "masks", "init_ref"}


def query_perm(gpu, cpu):
    """p with gpu_topk[p] == cpu_topk: the GPU query order mapped onto the
    CPU's.  The decoder treats every query alike (self-attention and the
    heads are permutation-equivariant), so two tokens whose encoder scores
    tie to rounding may swap places without changing any detection."""
    g, c = gpu[1]["topk"], cpu[0]["topk"]
    pos = {int(t): i for i, t in enumerate(g)}
    return np.array([pos[int(t)] for t in c])


def aligned(name, got, gpu, cpu):
    p = query_perm(gpu, cpu)
    if name == "order":
        return got[p][:, p]
    return got[p] if name in QUERY_ROWS else got


def test_topk_selection_identical(gpu, cpu):
    _, raw, _, _, _ = gpu
    out = cpu[0]
    # the same 300 tokens ...
    assert np.array_equal(np.sort(raw["topk"]), np.sort(out["topk"]))
    # ... in the same order up to swaps of tokens whose scores tie to rounding
    score = cpu[1]["enc_logits"].max(1)
    diff = np.where(raw["topk"] != out["topk"])[0]
    gap = np.abs(score[raw["topk"][diff]] - score[out["topk"][diff]])
    say("top-300 positions that differ:", diff.tolist(), "score gaps", gap.tolist())
    assert np.all(gap <= 1e-4 * np.abs(score).max())


@pytest.mark.parametrize("name", ["stem1", "stem", "st0", "st1", "st2", "st3", "aifi", "f8", "n16", "n32",
                                  "mask_feat", "source", "target", "enc_masks", "init_ref_unact",
                                  "hidden0", "hidden1", "hidden2", "hidden3", "hidden4", "hidden5"])
def test_intermediate_matches_cpu(gpu, cpu, name):
    dumps = gpu[2]
    ref = cpu[1][name]
    got = aligned(name, dumps[name], gpu, cpu)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all()
    err = normwise(got, ref)
    say("%-16s normwise %.3g" % (name, err))
    assert err <= TOL_FEATURE, (name, err)


@pytest.mark.parametrize("name", ["logits", "boxes", "order", "masks", "init_ref"])
def test_raw_output_matches_cpu(gpu, cpu, name):
    got = aligned(name, gpu[1][name], gpu, cpu)
    ref = cpu[0][name]
    assert got.shape == ref.shape
    err = normwise(got, ref)
    say("%-10s normwise %.3g  max abs %.3g" % (name, err, float(np.abs(got - ref).max())))
    assert err <= TOL_OUTPUT, (name, err)


def test_postprocessed_detections_pass_gates(gpu, cpu):
    import e2e_gates

    _, _, _, dets, masks = gpu
    m = e2e_gates.compare(cpu[2], cpu[3], dets, masks)
    say("e2e gates:", m)
    assert m["n_conf"] > 0
    assert e2e_gates.passes(m), m


def test_host_result_equals_restated_postprocess(gpu, tmp_path):
    """ppdl_infer's host result (mask bits packed on the device, key-based
    selection and reading ranks on the host) against the oracle's
    restatement of the reference postprocess (src/ppdoclayout.cpp:927-993)
    applied to the same raw outputs: labels, boxes, ranks, the picked flat
    indices and the masks bit for bit; scores to 2 ulp (host expf against
    numpy's exp)."""
    from oracle import ppdl_net

    ctx, raw, _, dets, masks = gpu
    d, m, sel = ppdl_net.postprocess(raw["logits"], raw["boxes"], raw["order"], raw["masks"], 1000, 700)
    pfx = str(tmp_path / "run_")
    assert ctx.dump_raw(pfx) == 0
    assert np.array_equal(np.fromfile(pfx + "sel.bin", np.int32), sel)
    cols = [0, 2, 3, 4, 5, 6]
    assert np.array_equal(dets[:, cols], d[:, cols])
    assert np.all(np.abs(dets[:, 1] - d[:, 1]) <= 2 * np.spacing(np.float32(1.0)))
    assert np.array_equal(masks.reshape(300, -1), m)


def test_result_contract(gpu):
    _, raw, _, dets, masks = gpu
    assert dets.shape == (300, 7) and masks.shape == (300, 200, 200)
    assert np.all(np.diff(dets[:, 1]) <= 0)  # score-descending
    assert set(np.unique(masks)) <= {0, 1}
    assert np.all((dets[:, 0] >= 0) & (dets[:, 0] < 25))
    assert np.array_equal(dets[:, 6], np.round(dets[:, 6]))  # ranks are integers
    assert np.all((dets[:, 6] >= 0) & (dets[:, 6] < 300))


def test_graph_replay_is_bit_identical(gpu, image):
    import ppdoclayout as P

    ctx, raw, _, _, _ = gpu
    for _ in range(2):
        ctx.compute(image)
        for k, w in (("logits", P.RAW_LOGITS), ("boxes", P.RAW_BOXES), ("order", P.RAW_ORDER),
                     ("masks", P.RAW_MASKS)):
            assert np.array_equal(ctx.raw(w), raw[k]), k


def test_time_graph(gpu):
    ctx = gpu[0]
    ms = ctx.time_graph(10)
    say("graph replay %.3f ms/image" % ms)
    assert 0 < ms < 1000


def test_bad_arguments(gpu, image, model):
    import ctypes

    import ppdoclayout as P

    ctx = gpu[0]
    L = P.lib()
    r = P.Result()
    assert L.ppdl_infer(ctx._ctx, image.ctypes.data, 0, 700, ctypes.byref(r)) == 1
    assert L.ppdl_infer(None, image.ctypes.data, 800, 800, ctypes.byref(r)) == 1
    assert L.ppdl_get_raw(ctx._ctx, 9, image.ctypes.data, 10) == -1
    assert L.ppdl_get_raw(ctx._ctx, P.RAW_LOGITS, image.ctypes.data, 10) == -1  # capacity too small
    assert L.ppdl_init(b"/nonexistent.gguf", P.BACKEND_HIP) is None
    assert L.ppdl_init(model[0].encode(), P.BACKEND_CPU) is None  # no CPU backend in this library


def test_dump_raw_files(gpu, tmp_path):
    ctx, raw, _, _, _ = gpu
    pfx = str(tmp_path / "run_")
    assert ctx.dump_raw(pfx) == 0
    lg = np.fromfile(pfx + "logits.bin", np.float32).reshape(300, 25)
    assert np.array_equal(lg, raw["logits"])
    assert os.path.getsize(pfx + "sel.bin") == 300 * 4


def test_cli_matches_api(gpu, model, image, tmp_path):
    """lib/ppdoclayout (the reference CLI's flags and files) on the same model
    and page: out0/out2 equal the API's result, out1 holds the count; batch
    mode writes the same files per manifest line."""
    import subprocess

    cli = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "ppdoclayout-ggml_amd", "lib",
                       "ppdoclayout")
    _, _, _, dets, masks = gpu
    inp = tmp_path / "page.bin"
    image.astype(np.float32).tofile(inp)
    out = tmp_path / "single"
    r = subprocess.run([cli, "-m", model[0], "-i", str(inp), "--ori-h", "1000", "--ori-w", "700", "-o", str(out),
                        "--bench", "2"], capture_output=True, text=True, timeout=240)
    say(r.stdout.strip(), r.stderr.strip().splitlines()[-1:])
    assert r.returncode == 0, r.stderr
    assert "bench_ms mean=" in r.stdout
    assert np.array_equal(np.fromfile(out / "out0.bin", np.float32).reshape(300, 7), dets)
    assert np.fromfile(out / "out1.bin", np.int32).tolist() == [300]
    assert np.array_equal(np.fromfile(out / "out2.bin", np.int32).reshape(300, 200, 200), masks)
    man = tmp_path / "manifest.txt"
    man.write_text("%s|%s|1000|700\n%s|%s|1000|700\n" % (inp, tmp_path / "b0", inp, tmp_path / "b1"))
    r = subprocess.run([cli, "-m", model[0], "--batch", str(man)], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    for d in ("b0", "b1"):
        assert np.array_equal(np.fromfile(tmp_path / d / "out0.bin", np.float32).reshape(300, 7), dets)


def test_chained_winograd_transforms_match(gpu, model, image, monkeypatch):
    """The opt-in chained Winograd transforms (PPDL_WG_CHAIN=1: one kernel
    writes a conv's output and the next conv's transformed input) against
    the default graph on the same page: fewer launches, raw outputs within
    the network tolerance, the same top-300 selection."""
    import ppdoclayout as P

    _, raw, _, _, _ = gpu
    monkeypatch.setenv("PPDL_WG_CHAIN", "1")
    ctx = P.PPDocLayout(model[0], P.BACKEND_HIP)
    try:
        n_default, n_chain = gpu[0].graph_nodes(), ctx.graph_nodes()
        say("graph kernel launches: default", n_default, "chained", n_chain)
        assert n_chain < n_default
        ctx.compute(image)
        topk = ctx.raw(P.RAW_TOPK)
        assert np.array_equal(np.sort(topk), np.sort(raw["topk"]))
        pos = {int(t): i for i, t in enumerate(topk)}
        p = np.array([pos[int(t)] for t in raw["topk"]])  # swaps of tied scores only
        for k, w in (("logits", P.RAW_LOGITS), ("boxes", P.RAW_BOXES), ("order", P.RAW_ORDER),
                     ("masks", P.RAW_MASKS)):
            got = ctx.raw(w)
            got = got[p][:, p] if k == "order" else got[p]
            err = normwise(got, raw[k])
            say("%-10s chained vs default normwise %.3g" % (k, err))
            assert err <= TOL_OUTPUT, (k, err)
    finally:
        ctx.close()


@pytest.mark.parametrize("knob", ["PPDL_DW_ROWS=0", "PPDL_MEMORY=1", "PPDL_UP2X=0"])
def test_exact_variants_match_default(gpu, model, image, monkeypatch, knob):
    """Graph variants that must not change a bit: the depthwise conv with LDS
    staging against the register version (the stride-2 convs), the
    source * valid multiply as its own node against the masked-row LayerNorm
    that replaces it, and the generic interpolation against the exact-2x
    kernels (nearest and bilinear)."""
    import ppdoclayout as P

    _, raw, _, _, _ = gpu
    k, v = knob.split("=")
    monkeypatch.setenv(k, v)
    ctx = P.PPDocLayout(model[0], P.BACKEND_HIP)
    try:
        ctx.compute(image)
        assert np.array_equal(ctx.raw(P.RAW_TOPK), raw["topk"])
        for name, w in (("logits", P.RAW_LOGITS), ("boxes", P.RAW_BOXES), ("order", P.RAW_ORDER),
                        ("masks", P.RAW_MASKS)):
            assert np.array_equal(ctx.raw(w), raw[name]), (knob, name)
    finally:
        ctx.close()


@pytest.mark.parametrize("knob", ["PPDL_ATT16=0", "PPDL_BOX_FUSE=0", "PPDL_SOURCE_TM=1"])
def test_numeric_variants_match_default(gpu, model, image, monkeypatch, knob):
    """Graph variants with another summation order: the attention with 32
    queries per block (v_mfma_f32_32x32x2f32) against the default 16-query
    kernel (v_mfma_f32_16x16x4f32), and each layer's box-head output linear
    + refinement as its own GEMM against the default, where the next
    layer's query-position GEMM computes it in its loader; and the
    token-major source with row-major value / enc_out GEMMs against the
    default channel-major source on the DMA-staged kernel.  Raw outputs
    within the network tolerance, the same top-300 selection up to swaps of
    tied scores."""
    import ppdoclayout as P

    _, raw, _, _, _ = gpu
    k, v = knob.split("=")
    monkeypatch.setenv(k, v)
    ctx = P.PPDocLayout(model[0], P.BACKEND_HIP)
    try:
        ctx.compute(image)
        topk = ctx.raw(P.RAW_TOPK)
        assert np.array_equal(np.sort(topk), np.sort(raw["topk"]))
        pos = {int(t): i for i, t in enumerate(topk)}
        p = np.array([pos[int(t)] for t in raw["topk"]])
        for name, w in (("logits", P.RAW_LOGITS), ("boxes", P.RAW_BOXES), ("order", P.RAW_ORDER),
                        ("masks", P.RAW_MASKS)):
            got = ctx.raw(w)
            got = got[p][:, p] if name == "order" else got[p]
            err = normwise(got, raw[name])
            say("%-10s %s vs default normwise %.3g" % (name, knob, err))
            assert err <= TOL_OUTPUT, (knob, name, err)
    finally:
        ctx.close()
