"""ppdl_hip_run_noalloc against ppdl_hip_run, through the C-ABI.

The no-allocation entry point takes the op's own srcs only and runs the node's
kernels with the library's device scratch array as their workspace (split-K
partials, top-k keys).  With a full caller workspace ppdl_hip_run plans the
same kernels, so the two must agree bit for bit.  Each case makes two calls in
a row, the second on a smaller input, so a result that leaned on what the
first call left in the array would show.  Nodes whose workspace exceeds the
array are rejected before anything is launched.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


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


def conv_case(hip, rng, IC, H, W, OC, K, S, P, act):
    x = rng.random((IC, H, W)).astype(np.float32)
    w = (rng.standard_normal((OC, IC, K, K)) / np.sqrt(K * K * IC)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, OC).astype(np.float32)
    wr, _ = hip.repack_conv(w)
    OH, OW = (H + 2 * P - K) // S + 1, (W + 2 * P - K) // S + 1
    if K == 1:
        op, p14 = hip.OP_CONV1X1_BA, act
    else:
        op, p14 = hip.OP_CONV_IM2COL, K | (S << 8) | (P << 16) | (act << 24)
    return op, p14, [dev(x), dev(wr), dev(b)], (OC, OH, OW)


def both(hip, op, p14, srcs, shape, dtype=torch.float32):
    """(ppdl_hip_run with a full workspace, ppdl_hip_run_noalloc) outputs; both
    outputs start NaN (or -1) so an unwritten element shows."""
    fill = float("nan") if dtype == torch.float32 else -1
    ref = torch.full(shape, fill, dtype=dtype, device="cuda")
    out = torch.full(shape, fill, dtype=dtype, device="cuda")
    nb = hip.workspace_bytes(op, ref, srcs, p14)
    assert 0 <= nb <= hip.NOALLOC_SCRATCH_BYTES
    ws = [hip.make_workspace(nb)] if nb > 0 else []
    hip.run_checked(op, ref, srcs + ws, p14)
    assert hip.run_noalloc(op, out, srcs, p14) == hip.OK
    return host(ref), host(out), nb


@pytest.mark.parametrize("first,second", [
    # split-K 1x1 convs: 10.2 MB of partials, then 1.6 MB
    ((2048, 25, 25, 512, 1, 1, 0, 1), (1024, 20, 20, 256, 1, 1, 0, 2)),
    # split-K implicit-im2col k3 s2 convs, then an unsplit 1x1 (no workspace)
    ((256, 50, 50, 256, 3, 2, 1, 2), (64, 40, 40, 96, 1, 1, 0, 0)),
])
def test_noalloc_matches_run_twice(hip, first, second):
    rng = np.random.default_rng(sum(first) + sum(second))
    for i, shp in enumerate((first, second)):
        say(f"noalloc call {i}: conv IC,H,W,OC,K,S,P,act = {shp}")
        op, p14, srcs, oshape = conv_case(hip, rng, *shp)
        ref, out, nb = both(hip, op, p14, srcs, oshape)
        if i == 0:
            assert nb > 0, "the first call must use the scratch array"
        assert np.isfinite(ref).all()
        assert np.array_equal(ref, out), f"call {i}: noalloc differs from ppdl_hip_run"


def test_noalloc_topk_twice(hip):
    rng = np.random.default_rng(31)
    for i, (nt, nc, nq) in enumerate(((13125, 25, 300), (50, 3, 50))):
        say(f"noalloc call {i}: top-{nq} of {nt} x {nc}")
        lg = rng.standard_normal((nt, nc)).astype(np.float32)
        lg[5:9] = 4.0  # ties: lower index first
        ref, out, nb = both(hip, hip.OP_TOPK, 0, [dev(lg)], (nq,), torch.int32)
        assert nb == 8 * nt
        assert np.array_equal(ref, out)
        assert len(set(out.tolist())) == nq and out.min() >= 0 and out.max() < nt


def test_noalloc_rejects_oversized_and_workspace_src(hip, monkeypatch):
    rng = np.random.default_rng(32)
    # 16 splits of a 1024 x 625 output: 41 MB of partials > the 16 MiB array
    monkeypatch.setenv("PPDL_GEMM_TILE", "3,16")
    op, p14, srcs, oshape = conv_case(hip, rng, 4096, 25, 25, 1024, 1, 1, 0, 0)
    out = torch.full(oshape, 7.0, device="cuda")
    assert hip.workspace_bytes(op, out, srcs, p14) > hip.NOALLOC_SCRATCH_BYTES
    say("noalloc rejects a 41 MB split-K plan")
    assert hip.run_noalloc(op, out, srcs, p14) == hip.EINVAL
    assert (host(out) == 7.0).all(), "a rejected node must launch nothing"
    monkeypatch.delenv("PPDL_GEMM_TILE")
    # a workspace src is not part of this entry point's contract
    ws = hip.make_workspace(1 << 20)
    say("noalloc rejects an attached workspace src")
    assert hip.run_noalloc(op, out, srcs + [ws], p14) == hip.EINVAL
    assert (host(out) == 7.0).all()
