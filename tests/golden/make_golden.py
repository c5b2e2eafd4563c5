"""Writes the golden fixtures under tests/golden/ (run from the repo root:
`python tests/golden/make_golden.py`).

The reference commits no golden vectors for this path, so the fixtures come
from library routines that fix the mathematics, evaluated in float64 on the
CPU with torch:
  * conv_*.npz   torch.nn.functional.conv2d (cross-correlation) + bias + act
  * msdef_*.npz  torch.nn.functional.grid_sample (bilinear, zeros,
                 align_corners=False) per level on the head-split value map,
                 weighted by the softmax over the 12 (level, point) logits
                 and summed: the textbook MSDeformAttn reduction that
                 op_msdeform (src/ppdoclayout.cpp:148-198) restates.
Inputs are float32; expected outputs are float64.  The MSDeformAttn value map
is regenerated from an integer hash (fixture_inputs.py) rather than stored.  The first conv fixture
uses the deterministic pattern of the reference's Winograd check
(bench/wg_test.cu:97-101) at its 10x9x3 -> 2 shape, with a 3x3 s1 p1 conv.
"""
import os

import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from fixture_inputs import msdef_value_map  # noqa: E402


def conv_case(name, x, w, b, stride, pad, act):
    y = F.conv2d(torch.from_numpy(x[None].astype(np.float64)), torch.from_numpy(w.astype(np.float64)),
                 torch.from_numpy(b.astype(np.float64)), stride=stride, padding=pad)[0]
    if act == 1:
        y = torch.relu(y)
    elif act == 2:
        y = y * torch.sigmoid(y)
    np.savez(os.path.join(HERE, f"conv_{name}.npz"), x=x, w=w, b=b,
             meta=np.array([stride, pad, act], np.int32), y=y.numpy())


def wgtest_pattern(IC, H, W, OC):
    n_x = IC * H * W
    x = (np.sin(0.7 * np.arange(n_x, dtype=np.float32)) * 0.5).astype(np.float32).reshape(IC, H, W)
    w = (np.cos(0.3 * np.arange(OC * IC * 9, dtype=np.float32)) * 0.4).astype(np.float32).reshape(OC, IC, 3, 3)
    b = (0.1 * np.arange(OC, dtype=np.float32)).astype(np.float32)
    return x, w, b


def msdef_case(name, nq, seed):
    rng = np.random.default_rng(seed)
    lv = [100, 50, 25]
    val = msdef_value_map(seed)
    ref = np.concatenate([rng.random((nq, 2)), rng.uniform(0.05, 1.0, (nq, 2))], 1).astype(np.float32)
    off = (rng.standard_normal((nq, 192)) * 2.0).astype(np.float32)
    awr = rng.standard_normal((nq, 96)).astype(np.float32)
    # float64 reduction with grid_sample
    v64 = torch.from_numpy(val.astype(np.float64))
    o = torch.from_numpy(off.astype(np.float64)).view(nq, 8, 3, 4, 2)
    r = torch.from_numpy(ref.astype(np.float64))
    a = torch.softmax(torch.from_numpy(awr.astype(np.float64)).view(nq, 8, 12), -1).view(nq, 8, 3, 4)
    loc = r[:, None, None, None, :2] + o / 4.0 * r[:, None, None, None, 2:] * 0.5  # (nq,8,3,4,2)
    out = torch.zeros(nq, 8, 32, dtype=torch.float64)
    st = 0
    for l, W in enumerate(lv):
        vm = v64[st:st + W * W].view(W, W, 8, 32).permute(2, 3, 0, 1)  # (8, 32, H, W)
        grid = (loc[:, :, l] * 2.0 - 1.0).permute(1, 0, 2, 3)  # (8, nq, 4, 2)
        s = F.grid_sample(vm, grid, mode="bilinear", padding_mode="zeros", align_corners=False)  # (8,32,nq,4)
        out += (s.permute(2, 0, 1, 3) * a[:, :, l][:, :, None, :]).sum(-1)
        st += W * W
    np.savez(os.path.join(HERE, f"msdef_{name}.npz"), val_salt=np.array(seed), off=off, awr=awr,
             ref=ref, y=out.reshape(nq, 256).numpy())


def main():
    rng = np.random.default_rng(20261201)
    x, w, b = wgtest_pattern(3, 9, 10, 2)
    conv_case("wgtest_k3s1p1", x, w, b, 1, 1, 0)
    conv_case("wgtest_k3s1p1_silu", x, w, b, 1, 1, 2)
    shapes = [  # name, IC, H, W, OC, K, S, P, act
        ("k1_relu", 16, 7, 9, 12, 1, 1, 0, 1),
        ("k2s1p0", 6, 11, 11, 5, 2, 1, 0, 1),
        ("k3s2p1", 5, 13, 12, 7, 3, 2, 1, 2),
        ("k3s1p1_odd", 9, 13, 17, 6, 3, 1, 1, 2),
    ]
    for name, IC, H, W, OC, K, S, P, act in shapes:
        xx = rng.random((IC, H, W)).astype(np.float32)
        ww = (rng.standard_normal((OC, IC, K, K)) / np.sqrt(K * K * IC)).astype(np.float32)
        bb = rng.uniform(-0.1, 0.1, OC).astype(np.float32)
        conv_case(name, xx, ww, bb, S, P, act)
    msdef_case("nq7", 7, 7)


if __name__ == "__main__":
    main()
