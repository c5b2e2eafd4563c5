"""The single-op benchmark workloads of the tagged-op path (1x1 conv, the F(4,3)
sweep, the im2col convs, MSDeformAttn), as ready-to-launch op lists.

`ConvSuite` holds them at their real shapes: device-resident seeded
inputs, weights repacked once by the library's own repack (as the reference
repacks at load, src/ppdoclayout.cpp:251-346), intermediate buffers, and the
tagged-op nodes that one pass enqueues.  Every launch goes through the C-ABI
(ppdl_hip_run); torch only allocates device memory.
"""
import numpy as np
import torch

import ppdl_hip as H

SEED = 0x5050444C

# (IC, H, W) -> same IC out; 3x3 s1 p1 + SiLU
WINOGRAD_SWEEP = [(256, 100, 100), (256, 50, 50), (256, 25, 25), (48, 200, 200), (96, 100, 100)]
# (IC, IH, IW, OC, K, S, P); the k2 conv's input carries the reference's
# right/bottom pad (ggml_pad by 1, src/ppdoclayout.cpp:621-624)
IM2COL_CONVS = [(48, 401, 401, 24, 2, 1, 0), (256, 100, 100, 256, 3, 2, 1), (256, 50, 50, 256, 3, 2, 1),
                (3, 800, 800, 32, 3, 2, 1)]


def _conv_weights(rng, IC, OC, K):
    w = (rng.standard_normal((OC, IC, K, K)) / np.sqrt(K * K * IC)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, OC).astype(np.float32)
    return w, b


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def msdef_inputs(rng, nq=300):
    """Config 4 inputs (values N(0,1); ref cx,cy U(0,1), w,h U(0.05,1);
    normalised displacement N(0, 0.05) with off = d*8/wh, loc clamped to
    [-0.1, 1.1]; attention logits N(0,1))."""
    val = rng.standard_normal((13125, 256)).astype(np.float32)
    ref = np.concatenate([rng.random((nq, 2)), rng.uniform(0.05, 1.0, (nq, 2))], 1).astype(np.float32)
    d = rng.normal(0.0, 0.05, (nq, 8, 3, 4, 2))
    loc = np.clip(ref[:, None, None, None, :2] + d, -0.1, 1.1)
    off = ((loc - ref[:, None, None, None, :2]) * 8.0 / ref[:, None, None, None, 2:]).astype(np.float32)
    awr = rng.standard_normal((nq, 96)).astype(np.float32)
    return val, off.reshape(nq, 192), awr, ref


class Node:
    """One tagged op: id, params[14]/[15], dst and src tensors, and the
    algorithmic work it represents (GEMM FLOPs or compulsory bytes)."""

    def __init__(self, name, op, dst, srcs, p14=0, p15=0, flops=0.0, bytes_=0.0, kind="gemm"):
        self.name, self.op, self.dst, self.srcs = name, op, dst, srcs
        self.p14, self.p15, self.flops, self.bytes, self.kind = p14, p15, flops, bytes_, kind

    def attach_workspace(self):
        """Append the split-K workspace this GEMM's plan asks for (zeroed once)."""
        nb = H.workspace_bytes(self.op, self.dst, self.srcs, self.p14, self.p15)
        if nb < 0:
            raise H.PpdlError(f"{self.name}: invalid node")
        if nb > 0:
            self.srcs = list(self.srcs) + [H.make_workspace(nb)]
        return nb

    def launch(self, stream):
        rc = H.run(self.op, self.dst, self.srcs, self.p14, self.p15, stream)
        if rc != H.OK:
            raise H.PpdlError(f"{self.name}: ppdl_hip_run returned {rc}")


class ConvSuite:
    """Configs 1-4: one pass = 1 + 5x3 + 4 + 1 = 21 tagged-op launches."""

    def __init__(self, keep_host=False):
        rng = np.random.default_rng(SEED)
        self.nodes = []
        self.host = {} if keep_host else None
        f32 = 4.0

        # 1x1 512->256 @100x100, bias + ReLU fused (op 14)
        x = rng.random((512, 100, 100)).astype(np.float32)
        w, b = _conv_weights(rng, 512, 256, 1)
        wr, _ = H.repack_conv(w)
        out = torch.empty((256, 100, 100), device="cuda")
        P = 100 * 100
        self.nodes.append(Node("c1_conv1x1_512_256_100", H.OP_CONV1X1_BA, out, [_dev(x), _dev(wr), _dev(b)], 1,
                               flops=2.0 * 512 * 256 * P, bytes_=f32 * (512 * P + 256 * 512 + 256 + 256 * P)))
        if keep_host:
            self.host["c1"] = (x, w, b, out)

        # Winograd F(4,3) sweep, SiLU
        for (C, Hh, W) in WINOGRAD_SWEEP:
            x = rng.random((C, Hh, W)).astype(np.float32)
            w, b = _conv_weights(rng, C, C, 3)
            _, wg4 = H.repack_conv(w)
            TW, TH = (W + 3) // 4, (Hh + 3) // 4
            T = TW * TH
            xt, wt, bt = _dev(x), _dev(wg4), _dev(b)
            dt = torch.empty((36, C, T), device="cuda")
            yt = torch.empty((36, C, T), device="cuda")
            out = torch.empty((C, Hh, W), device="cuda")
            tag = f"c2_wg4_{C}_{Hh}"
            self.nodes.append(Node(tag + "_input", H.OP_WG4_INPUT_PAD, dt, [xt], T, TH, kind="xform",
                                   bytes_=f32 * (C * Hh * W + 36 * C * T)))
            self.nodes.append(Node(tag + "_madd", H.OP_WG4_MADD, yt, [dt, wt],
                                   flops=2.0 * 36 * C * C * T, bytes_=f32 * 36 * (C * T + C * C + C * T)))
            self.nodes.append(Node(tag + "_output", H.OP_WG4_OUTPUT, out, [yt, bt], H.ACT_SILU, TW, kind="xform",
                                   bytes_=f32 * (36 * C * T + C + C * Hh * W)))
            if keep_host:
                self.host[tag] = (x, w, b, out)

        # implicit-im2col GEMM convs (op 16), act none
        for (IC, IH, IW, OC, K, S, Pd) in IM2COL_CONVS:
            x = rng.random((IC, IH, IW)).astype(np.float32)
            w, b = _conv_weights(rng, IC, OC, K)
            wr, _ = H.repack_conv(w)
            OH, OW = (IH + 2 * Pd - K) // S + 1, (IW + 2 * Pd - K) // S + 1
            out = torch.empty((OC, OH, OW), device="cuda")
            tag = f"c3_k{K}s{S}_{IC}_{OC}_{IH}"
            self.nodes.append(Node(tag, H.OP_CONV_IM2COL, out, [_dev(x), _dev(wr), _dev(b)],
                                   K | (S << 8) | (Pd << 16),
                                   flops=2.0 * OC * IC * K * K * OH * OW,
                                   bytes_=f32 * (IC * IH * IW + OC * IC * K * K + OC + OC * OH * OW)))
            if keep_host:
                self.host[tag] = (x, w, b, out)

        # MSDeformAttn sampling, 300 queries
        val, off, awr, ref = msdef_inputs(rng)
        out = torch.empty((300, 256), device="cuda")
        self.nodes.append(Node("c4_msdeform", H.OP_MSDEF, out, [_dev(val), _dev(off), _dev(awr), _dev(ref)],
                               kind="sampler",
                               bytes_=f32 * (13125 * 256 + 300 * (192 + 96 + 4) + 300 * 256)))
        if keep_host:
            self.host["c4"] = (val, off, awr, ref, out)
        for n in self.nodes:
            if n.kind == "gemm":
                n.attach_workspace()
        torch.cuda.synchronize()

    def run(self, stream):
        for n in self.nodes:
            n.launch(stream)

    def gemm_flops(self):
        return sum(n.flops for n in self.nodes if n.kind == "gemm")
