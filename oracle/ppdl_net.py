"""CPU restatement of the whole PP-DocLayoutV3 graph and its postprocess.

TEST INFRASTRUCTURE ONLY: the checker for the GPU runtime's end-to-end
outputs (tests/, bench.py's CPU-baseline leg), never part of the product.

It follows the reference's CPU path (the graph of src/ppdoclayout.cpp:363-883
with gpu_convs off, i.e. every conv as F32 im2col + FP32 GEMM, depthwise as
ggml_conv_2d_dw_direct) and its host postprocess (:927-993).  The conv,
deformable-sampling, mask->box and top-300 steps call this directory's C
restatement (oracle.c), each pinned by its own tests; the stock ggml ops
(layer norm, softmax, interpolation, pooling, activations) are restated here
in numpy with the arithmetic ggml's CPU kernels use: float32 elements,
float64 sums where ggml uses ggml_float.

Layouts: images (C, H, W); token tensors (tokens, 256); weights as the GGUF
stores them in numpy order (conv OIHW, linear (out, in)).

Composition pinned: backbone(), encoder() and decode() agree with
transformers' PPDocLayoutV3 (an independent implementation of the network)
evaluated in float64 on the same synthetic weights to <= 1e-5 normwise
(tests/test_net_cpu.py against tests/golden/net_*.npz), with the reference's
one deviation from it followed: the order head reads the pre-dec_norm
hidden state (src/ppdoclayout.cpp:861-866).
"""
import numpy as np

from . import oracle as K

IMG, NQ, NC, DM, NH, HD = 800, 300, 25, 256, 8, 32
MASK_HW = 200
ACT_NONE, ACT_RELU, ACT_SILU = 0, 1, 2
LVL = (100, 50, 25)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def silu(x):
    # ggml CPU silu: x / (1 + expf(-x))
    x = _f32(x)
    return x / (np.float32(1.0) + np.exp(-x))


def sigmoid(x):
    x = _f32(x)
    return np.float32(1.0) / (np.float32(1.0) + np.exp(-x))


def relu(x):
    return np.maximum(_f32(x), np.float32(0.0))


def gelu_erf(x):
    # ggml_gelu_erf: 0.5 x (1 + erf(x / sqrt 2)); erf evaluated in float64
    from scipy.special import erf

    x = _f32(x)
    e = erf(x.astype(np.float64) * (1.0 / np.sqrt(2.0))).astype(np.float32)
    return np.float32(0.5) * x * (np.float32(1.0) + e)


def act(x, a):
    return relu(x) if a == ACT_RELU else silu(x) if a == ACT_SILU else _f32(x)


def layer_norm(x, w, b, eps=1e-5):
    """ggml_norm (mean and variance summed in float64, elements float32)
    then * w + b (src/ppdoclayout.cpp:550-554)."""
    x = _f32(x)
    mean = (x.astype(np.float64).sum(-1, keepdims=True) / x.shape[-1]).astype(np.float32)
    v = x - mean
    var = (v.astype(np.float64) ** 2).sum(-1, keepdims=True) / x.shape[-1]
    scale = (np.float32(1.0) / np.sqrt(np.float32(var + eps))).astype(np.float32)
    return (v * scale) * _f32(w) + _f32(b)


def softmax_rows(x):
    """ggml_soft_max over the last axis: exp(x - max) in float32, sum in float64."""
    x = _f32(x)
    e = np.exp(x - x.max(-1, keepdims=True))
    s = e.astype(np.float64).sum(-1, keepdims=True)
    return (e * (1.0 / s).astype(np.float32)).astype(np.float32)


def interp_nearest(x, OH, OW):
    C, IH, IW = x.shape
    iy = (np.arange(OH) * IH) // OH
    ix = (np.arange(OW) * IW) // OW
    return _f32(x[:, iy][:, :, ix])


def interp_bilinear(x, OH, OW):
    """ggml_interpolate bilinear, half-pixel centres, edge clamped."""
    x = _f32(x)
    C, IH, IW = x.shape

    def axis(O, I):
        sf = np.float32(O) / np.float32(I)
        f = (np.arange(O, dtype=np.float32) + np.float32(0.5)) / sf - np.float32(0.5)
        fl = np.floor(f)
        i0 = fl.astype(np.int64)
        i1 = i0 + 1
        d = np.clip(f - fl, 0.0, 1.0).astype(np.float32)
        return np.clip(i0, 0, I - 1), np.clip(i1, 0, I - 1), d

    y0, y1, dy = axis(OH, IH)
    x0, x1, dx = axis(OW, IW)
    a = x[:, y0][:, :, x0]
    b = x[:, y0][:, :, x1]
    c = x[:, y1][:, :, x0]
    d = x[:, y1][:, :, x1]
    dx = dx[None, None, :]
    dy = dy[None, :, None]
    one = np.float32(1.0)
    return _f32(a * (one - dx) * (one - dy) + b * dx * (one - dy) + c * (one - dx) * dy + d * dx * dy)


def dwconv(x, w, bias, s, p, a):
    """ggml_conv_2d_dw_direct + bias + act: taps accumulated in (kh, kw) order."""
    x, w = _f32(x), _f32(w)
    C, IH, IW = x.shape
    k = w.shape[-1]
    OH, OW = (IH + 2 * p - k) // s + 1, (IW + 2 * p - k) // s + 1
    xp = np.pad(x, ((0, 0), (p, p), (p, p)))
    out = np.zeros((C, OH, OW), np.float32)
    for kh in range(k):
        for kw in range(k):
            tap = xp[:, kh:kh + s * (OH - 1) + 1:s, kw:kw + s * (OW - 1) + 1:s]
            out = out + tap * w[:, 0, kh, kw][:, None, None]
    return act(out + _f32(bias)[:, None, None], a)


def maxpool2_padend(x):
    """ggml_pad(x, 1, 1) then 2x2 stride-1 max pool (src/ppdoclayout.cpp:621-626)."""
    xp = np.pad(_f32(x), ((0, 0), (0, 1), (0, 1)))
    return np.maximum(np.maximum(xp[:, :-1, :-1], xp[:, :-1, 1:]), np.maximum(xp[:, 1:, :-1], xp[:, 1:, 1:]))


class Net:
    """The graph of src/ppdoclayout.cpp:733-882 over a weight dict."""

    def __init__(self, weights, threads=0):
        self.w = weights
        self.threads = threads
        self.dumps = {}

    def W(self, name):
        return self.w[name]

    def dump(self, name, t):
        self.dumps[name] = np.array(t, copy=True)

    # builder::conv on the CPU backend (:388-404, :535-542)
    def conv(self, x, name, s, p, a, pad_end=0):
        w, b = self.W(name + ".weight"), self.W(name + ".bias")
        if w.shape[1] == 1 and x.shape[0] != 1:
            return dwconv(x, w, b, s, p, a)
        if pad_end:
            x = np.pad(x, ((0, 0), (0, pad_end), (0, pad_end)))
        return K.conv2d_ref(x, w, b, stride=s, pad=p, act=a, nthreads=self.threads)

    def lin(self, x, name):
        # ggml_mul_mat(W, x) + b (:545-548)
        return _f32(_f32(x) @ self.W(name + ".weight").T) + self.W(name + ".bias")

    def ln(self, x, name):
        return layer_norm(x, self.W(name + ".weight"), self.W(name + ".bias"))

    def mlp3(self, x, pfx):
        x = relu(self.lin(x, pfx + ".0"))
        x = relu(self.lin(x, pfx + ".1"))
        return self.lin(x, pfx + ".2")

    def mha(self, qk_in, v_in, pfx):
        """8 heads x 32 (:572-587): softmax(q k^T / sqrt 32) v, then .o."""
        T = qk_in.shape[0]
        q = self.lin(qk_in, pfx + ".q").reshape(T, NH, HD).transpose(1, 0, 2)
        k = self.lin(qk_in, pfx + ".k").reshape(T, NH, HD).transpose(1, 0, 2)
        v = self.lin(v_in, pfx + ".v").reshape(T, NH, HD).transpose(1, 0, 2)
        kq = _f32(np.matmul(q, k.transpose(0, 2, 1))) * np.float32(1.0 / np.sqrt(np.float32(HD)))
        att = _f32(np.matmul(softmax_rows(kq), v))  # (8, T, 32)
        return self.lin(att.transpose(1, 0, 2).reshape(T, DM), pfx + ".o")

    def hg_block(self, x, pfx, light):
        cat = [x]
        cur = x
        for l in range(6):
            lp = "%s.l%d" % (pfx, l)
            if light:
                cur = self.conv(cur, lp + ".c1", 1, 0, ACT_NONE)
                cur = self.conv(cur, lp + ".c2", 1, 2, ACT_RELU)
            else:
                cur = self.conv(cur, lp, 1, 1, ACT_RELU)
            cat.append(cur)
        y = self.conv(np.concatenate(cat, 0), pfx + ".agg0", 1, 0, ACT_RELU)
        return self.conv(y, pfx + ".agg1", 1, 0, ACT_RELU)

    def backbone(self, img):
        # :616-652
        x = self.conv(img, "stem1", 2, 1, ACT_RELU)
        self.dump("stem1", x)
        a = self.conv(x, "stem2a", 1, 0, ACT_RELU, pad_end=1)
        a = self.conv(a, "stem2b", 1, 0, ACT_RELU, pad_end=1)
        x = np.concatenate([maxpool2_padend(x), a], 0)
        x = self.conv(x, "stem3", 2, 1, ACT_RELU)
        x = self.conv(x, "stem4", 1, 0, ACT_RELU)
        self.dump("stem", x)
        s0 = self.hg_block(x, "st0.b0", False)
        self.dump("st0", s0)
        s1 = self.hg_block(self.conv(s0, "st1.ds", 2, 1, ACT_NONE), "st1.b0", False)
        self.dump("st1", s1)
        s2 = self.hg_block(self.conv(s1, "st2.ds", 2, 1, ACT_NONE), "st2.b0", True)
        s2 = self.hg_block(s2, "st2.b1", True) + s2
        s2 = self.hg_block(s2, "st2.b2", True) + s2
        self.dump("st2", s2)
        s3 = self.hg_block(self.conv(s2, "st3.ds", 2, 1, ACT_NONE), "st3.b0", True)
        self.dump("st3", s3)
        return s0, s1, s2, s3

    def csp(self, x, pfx):
        # :656-668; repvgg = silu(c1_3x3(a) + c2_1x1(a))
        a = self.conv(x, pfx + ".c1", 1, 0, ACT_SILU)
        for i in range(3):
            bp = "%s.bn%d" % (pfx, i)
            a = silu(self.conv(a, bp + ".c1", 1, 1, ACT_NONE) + self.conv(a, bp + ".c2", 1, 0, ACT_NONE))
        return a + self.conv(x, pfx + ".c2", 1, 0, ACT_SILU)

    def aifi(self, s, pos):
        """The one AIFI encoder layer on tokens s (T, 256) with position
        embedding pos (T, 256): post-norm attention + GELU FFN (:681-693)."""
        at = self.mha(s + pos, s, "aifi")
        s = self.ln(s + at, "aifi.ln1")
        ff = self.lin(gelu_erf(self.lin(s, "aifi.fc1")), "aifi.fc2")
        return self.ln(s + ff, "aifi.ln2")

    def encoder(self, x4, p8r, p16r, p32r, pos=None):
        """:674-729.  The reference fixes the 800x800 geometry (p32 25x25,
        p16 50x50, p8 100x100, masks 200x200); every resize here is the 2x
        step those sizes imply, so smaller maps follow the same graph."""
        p8 = self.conv(p8r, "enc_in0", 1, 0, ACT_NONE)
        p16 = self.conv(p16r, "enc_in1", 1, 0, ACT_NONE)
        p32 = self.conv(p32r, "enc_in2", 1, 0, ACT_NONE)
        h32, w32 = p32.shape[1:]
        if pos is None:
            pos = pos_embed(h32, w32)
        s = p32.reshape(DM, -1).T.copy()  # to_seq: token = y*W + x
        p32 = self.aifi(s, pos).T.reshape(DM, h32, w32).copy()
        self.dump("aifi", p32)
        lat0 = self.conv(p32, "lat0", 1, 0, ACT_SILU)
        f16 = self.csp(np.concatenate([interp_nearest(lat0, 2 * h32, 2 * w32), p16], 0), "fpn0")
        lat1 = self.conv(f16, "lat1", 1, 0, ACT_SILU)
        h16, w16 = f16.shape[1:]
        f8 = self.csp(np.concatenate([interp_nearest(lat1, 2 * h16, 2 * w16), p8], 0), "fpn1")
        self.dump("f8", f8)
        h8, w8 = f8.shape[1:]
        n16 = self.csp(np.concatenate([self.conv(f8, "pand0", 2, 1, ACT_SILU), lat1], 0), "pan0")
        self.dump("n16", n16)
        n32 = self.csp(np.concatenate([self.conv(n16, "pand1", 2, 1, ACT_SILU), lat0], 0), "pan1")
        self.dump("n32", n32)
        h0 = self.conv(f8, "mh0.0", 1, 1, ACT_SILU)
        h1 = interp_bilinear(self.conv(n16, "mh1.0", 1, 1, ACT_SILU), h8, w8)
        h2 = interp_bilinear(self.conv(n32, "mh2.0", 1, 1, ACT_SILU), h16, w16)
        h2 = interp_bilinear(self.conv(h2, "mh2.2", 1, 1, ACT_SILU), h8, w8)
        mf = (h0 + h1) + h2
        mf = interp_bilinear(self.conv(mf, "mh.out", 1, 1, ACT_SILU), 2 * h8, 2 * w8)
        mf = mf + self.conv(x4, "mlat", 1, 1, ACT_SILU)
        mf = self.conv(mf, "mout.base", 1, 1, ACT_SILU)
        mf = self.conv(mf, "mout.conv", 1, 0, ACT_NONE)
        self.dump("mask_feat", mf)
        return f8, n16, n32, mf

    def decoder_layer(self, i, x, ref, source):
        """Decoder layer i (:824-846): self-attention with the query
        position MLP of ref, deformable cross-attention into source, FFN;
        post-norm after each."""
        dp = "dec%d" % i
        qpos = self.lin(relu(self.lin(ref, "qpos.0")), "qpos.1")
        x = self.ln(x + self.mha(x + qpos, x, dp + ".sa"), dp + ".ln1")
        z = x + qpos
        ca = K.msdeform(self.lin(source, dp + ".ca.vp"), self.lin(z, dp + ".ca.so"),
                        self.lin(z, dp + ".ca.aw"), ref, nthreads=self.threads)
        x = self.ln(x + self.lin(ca, dp + ".ca.op"), dp + ".ln2")
        return self.ln(x + self.lin(relu(self.lin(x, dp + ".fc1")), dp + ".fc2"), dp + ".ln3")

    def decode(self, f8, n16, n32, mf):
        """Everything after the hybrid encoder (:733-882) at the 800x800
        geometry: decoder inputs, query selection, mask-derived initial
        boxes, six refining decoder layers and the heads."""
        mflat = mf.reshape(32, -1)  # (32, 40000)
        source = np.concatenate([self.conv(f, "dec_in%d" % i, 1, 0, ACT_NONE).reshape(DM, -1).T
                                 for i, f in enumerate((f8, n16, n32))], 0)
        self.dump("source", source)
        memory = source * valid_mask()[:, None]
        om = self.ln(self.lin(memory, "enc_out.l"), "enc_out.ln")
        ecls = self.lin(om, "score_head")
        self.dump("enc_logits", ecls)
        topk = K.topk(ecls, NQ)
        self.dump("topk_idx", topk)
        target = om[topk]
        self.dump("target", target)
        mq0 = self.mlp3(self.ln(target, "dec_norm"), "mq")
        encm = _f32(mq0 @ mflat)
        self.dump("enc_masks", encm)
        refu = K.mask_box(encm)
        self.dump("init_ref_unact", refu)
        ref = sigmoid(refu)
        x = target
        for i in range(6):
            x = self.decoder_layer(i, x, ref, source)
            self.dump("hidden%d" % i, x)
            ref = sigmoid(self.mlp3(x, "bbox_head") + inv_sigmoid(ref))
        outq = self.ln(x, "dec_norm")
        mq = self.mlp3(outq, "mq")
        self.dump("mq", mq)
        # the order head reads the last hidden state before dec_norm (:861-866)
        gp = self.lin(self.lin(x, "order5"), "gp")
        self.dump("gp", gp)
        return {
            "logits": self.lin(outq, "score_head"),
            "boxes": ref,
            "masks": _f32(mq @ mflat),
            "order": _f32(gp[:, :64] @ gp[:, 64:].T) * np.float32(1.0 / 8.0),
            "topk": topk,
            "init_ref": refu,
        }

    def forward(self, img):
        """-> dict of raw outputs: logits (300, 25), boxes (300, 4), order
        (300, 300) with [i][j] = q_i . k_j / 8, masks (300, 40000)."""
        self.dumps = {}
        x4, p8, p16, p32 = self.backbone(_f32(img))
        f8, n16, n32, mf = self.encoder(x4, p8, p16, p32, pos_embed())
        return self.decode(f8, n16, n32, mf)


def inv_sigmoid(x):
    # :589-594
    x = np.clip(_f32(x), 0.0, 1.0)
    x1 = np.clip(x, 1e-5, 1.0).astype(np.float32)
    x2 = np.clip(np.float32(1.0) - x, 1e-5, 1.0).astype(np.float32)
    return np.log(x1) - np.log(x2)


def pos_embed(h=25, w=25):
    """(h*w, 256) [sin_h | cos_h | sin_w | cos_w], float64 math (:887-903)."""
    omega = 1.0 / np.power(10000.0, np.arange(64) / 64.0)
    hh = np.repeat(np.arange(h), w).astype(np.float64)[:, None]
    ww = np.tile(np.arange(w), h).astype(np.float64)[:, None]
    return np.concatenate([np.sin(hh * omega), np.cos(hh * omega), np.sin(ww * omega), np.cos(ww * omega)],
                          1).astype(np.float32)


def valid_mask():
    """(13125,) anchor validity (:905-923): centre inside (eps, 1-eps), eps 1e-2."""
    out = []
    eps = np.float32(1e-2)
    for l, n in enumerate(LVL):
        wh = np.float32(0.05) * np.float32(2.0 ** l)
        c = (np.arange(n, dtype=np.float32) + np.float32(0.5)) / np.float32(n)
        okc = (c > eps) & (c < np.float32(1.0) - eps)
        ok = okc[:, None] & okc[None, :] & bool(wh > eps and wh < np.float32(1.0) - eps)
        out.append(ok.reshape(-1).astype(np.float32))
    return np.concatenate(out)


def postprocess(logits, boxes, order, masks, ori_h, ori_w):
    """Host postprocess (:927-993) -> (dets (300, 7), masks int32 (300, 40000), sel (300,)).

    order[i][j] = q_i . k_j / 8 (the reference's order[j + 300 i]); votes[j] =
    sum_{i != j} sigmoid(order[i][j] - order[j][i]) summed in float32 in i
    order; ranks by stable sort of votes; top-300 of the 7500 sigmoid scores,
    ties to the lower flat index."""
    logits, boxes, order = _f32(logits), _f32(boxes), _f32(order)
    d = order - order.T  # d[i][j] = order[i][j] - order[j][i]
    sg = np.float32(1.0) / (np.float32(1.0) + np.exp(-d))
    votes = np.zeros(NQ, np.float32)
    for i in range(NQ):  # float32 accumulation in i order, skipping i == j
        row = sg[i].copy()
        row[i] = 0.0
        votes = votes + row
    # note: adding 0 for i == j leaves the float32 running sum unchanged
    rank_of = np.argsort(votes, kind="stable")
    order_seq = np.empty(NQ, np.int64)
    order_seq[rank_of] = np.arange(NQ)
    scores = (np.float32(1.0) / (np.float32(1.0) + np.exp(-logits))).reshape(-1)
    flat = np.lexsort((np.arange(scores.size), -scores.astype(np.float64)))[:NQ]
    sf_h, sf_w = np.float32(IMG) / np.float32(ori_h), np.float32(IMG) / np.float32(ori_w)
    oh = np.floor(np.float32(IMG) / sf_h + np.float32(0.5))
    ow = np.floor(np.float32(IMG) / sf_w + np.float32(0.5))
    q, c = flat // NC, flat % NC
    b = boxes[q]
    half = np.float32(0.5)
    dets = np.stack([c.astype(np.float32), scores[flat],
                     (b[:, 0] - b[:, 2] * half) * ow, (b[:, 1] - b[:, 3] * half) * oh,
                     (b[:, 0] + b[:, 2] * half) * ow, (b[:, 1] + b[:, 3] * half) * oh,
                     order_seq[q].astype(np.float32)], 1).astype(np.float32)
    m = (_f32(masks)[q] > 0).astype(np.int32)
    return dets, m, flat.astype(np.int32)
