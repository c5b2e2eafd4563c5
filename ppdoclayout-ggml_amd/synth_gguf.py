"""PP-DocLayoutV3 model files with random weights.

No checkpoint can be downloaded here, so the full network runs on weights of
the right architecture drawn from a seeded generator.  `tensor_specs()` lists
every tensor the graph reads, with the names and numpy shapes the reference's
converter writes (scripts/convert.py:17-67 renames, :90-127 BN folding into
conv weight/bias, :132-143 GGUF layout); `write_gguf()` writes a GGUF v3 file
in the same layout (F32 tensors sorted by name, 32-byte alignment, the
converter's four ppdlv3.* keys); `read_gguf()` reads one back for checking.

Backbone stage table (in, mid, out, blocks, light, kernel) follows the graph
in src/ppdoclayout.cpp:616-652 (HGNetV2 with 6 layers per block).
"""
import struct

import numpy as np

DM = 256
STAGES = [  # (in, mid, out, blocks, light, k)
    (48, 48, 128, 1, False, 3),
    (128, 96, 512, 1, False, 3),
    (512, 192, 1024, 3, True, 5),
    (1024, 384, 2048, 1, True, 5),
]
ALIGN = 32
GGML_F32 = 0


def tensor_specs():
    """[(name, numpy shape, kind)] for every tensor of the model.

    kind: conv_relu / conv_silu / conv_lin (conv followed by ReLU, SiLU or
    nothing), dw (depthwise), lin / lin_relu, ln, head (score head),
    small (last layer of a refinement head), so (sampling offsets)."""
    s = []

    def conv(name, oc, ic, k, kind):
        s.append((name + ".weight", (oc, ic, k, k), kind))
        s.append((name + ".bias", (oc,), kind))

    def lin(name, out, inp, kind="lin"):
        s.append((name + ".weight", (out, inp), kind))
        s.append((name + ".bias", (out,), kind))

    def ln(name):
        s.append((name + ".weight", (DM,), "ln"))
        s.append((name + ".bias", (DM,), "ln"))

    conv("stem1", 32, 3, 3, "conv_relu")
    conv("stem2a", 16, 32, 2, "conv_relu")
    conv("stem2b", 32, 16, 2, "conv_relu")
    conv("stem3", 32, 64, 3, "conv_relu")
    conv("stem4", 48, 32, 1, "conv_relu")
    for si, (cin, mid, cout, nb, light, k) in enumerate(STAGES):
        if si > 0:
            conv("st%d.ds" % si, cin, 1, 3, "dw_lin")
        for b in range(nb):
            bin_ = cin if b == 0 else cout
            for l in range(6):
                lin_ = bin_ if l == 0 else mid
                lp = "st%d.b%d.l%d" % (si, b, l)
                if light:
                    conv(lp + ".c1", mid, lin_, 1, "conv_lin")
                    conv(lp + ".c2", mid, 1, k, "dw_relu")
                else:
                    conv(lp, mid, lin_, 3, "conv_relu")
            conv("st%d.b%d.agg0" % (si, b), cout // 2, bin_ + 6 * mid, 1, "conv_relu")
            conv("st%d.b%d.agg1" % (si, b), cout, cout // 2, 1, "conv_relu")

    for i, c in enumerate((512, 1024, 2048)):
        conv("enc_in%d" % i, DM, c, 1, "conv_lin")
    for p in ("q", "k", "v", "o"):
        lin("aifi." + p, DM, DM)
    ln("aifi.ln1")
    ln("aifi.ln2")
    lin("aifi.fc1", 1024, DM, "lin_relu")
    lin("aifi.fc2", DM, 1024)
    for i in range(2):
        conv("lat%d" % i, DM, DM, 1, "conv_silu")
        conv("pand%d" % i, DM, DM, 3, "conv_silu")
    for blk in ("fpn0", "fpn1", "pan0", "pan1"):
        conv(blk + ".c1", DM, 2 * DM, 1, "conv_silu")
        conv(blk + ".c2", DM, 2 * DM, 1, "conv_silu")
        for i in range(3):
            conv("%s.bn%d.c1" % (blk, i), DM, DM, 3, "conv_half")
            conv("%s.bn%d.c2" % (blk, i), DM, DM, 1, "conv_half")
    for i in range(3):
        conv("mh%d.0" % i, 64, DM, 3, "conv_silu")
    conv("mh2.2", 64, 64, 3, "conv_silu")
    conv("mh.out", 64, 64, 3, "conv_silu")
    conv("mlat", 64, 128, 3, "conv_silu")
    conv("mout.base", 64, 64, 3, "conv_silu")
    conv("mout.conv", 32, 64, 1, "mask_out")
    for i in range(3):
        conv("dec_in%d" % i, DM, DM, 1, "conv_lin")
    lin("enc_out.l", DM, DM, "enc_out")
    s.append(("enc_out.ln.weight", (DM,), "ln"))
    s.append(("enc_out.ln.bias", (DM,), "enc_out"))
    lin("score_head", 25, DM, "head")
    lin("bbox_head.0", DM, DM, "lin_relu")
    lin("bbox_head.1", DM, DM, "lin_relu")
    lin("bbox_head.2", 4, DM, "small")
    for d in range(6):
        dp = "dec%d" % d
        for p in ("q", "k", "v"):
            lin(dp + ".sa." + p, DM, DM)
        lin(dp + ".sa.o", DM, DM, "res_out")
        ln(dp + ".ln1")
        ln(dp + ".ln2")
        ln(dp + ".ln3")
        lin(dp + ".ca.so", 192, DM, "so")
        lin(dp + ".ca.aw", 96, DM)
        lin(dp + ".ca.vp", DM, DM)
        lin(dp + ".ca.op", DM, DM, "res_out")
        lin(dp + ".fc1", 1024, DM, "lin_relu")
        lin(dp + ".fc2", DM, 1024, "res_out")
    lin("qpos.0", 512, 4, "lin_relu")
    lin("qpos.1", DM, 512)
    ln("dec_norm")
    lin("mq.0", DM, DM, "lin_relu")
    lin("mq.1", DM, DM, "lin_relu")
    lin("mq.2", 32, DM, "mask_out")
    lin("order5", DM, DM)
    lin("gp", 128, DM)
    return s


def random_weights(seed=0):
    """name -> float32 array.  Scales keep activations O(1) through the
    network: He-style for layers followed by ReLU/SiLU, 1/sqrt(fan_in)
    otherwise, damped where branches are summed (repvgg), feed the mask
    logits or join a decoder residual (so the queries stay distinct); the score head's bias is set so that a few dozen detections
    score above 0.3, and the last refinement layer gets small weights."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape, kind in tensor_specs():
        is_w = name.endswith(".weight")
        if kind == "ln":
            base = 1.0 if is_w else 0.0
            a = base + 0.05 * rng.standard_normal(shape)
        elif is_w:
            fan_in = int(np.prod(shape[1:]))
            gain = {"conv_relu": 2.0, "dw_relu": 2.0, "conv_silu": 1.5, "lin_relu": 2.0, "conv_half": 0.6,
                    "small": 0.01, "so": 0.05, "mask_out": 0.25, "head": 3.0,
                    "res_out": 0.05}.get(kind, 1.0)
            a = rng.standard_normal(shape) * np.sqrt(gain / fan_in)
        else:
            if kind == "head":
                a = -3.5 + 0.7 * rng.standard_normal(shape)
            elif kind == "so":
                a = rng.standard_normal(shape)
            elif kind == "enc_out":
                # masked-out anchors (memory row 0) then map to om = 0 and
                # score at the head's bias, below the real tokens
                a = np.zeros(shape)
            else:
                a = 0.05 * rng.standard_normal(shape)
        out[name] = a.astype(np.float32)
    return out


def _str(b):
    b = b.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, tensors, kv_u32=None, description="PP-DocLayoutV3 F32, BN folded"):
    """Write `tensors` (name -> float32 array) as a GGUF v3 file: ne is the
    reversed numpy shape (ne[0] fastest), data F32, every tensor at a
    32-byte aligned offset."""
    if kv_u32 is None:
        kv_u32 = {"ppdlv3.d_model": 256, "ppdlv3.decoder_layers": 6,
                  "ppdlv3.num_queries": 300, "ppdlv3.num_classes": 25}
    names = sorted(tensors)
    kvs = [("general.architecture", 8, "pp-doclayout-v3"), ("general.description", 8, description)]
    kvs += [(k, 4, int(v)) for k, v in kv_u32.items()]
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(names), len(kvs)))
    for key, ty, val in kvs:
        head += _str(key) + struct.pack("<I", ty)
        head += _str(val) if ty == 8 else struct.pack("<I", val)
    offset = 0
    offsets = []
    for n in names:
        a = tensors[n]
        assert a.dtype == np.float32 and len(n) < 64
        head += _str(n) + struct.pack("<I", a.ndim)
        for d in reversed(a.shape):
            head += struct.pack("<Q", d)
        head += struct.pack("<IQ", GGML_F32, offset)
        offsets.append(offset)
        offset += (a.nbytes + ALIGN - 1) // ALIGN * ALIGN
    head += b"\0" * ((-len(head)) % ALIGN)
    with open(path, "wb") as f:
        f.write(head)
        for n, off in zip(names, offsets):
            a = np.ascontiguousarray(tensors[n])
            f.write(a.tobytes())
            f.write(b"\0" * ((-a.nbytes) % ALIGN))


def read_gguf(path):
    """(kv dict, name -> float32 array) of a GGUF v2/v3 file with F32
    tensors; enough to check files written by write_gguf or the converter."""
    data = open(path, "rb").read()
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from("<" + fmt, data, pos)
        pos += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def sval():
        n = take("Q")
        nonlocal pos
        s = data[pos:pos + n].decode()
        pos += n
        return s

    if data[:4] != b"GGUF":
        raise ValueError("not a GGUF file")
    pos = 4
    version, nt, nkv = take("I"), take("Q"), take("Q")
    if version not in (2, 3):
        raise ValueError("unsupported GGUF version %d" % version)
    scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "B", 10: "Q", 11: "q", 12: "d"}
    kv = {}
    for _ in range(nkv):
        key = sval()
        ty = take("I")
        if ty == 8:
            kv[key] = sval()
        elif ty == 9:
            et, n = take("I"), take("Q")
            kv[key] = [sval() if et == 8 else take(scalar[et]) for _ in range(n)]
        else:
            kv[key] = take(scalar[ty])
    align = int(kv.get("general.alignment", ALIGN))
    infos = []
    for _ in range(nt):
        name = sval()
        nd = take("I")
        ne = [take("Q") for _ in range(nd)]
        ty, off = take("I"), take("Q")
        infos.append((name, ne, ty, off))
    base = (pos + align - 1) // align * align
    out = {}
    for name, ne, ty, off in infos:
        if ty != GGML_F32:
            raise ValueError("tensor %s is not F32" % name)
        n = int(np.prod(ne))
        a = np.frombuffer(data, np.float32, n, base + off)
        out[name] = a.reshape(tuple(reversed(ne))).copy()
    return kv, out


def write_random_model(path, seed=0):
    w = random_weights(seed)
    write_gguf(path, w)
    return w


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="write a random-weight PP-DocLayoutV3 GGUF")
    ap.add_argument("out")
    ap.add_argument("--seed", type=int, default=0)
    a = ap.parse_args()
    w = write_random_model(a.out, a.seed)
    print("wrote %s: %d tensors, %.1f M parameters" % (a.out, len(w), sum(x.size for x in w.values()) / 1e6))
