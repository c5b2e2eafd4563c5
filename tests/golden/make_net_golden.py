"""Writes tests/golden/net_*.npz: PP-DocLayoutV3 pieces evaluated by the
transformers implementation (run from the repo root:
`python tests/golden/make_net_golden.py`; needs torch and transformers, which
the tests themselves do not).

transformers' PPDocLayoutV3ForObjectDetection (models/pp_doclayout_v3 of the
installed transformers) is an implementation of the network written
independently of the reference's ggml graph, so it pins the composition the
oracle restates: which tensor feeds which layer, the order of norms,
residuals and activations, the resize steps and the query selection.

Weights: the synthetic model of synth_gguf.random_weights(seed) (GGUF names,
BatchNorm already folded into the convs) is loaded into the transformers
model through the reference converter's renames (scripts/convert.py:17-67,
restated below in the opposite direction) with the fold undone: each folded
conv (w, b) gets a seeded BatchNorm (gamma, beta, mean, var) and the
unfolded weight w / s, s = gamma / sqrt(var + 1e-5), beta = b + mean * s, so
that the converter's fold (scripts/convert.py:99-103) maps the transformers
parameters back to exactly the GGUF tensors; the script asserts that.

Everything runs in float64.  Inputs are seeded numpy arrays the tests
regenerate (net_inputs below), outputs are stored as float32.

Fixtures
  net_backbone.npz  HGNetV2 backbone on a 3x48x48 image: the stem and the
                    four stage outputs (every block kind: plain 3x3 layers,
                    light 1x1 + depthwise 5x5 layers, the stride-2 depthwise
                    downsamples and the residual blocks of stage 3)
  net_encoder.npz   encoder input projections + hybrid encoder at 1/8 of the
                    800x800 geometry (p32 3x3, p16 6x6, p8 12x12, x4 24x24):
                    the AIFI layer, FPN / PAN CSP-RepVGG blocks and the mask
                    feature head
  net_decode.npz    everything after the encoder at the full 800x800
                    geometry from seeded encoder outputs: decoder input
                    projections, query selection (top-300), mask-derived
                    initial boxes, the six decoder layers with box
                    refinement and the heads

Deviations the reference makes from transformers, followed here so that the
fixtures state the reference's network:
  * the order head reads the last decoder hidden state before dec_norm
    (src/ppdoclayout.cpp:861-866); transformers feeds it the normed one and
    masks the lower triangle with -1e4.  The fixture stores the global
    pointer projection gp = dense(order_head[5](h)) of the pre-norm h.
The transformers names differ from the published checkpoint's in a few
places the converter's table spells the checkpoint way: self_attn.out_proj
is o_proj, fc1/fc2 sit under .mlp, and the AIFI layer is encoder.aifi.0
rather than encoder.encoder.0.
"""
import os
import re
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(ROOT, "ppdoclayout-ggml_amd"))
import synth_gguf as S  # noqa: E402
from net_inputs import WEIGHT_SEED, backbone_input, decode_inputs, encoder_inputs  # noqa: E402

BN_EPS = 1e-5
BB = "model.backbone.model."

# (GGUF prefix pattern, transformers prefix, kind).  kind: how the unit is
# stored on the transformers side -- "cl" conv .convolution + .normalization
# (HGNetV2ConvLayer / PPDocLayoutV3ConvLayer), "cn" conv .conv + .norm
# (ConvNormLayer), "seq" nn.Sequential(conv, bn) as .0 / .1, "p" plain module
# with its own weight and bias (Linear, LayerNorm, biased Conv2d).
MAP = [
    (r"(stem[1234ab]+)", BB + r"embedder.\1", "cl"),
    (r"st(\d)\.ds", BB + r"encoder.stages.\1.downsample", "cl"),
    (r"st(\d)\.b(\d)\.l(\d)\.c([12])", BB + r"encoder.stages.\1.blocks.\2.layers.\3.conv\4", "cl"),
    (r"st(\d)\.b(\d)\.l(\d)", BB + r"encoder.stages.\1.blocks.\2.layers.\3", "cl"),
    (r"st(\d)\.b(\d)\.agg(\d)", BB + r"encoder.stages.\1.blocks.\2.aggregation.\3", "cl"),
    (r"enc_in(\d)", r"model.encoder_input_proj.\1", "seq"),
    (r"dec_in(\d)", r"model.decoder_input_proj.\1", "seq"),
    (r"aifi\.([qkvo])", r"model.encoder.aifi.0.layers.0.self_attn.\1_proj", "p"),
    (r"aifi\.ln1", r"model.encoder.aifi.0.layers.0.self_attn_layer_norm", "p"),
    (r"aifi\.ln2", r"model.encoder.aifi.0.layers.0.final_layer_norm", "p"),
    (r"aifi\.fc([12])", r"model.encoder.aifi.0.layers.0.mlp.fc\1", "p"),
    (r"lat(\d)", r"model.encoder.lateral_convs.\1", "cn"),
    (r"fpn(\d)\.bn(\d)\.c([12])", r"model.encoder.fpn_blocks.\1.bottlenecks.\2.conv\3", "cn"),
    (r"fpn(\d)\.c([12])", r"model.encoder.fpn_blocks.\1.conv\2", "cn"),
    (r"pand(\d)", r"model.encoder.downsample_convs.\1", "cn"),
    (r"pan(\d)\.bn(\d)\.c([12])", r"model.encoder.pan_blocks.\1.bottlenecks.\2.conv\3", "cn"),
    (r"pan(\d)\.c([12])", r"model.encoder.pan_blocks.\1.conv\2", "cn"),
    (r"mh(\d)\.(\d)", r"model.encoder.mask_feature_head.scale_heads.\1.layers.\2", "cl"),
    (r"mh\.out", r"model.encoder.mask_feature_head.output_conv", "cl"),
    (r"mlat", r"model.encoder.encoder_mask_lateral", "cl"),
    (r"mout\.base", r"model.encoder.encoder_mask_output.base_conv", "cl"),
    (r"mout\.conv", r"model.encoder.encoder_mask_output.conv", "p"),
    (r"enc_out\.l", r"model.enc_output.0", "p"),
    (r"enc_out\.ln", r"model.enc_output.1", "p"),
    (r"score_head", r"model.enc_score_head", "p"),
    (r"bbox_head\.(\d)", r"model.enc_bbox_head.layers.\1", "p"),
    (r"dec(\d)\.sa\.([qkvo])", r"model.decoder.layers.\1.self_attn.\2_proj", "p"),
    (r"dec(\d)\.ln1", r"model.decoder.layers.\1.self_attn_layer_norm", "p"),
    (r"dec(\d)\.ca\.so", r"model.decoder.layers.\1.encoder_attn.sampling_offsets", "p"),
    (r"dec(\d)\.ca\.aw", r"model.decoder.layers.\1.encoder_attn.attention_weights", "p"),
    (r"dec(\d)\.ca\.vp", r"model.decoder.layers.\1.encoder_attn.value_proj", "p"),
    (r"dec(\d)\.ca\.op", r"model.decoder.layers.\1.encoder_attn.output_proj", "p"),
    (r"dec(\d)\.ln2", r"model.decoder.layers.\1.encoder_attn_layer_norm", "p"),
    (r"dec(\d)\.ln3", r"model.decoder.layers.\1.final_layer_norm", "p"),
    (r"dec(\d)\.fc([12])", r"model.decoder.layers.\1.mlp.fc\2", "p"),
    (r"qpos\.(\d)", r"model.decoder.query_pos_head.layers.\1", "p"),
    (r"dec_norm", r"model.decoder_norm", "p"),
    (r"order(\d)", r"model.decoder_order_head.\1", "p"),
    (r"gp", r"model.decoder_global_pointer.dense", "p"),
    (r"mq\.(\d)", r"model.mask_query_head.layers.\1", "p"),
]
SUFFIX = {"cl": (".convolution", ".normalization"), "cn": (".conv", ".norm"), "seq": (".0", ".1")}


def hf_unit(gguf_prefix):
    for pat, rep, kind in MAP:
        if re.fullmatch(pat, gguf_prefix):
            return re.sub("^" + pat + "$", rep, gguf_prefix), kind
    raise KeyError(gguf_prefix)


def build_model(weights, seed=WEIGHT_SEED):
    from transformers import PPDocLayoutV3Config, PPDocLayoutV3ForObjectDetection

    torch.manual_seed(0)
    model = PPDocLayoutV3ForObjectDetection(PPDocLayoutV3Config(num_labels=25)).double().eval()
    rng = np.random.default_rng(seed + 1000)
    units = sorted({n.rsplit(".", 1)[0] for n in weights})
    set_params = set()
    with torch.no_grad():
        for u in units:
            w = weights[u + ".weight"].astype(np.float64)
            b = weights[u + ".bias"].astype(np.float64)
            hp, kind = hf_unit(u)
            if kind == "p":
                mod = model.get_submodule(hp)
                assert tuple(mod.weight.shape) == w.shape, (u, hp)
                mod.weight.copy_(torch.from_numpy(w))
                mod.bias.copy_(torch.from_numpy(b))
                set_params.update({hp + ".weight", hp + ".bias"})
                continue
            cs, ns = SUFFIX[kind]
            conv, bn = model.get_submodule(hp + cs), model.get_submodule(hp + ns)
            assert tuple(conv.weight.shape) == w.shape and conv.bias is None, (u, hp)
            oc = w.shape[0]
            gamma = rng.uniform(0.5, 1.5, oc)
            var = rng.uniform(0.5, 2.0, oc)
            mean = 0.1 * rng.standard_normal(oc)
            s = gamma / np.sqrt(var + BN_EPS)
            w_hf = w / s[:, None, None, None]
            beta = b + mean * s
            conv.weight.copy_(torch.from_numpy(w_hf))
            bn.weight.copy_(torch.from_numpy(gamma))
            bn.bias.copy_(torch.from_numpy(beta))
            bn.running_mean.copy_(torch.from_numpy(mean))
            bn.running_var.copy_(torch.from_numpy(var))
            # the converter's fold recovers the GGUF tensors
            s2 = gamma / np.sqrt(var + BN_EPS)
            assert np.array_equal((w_hf * s2[:, None, None, None]).astype(np.float32), weights[u + ".weight"]), u
            assert np.allclose((beta - mean * s2).astype(np.float32), weights[u + ".bias"], rtol=1e-6, atol=1e-7), u
            set_params.update({hp + cs + ".weight"} | {hp + ns + "." + k for k in
                                                      ("weight", "bias", "running_mean", "running_var")})
    # the decoder's class and box heads are tied to the encoder-side ones
    m = model.model
    assert m.decoder.class_embed.weight is m.enc_score_head.weight
    assert m.decoder.bbox_embed.layers[0].weight is m.enc_bbox_head.layers[0].weight
    return model, set_params


def f32(t):
    return t.detach().cpu().numpy().astype(np.float32)


def t64(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float64))[None]


def backbone_case(model):
    img = backbone_input()
    bb = model.model.backbone.model
    got = {}
    h = bb.embedder.register_forward_hook(lambda mod, i, o: got.__setitem__("stem", o))
    with torch.no_grad():
        maps = bb(t64(img)).feature_maps
    h.remove()
    out = {"stem": f32(got["stem"][0])}
    for i, fm in enumerate(maps):
        out["st%d" % i] = f32(fm[0])
    return out


def encoder_case(model):
    x4, p8r, p16r, p32r = encoder_inputs()
    m = model.model
    got = {}
    h = m.encoder.aifi[0].register_forward_hook(lambda mod, i, o: got.__setitem__("aifi", o))
    with torch.no_grad():
        proj = [m.encoder_input_proj[l](t64(x)) for l, x in enumerate((p8r, p16r, p32r))]
        enc = m.encoder(proj, (t64(x4), None))
    h.remove()
    f8, n16, n32 = enc.last_hidden_state
    return {"aifi": f32(got["aifi"][0]), "f8": f32(f8[0]), "n16": f32(n16[0]), "n32": f32(n32[0]),
            "mask_feat": f32(enc.mask_feat[0])}


class _NoBackbone(torch.nn.Module):
    """Stands in for the backbone when the encoder outputs are given: the
    model still projects the backbone maps, whose results it then ignores."""

    def forward(self, pixel_values, pixel_mask):
        z = lambda c: torch.zeros(1, c, 1, 1, dtype=torch.float64)
        m = torch.ones(1, 1, 1, dtype=torch.bool)
        return [(z(c), m) for c in (128, 512, 1024, 2048)]


def decode_case(model):
    import transformers.models.pp_doclayout_v3.modeling_pp_doclayout_v3 as hfm

    f8, n16, n32, mf = decode_inputs()
    m = model.model
    saved, m2b = m.backbone, hfm.mask_to_box_coordinate
    m.backbone = _NoBackbone()
    # mask -> box at float32: at float64 the function's empty-mask sentinel
    # (finfo(float64).max in a float32 tensor) is inf, and inf * 0 makes the
    # empty masks' boxes NaN; the float32 path gives (0, 0, 0, 0) for them
    hfm.mask_to_box_coordinate = lambda mask, dtype: m2b(mask, torch.float32).to(dtype)
    try:
        with torch.no_grad():
            out = model(torch.zeros(1, 3, 800, 800, dtype=torch.float64),
                        encoder_outputs=([t64(f8), t64(n16), t64(n32)], t64(mf)), output_hidden_states=False)
            h = out.last_hidden_state
            mq = m.mask_query_head(m.decoder_norm(h))
            gp = m.decoder_global_pointer.dense(m.decoder_order_head[5](h))
            topk = torch.topk(out.enc_outputs_class.max(-1).values, 300, dim=1).indices
            masks = torch.bmm(mq, t64(mf).flatten(2)).reshape(1, 300, 200, 200)
            assert torch.allclose(masks, out.out_masks, rtol=1e-12, atol=1e-12)
    finally:
        m.backbone, hfm.mask_to_box_coordinate = saved, m2b
    return {"topk": topk[0].numpy().astype(np.int32),
            "init_ref_unact": f32(out.init_reference_points[0]),
            "hidden_first32": f32(out.intermediate_hidden_states[0, :, :32]),
            "logits": f32(out.logits[0]), "boxes": f32(out.pred_boxes[0]),
            "mq": f32(mq[0]), "gp": f32(gp[0])}


def main():
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    weights = S.random_weights(WEIGHT_SEED)
    model, set_params = build_model(weights)
    for name, fn in (("backbone", backbone_case), ("encoder", encoder_case), ("decode", decode_case)):
        out = fn(model)
        np.savez(os.path.join(HERE, "net_%s.npz" % name), **out)
        print(name, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
