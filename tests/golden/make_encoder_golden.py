"""Writes tests/golden/encoder_tiny.json: the audio encoder at a small
configuration (oracle.encoder_tiny_config), with the synthetic encoder's
weights, run through the installed third-party transformers (5.15) where it
has the layers: HubertModel (the semantic features: the mean of the encoder
input and every layer output, every semantic_stride-th frame) and
transformers.models.dac's DacEncoder (the acoustic latents). The semantic
encoder, fc and the residual vector quantizer follow as torch float64
layers (HiggsAudioV2Tokenizer's SemanticEncoder and quantizer, whose module
needs torchaudio, absent here). The HuBERT input is the oracle's resampler
output (pinned separately against the reference's resampler vectors) with
160 zeros each side.

Run from the repository root: python3 tests/golden/make_encoder_golden.py
"""
import json
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402
from transformers import DacConfig, HubertConfig, HubertModel  # noqa: E402
from transformers.models.dac.modeling_dac import DacEncoder  # noqa: E402

SEED = 31
FRAMES = 20


def val(tid, shape, scale, offset=0.0):
    n = int(np.prod(shape))
    v = np.array([oracle.lib().orc_synth_normal(SEED, tid, e) for e in range(n)])
    return torch.from_numpy(offset + scale * v).view(*shape)


def alpha(tid, shape):
    n = int(np.prod(shape))
    v = np.array([oracle.lib().orc_synth_normal(SEED, tid, e) for e in range(n)])
    return torch.from_numpy(np.exp(0.1 * v)).view(*shape)


def signal(length):
    t = np.arange(length)
    rng = np.random.default_rng(5)
    return (0.2 * np.sin(2 * np.pi * 180 * t / 24000) * (0.5 + 0.5 * np.sin(t / 700))
            + 0.02 * rng.standard_normal(length)).astype(np.float32)


def main():
    c = oracle.encoder_tiny_config()
    W, I, L = c["width"], c["intermediate"], c["layers"]
    x = signal(FRAMES * c["frame_samples"])
    # ---- HuBERT (transformers)
    hc = HubertConfig(hidden_size=W, num_hidden_layers=L, num_attention_heads=c["heads"],
                      intermediate_size=I, conv_dim=c["conv_dim"], conv_kernel=c["conv_kernel"],
                      conv_stride=c["conv_stride"], conv_bias=False, feat_extract_norm="group",
                      feat_extract_activation="gelu", hidden_act="gelu",
                      do_stable_layer_norm=False, feat_proj_layer_norm=True,
                      num_conv_pos_embeddings=c["pos_kernel"],
                      num_conv_pos_embedding_groups=c["pos_groups"], layer_norm_eps=c["eps"])
    hubert = HubertModel(hc).double().eval()
    st = {}
    cin = 1
    for i, (cd, k) in enumerate(zip(c["conv_dim"], c["conv_kernel"])):
        st[f"feature_extractor.conv_layers.{i}.conv.weight"] = val(2000 + i, (cd, cin, k),
                                                                    (cin * k) ** -0.5)
        cin = cd
    st["feature_extractor.conv_layers.0.layer_norm.weight"] = val(2010, (c["conv_dim"][0],), 0.1, 1)
    st["feature_extractor.conv_layers.0.layer_norm.bias"] = val(2011, (c["conv_dim"][0],), 0.1)
    st["feature_projection.layer_norm.weight"] = val(2012, (cin,), 0.1, 1)
    st["feature_projection.layer_norm.bias"] = val(2013, (cin,), 0.1)
    st["feature_projection.projection.weight"] = val(2014, (W, cin), cin ** -0.5)
    st["feature_projection.projection.bias"] = val(2015, (W,), 0.01)
    K, G = c["pos_kernel"], c["pos_groups"]
    p = "encoder.pos_conv_embed.conv."
    st[p + "parametrizations.weight.original0"] = val(2016, (1, 1, K), 0.1, 1)
    st[p + "parametrizations.weight.original1"] = val(2017, (W, W // G, K), 1.0)
    st[p + "bias"] = val(2018, (W,), 0.01)
    st["encoder.layer_norm.weight"] = val(2019, (W,), 0.1, 1)
    st["encoder.layer_norm.bias"] = val(2020, (W,), 0.1)
    for l in range(L):
        b, q = 2100 + 16 * l, f"encoder.layers.{l}."
        for j, name in enumerate(("q_proj", "k_proj", "v_proj")):
            st[q + f"attention.{name}.weight"] = val(b + 2 * j, (W, W), W ** -0.5)
            st[q + f"attention.{name}.bias"] = val(b + 2 * j + 1, (W,), 0.01)
        st[q + "attention.out_proj.weight"] = val(b + 6, (W, W), W ** -0.5)
        st[q + "attention.out_proj.bias"] = val(b + 7, (W,), 0.01)
        st[q + "layer_norm.weight"] = val(b + 8, (W,), 0.1, 1)
        st[q + "layer_norm.bias"] = val(b + 9, (W,), 0.1)
        st[q + "feed_forward.intermediate_dense.weight"] = val(b + 10, (I, W), W ** -0.5)
        st[q + "feed_forward.intermediate_dense.bias"] = val(b + 11, (I,), 0.01)
        st[q + "feed_forward.output_dense.weight"] = val(b + 12, (W, I), 0.5 * I ** -0.5)
        st[q + "feed_forward.output_dense.bias"] = val(b + 13, (W,), 0.01)
        st[q + "final_layer_norm.weight"] = val(b + 14, (W,), 0.1, 1)
        st[q + "final_layer_norm.bias"] = val(b + 15, (W,), 0.1)
    st["masked_spec_embed"] = hubert.state_dict()["masked_spec_embed"]
    hubert.load_state_dict(st, strict=True)
    resampled = oracle.resample(x, c["sample_rate"], c["semantic_rate"]).astype(np.float64)
    padded = np.concatenate([np.zeros(160), resampled, np.zeros(160)])
    with torch.no_grad():
        states = hubert(torch.from_numpy(padded)[None], output_hidden_states=True).hidden_states
    features = torch.stack(states, dim=1).mean(dim=1)[0][::c["semantic_stride"]][:FRAMES]
    # ---- DAC encoder (transformers)
    dc = DacConfig(encoder_hidden_size=c["enc_channels"], downsampling_ratios=c["ratios"],
                   decoder_hidden_size=32, upsampling_ratios=c["ratios"], hidden_size=c["latent"],
                   n_codebooks=c["codebooks"], codebook_size=c["codebook_size"],
                   codebook_dim=c["codebook_dim"])
    dac = DacEncoder(dc).double().eval()
    sd = {"conv1.weight": val(2500, (c["enc_channels"], 1, 7), 7 ** -0.5),
          "conv1.bias": val(2501, (c["enc_channels"],), 0.01)}
    ch = c["enc_channels"]
    for i, s in enumerate(c["ratios"]):
        b, q = 2600 + 32 * i, f"block.{i}."
        for u in range(3):
            uid, r = b + 4 + 6 * u, q + f"res_unit{u + 1}."
            sd[r + "snake1.alpha"] = alpha(uid, (1, ch, 1))
            sd[r + "conv1.weight"] = val(uid + 1, (ch, ch, 7), (7 * ch) ** -0.5)
            sd[r + "conv1.bias"] = val(uid + 2, (ch,), 0.01)
            sd[r + "snake2.alpha"] = alpha(uid + 3, (1, ch, 1))
            sd[r + "conv2.weight"] = val(uid + 4, (ch, ch, 1), 0.3 * ch ** -0.5)
            sd[r + "conv2.bias"] = val(uid + 5, (ch,), 0.01)
        sd[q + "snake1.alpha"] = alpha(b, (1, ch, 1))
        sd[q + "conv1.weight"] = val(b + 1, (2 * ch, ch, 2 * s), (2 * ch * s) ** -0.5)
        sd[q + "conv1.bias"] = val(b + 2, (2 * ch,), 0.01)
        ch *= 2
    sd["snake1.alpha"] = alpha(2800, (1, ch, 1))
    sd["conv2.weight"] = val(2801, (c["latent"], ch, 3), (3 * ch) ** -0.5)
    sd["conv2.bias"] = val(2802, (c["latent"],), 0.01)
    dac.load_state_dict(sd, strict=True)
    with torch.no_grad():
        acoustic = dac(torch.from_numpy(x.astype(np.float64))[None, None])[0]  # [latent][F]
    # ---- semantic encoder, fc, RVQ (torch float64 layers)
    s = features.T[None]
    s = F.conv1d(s, val(2400, (W, W, 3), (3 * W) ** -0.5), padding=1)
    for b in range(2):
        for u in range(2):
            y = F.conv1d(F.elu(s), val(2410 + 10 * b + 2 * u, (W, W, 3), (3 * W) ** -0.5), padding=1)
            y = F.conv1d(F.elu(y), val(2411 + 10 * b + 2 * u, (W, W, 1), 0.3 * W ** -0.5))
            s = s + y
        s = F.conv1d(s, val(2450 + 2 * b, (W, W, 3), (3 * W) ** -0.5), val(2451 + 2 * b, (W,), 0.01),
                     padding=1)
    H = W + c["latent"]
    joint = torch.cat([acoustic, s[0]], dim=0).T  # [F][H]
    residual = F.linear(joint, val(2810, (H, H), H ** -0.5), val(2811, (H,), 0.01))
    embeddings = residual.clone()
    D, E = c["codebook_dim"], c["codebook_size"]
    codes = []
    for q in range(c["codebooks"]):
        proj = F.linear(residual, val(2900 + 2 * q, (D, H), H ** -0.5), val(2901 + 2 * q, (D,), 0.01))
        embed = val(1000 + 4 * q, (E, D), 0.35)
        dist = -((proj.pow(2).sum(1, keepdim=True) - 2 * proj @ embed.T) + embed.pow(2).sum(1)[None])
        idx = dist.argmax(dim=1)
        codes.append(idx.tolist())
        decoded = F.linear(F.embedding(idx, embed), val(1001 + 4 * q, (H, D), D ** -0.5),
                           val(1002 + 4 * q, (H,), 0.01))
        residual = residual - decoded
    out = {"source": "transformers 5.15 HubertModel and DacEncoder, torch float64 semantic "
                     "encoder / fc / RVQ, synthetic encoder weights",
           "config": c, "seed": SEED, "frames": FRAMES, "signal": x.tolist(),
           "semantic": features.numpy().round(10).tolist(),
           "acoustic": acoustic.T.numpy().round(10).tolist(),
           "embeddings": embeddings.numpy().round(10).tolist(), "codes": codes}
    path = os.path.join(ROOT, "tests", "golden", "encoder_tiny.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print(path, np.array(codes).shape, float(features.std()), float(acoustic.std()))


if __name__ == "__main__":
    main()
