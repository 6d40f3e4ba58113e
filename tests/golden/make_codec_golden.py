"""Writes tests/golden/codec_tiny.json: the audio decoder at a small
configuration, run by the installed third-party transformers (5.15):
transformers.models.dac's DacDecoder with the two changes that
HiggsAudioV2TokenizerModel._adjust_dac_decoder makes (output_padding =
stride % 2 on every transposed convolution, no final tanh), after the RVQ
decode (codebook embedding through project_out, summed over codebooks) and
fc2, in float64 on the CPU. The weights are the synthetic decoder's
specification (tensor ids and scales as in oracle/codec.cpp), so the oracle
and the GPU decoder can be compared with it.

Run from the repository root: python3 tests/golden/make_codec_golden.py
"""
import json
import math
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402  (the synthetic values only)
from transformers import DacConfig  # noqa: E402
from transformers.models.dac.modeling_dac import DacDecoder  # noqa: E402

CFG = dict(codebooks=3, codebook_size=16, codebook_dim=8, hidden=24, latent=12,
           channels=32, ratios=[2, 3, 4])
SEED = 77
FRAMES = 6


def value(tid, shape, scale, exp=False):
    n = int(np.prod(shape))
    return torch.from_numpy(oracle.codec_values(SEED, tid, n, scale, exp).astype(np.float64)
                            ).view(*shape)


def main():
    C, E, D, H, Lat = (CFG[k] for k in ("codebooks", "codebook_size", "codebook_dim",
                                        "hidden", "latent"))
    ch = CFG["channels"]
    dac = DacConfig(encoder_hidden_size=4, downsampling_ratios=CFG["ratios"],
                    decoder_hidden_size=ch, upsampling_ratios=CFG["ratios"], hidden_size=Lat,
                    n_codebooks=C, codebook_size=E, codebook_dim=D)
    decoder = DacDecoder(dac).double().eval()
    for module in decoder.modules():
        if isinstance(module, torch.nn.ConvTranspose1d):
            module.output_padding = (module.stride[0] % 2,)
    if hasattr(decoder, "tanh"):
        decoder.tanh = torch.nn.Identity()
    state = {"conv1.weight": value(1102, (ch, Lat, 7), (7 * Lat) ** -0.5),
             "conv1.bias": value(1103, (ch,), 0.01)}
    for i, s in enumerate(CFG["ratios"]):
        p, base, out = f"block.{i}", 1200 + 32 * i, ch // 2
        state[p + ".snake1.alpha"] = value(base, (1, ch, 1), 0.1, True)
        state[p + ".conv_t1.weight"] = value(base + 1, (ch, out, 2 * s), (2 * ch) ** -0.5)
        state[p + ".conv_t1.bias"] = value(base + 2, (out,), 0.01)
        for u in range(3):
            q, uid = f"{p}.res_unit{u + 1}", base + 4 + 6 * u
            state[q + ".snake1.alpha"] = value(uid, (1, out, 1), 0.1, True)
            state[q + ".conv1.weight"] = value(uid + 1, (out, out, 7), (7 * out) ** -0.5)
            state[q + ".conv1.bias"] = value(uid + 2, (out,), 0.01)
            state[q + ".snake2.alpha"] = value(uid + 3, (1, out, 1), 0.1, True)
            state[q + ".conv2.weight"] = value(uid + 4, (out, out, 1), 0.3 * out ** -0.5)
            state[q + ".conv2.bias"] = value(uid + 5, (out,), 0.01)
        ch = out
    state["snake1.alpha"] = value(1400, (1, ch, 1), 0.1, True)
    state["conv2.weight"] = value(1401, (1, ch, 7), 0.1 * (7 * ch) ** -0.5)
    state["conv2.bias"] = value(1402, (1,), 0.01)
    missing, unexpected = decoder.load_state_dict(state, strict=True), None
    del missing, unexpected

    codes = np.random.default_rng(11).integers(0, E, size=(C, FRAMES))
    quantized = 0
    for c in range(C):
        embed = value(1000 + 4 * c, (E, D), 0.35)
        entries = F.embedding(torch.from_numpy(codes[c]).long(), embed)
        quantized = quantized + F.linear(entries, value(1001 + 4 * c, (H, D), D ** -0.5),
                                         value(1002 + 4 * c, (H,), 0.01))
    latent = F.linear(quantized, value(1100, (Lat, H), H ** -0.5), value(1101, (Lat,), 0.01))
    with torch.no_grad():
        audio = decoder(latent.T[None])[0, 0].numpy()
    assert audio.shape == (FRAMES * math.prod(CFG["ratios"]),)
    out = {"source": "transformers 5.15 DacDecoder (HiggsAudioV2 output padding, no tanh), "
                     "float64, synthetic decoder weights",
           "config": CFG, "seed": SEED, "codes": codes.tolist(),
           "audio": [float(f"{v:.12g}") for v in audio]}
    path = os.path.join(ROOT, "tests", "golden", "codec_tiny.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print(path, audio.shape, float(np.abs(audio).max()))


if __name__ == "__main__":
    main()
