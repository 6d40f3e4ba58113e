#!/usr/bin/env python3
"""Writes tests/golden/forward_tiny.json: target logits of a tiny OmniVoice
backbone computed with the installed third-party `transformers` Qwen3
decoder layers (not the reference) in float64 on the CPU.

The CFG batch is built the way the reference's Python fixture tool builds it
(gufo-extensions/omnivoice tools/reference/generator_golden.py:40-54): two
rows of the conditional length; row 0 the conditional sequence with full
attention, row 1 its last `target` frames with attention among them only
(padding positions attend to themselves); default positions 0 .. L-1.
Embeddings follow the reference's Embed kernel (text rows: the first
codebook's token row; audio rows: the sum over codebooks of
audio_embeddings[c * V + id]); logits are audio_heads @ final_norm(h) for
the conditional target rows, then the unconditional ones.

Weights come from the seeded synthetic model (the oracle's restatement of
the spec), so the test side rebuilds them from (seed, norm_jitter); only
inputs and logits are stored.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

CONFIG = dict(vocab_size=97, hidden_size=256, intermediate_size=384, layers=2,
              heads=4, kv_heads=2, head_dim=128, max_positions=4096,
              rms_norm_eps=1e-6, rope_theta=1e6, audio_codebooks=8,
              audio_vocab_size=33, audio_mask_id=32)
CASES = [  # (seed, norm_jitter, text, reference, target, unmasked fraction)
    (7, 0.1, 5, 3, 6, 0.0),
    (11, 0.2, 4, 0, 9, 0.4),
]


def synth(seed, tensor, shape, norm=False, jitter=0.0):
    n = int(np.prod(shape))
    out = np.zeros(n, dtype=np.float32)
    oracle.lib().orc_synth_values(seed, tensor, 0, n, int(norm), jitter,
                                  out.ctypes.data)
    return out.reshape(shape).astype(np.float64)


def layer_tensor(layer, kind):
    return 100 + 16 * layer + kind


def run_case(seed, jitter, text, reference, target, fill):
    from transformers import Qwen3Config
    from transformers.models.qwen3 import modeling_qwen3 as q3
    c = CONFIG
    H, I, d = c["hidden_size"], c["intermediate_size"], c["head_dim"]
    C, V, mask = c["audio_codebooks"], c["audio_vocab_size"], c["audio_mask_id"]
    rng = np.random.default_rng(seed)
    length = text + reference + target
    ids = np.full((C, length), mask, dtype=np.int64)
    ids[:, :text] = rng.integers(0, c["vocab_size"], size=text)[None, :]
    if reference:
        ids[:, text:text + reference] = rng.integers(0, V - 1, size=(C, reference))
    if fill:
        chosen = rng.random((C, target)) < fill
        vals = rng.integers(0, V - 1, size=(C, target))
        block = ids[:, text + reference:]
        block[chosen] = vals[chosen]

    cfg = Qwen3Config(vocab_size=c["vocab_size"], hidden_size=H,
                      intermediate_size=I, num_hidden_layers=c["layers"],
                      num_attention_heads=c["heads"],
                      num_key_value_heads=c["kv_heads"], head_dim=d,
                      rms_norm_eps=c["rms_norm_eps"],
                      rope_parameters={"rope_theta": c["rope_theta"],
                                       "rope_type": "default"},
                      max_position_embeddings=c["max_positions"],
                      attention_bias=False)
    cfg._attn_implementation = "eager"
    text_emb = synth(seed, 1, (c["vocab_size"], H))
    audio_emb = synth(seed, 2, (C * V, H))
    heads = synth(seed, 3, (C * V, H))
    final_norm = synth(seed, 4, (H,), True, jitter)

    def embed(row_ids, text_rows):
        out = np.zeros((row_ids.shape[1], H))
        for p in range(row_ids.shape[1]):
            if p < text_rows:
                out[p] = text_emb[row_ids[0, p]]
            else:
                out[p] = sum(audio_emb[cb * V + row_ids[cb, p]] for cb in range(C))
        return out

    # generator_golden.py batch_inputs: row 0 conditional, row 1 the target
    # frames moved to the front, the rest mask ids.
    uncond = np.full((C, length), mask, dtype=np.int64)
    uncond[:, :target] = ids[:, -target:]
    x = torch.tensor(np.stack([embed(ids, text), embed(uncond, 0)]))
    allowed = torch.zeros((2, 1, length, length), dtype=torch.bool)
    allowed[0] = True
    allowed[1, :, :target, :target] = True
    pad = torch.arange(target, length)
    allowed[1, :, pad, pad] = True
    additive = torch.zeros(allowed.shape, dtype=torch.float64)
    additive[~allowed] = -1e300
    positions = torch.arange(length)[None, :].expand(2, -1)
    rotary = q3.Qwen3RotaryEmbedding(cfg)
    pe = rotary(x, positions)
    for l in range(c["layers"]):
        layer = q3.Qwen3DecoderLayer(cfg, l).double().eval()
        sd = {
            "self_attn.q_proj.weight": synth(seed, layer_tensor(l, 0), (c["heads"] * d, H)),
            "self_attn.k_proj.weight": synth(seed, layer_tensor(l, 1), (c["kv_heads"] * d, H)),
            "self_attn.v_proj.weight": synth(seed, layer_tensor(l, 2), (c["kv_heads"] * d, H)),
            "self_attn.o_proj.weight": synth(seed, layer_tensor(l, 3), (H, c["heads"] * d)),
            "mlp.gate_proj.weight": synth(seed, layer_tensor(l, 4), (I, H)),
            "mlp.up_proj.weight": synth(seed, layer_tensor(l, 5), (I, H)),
            "mlp.down_proj.weight": synth(seed, layer_tensor(l, 6), (H, I)),
            "input_layernorm.weight": synth(seed, layer_tensor(l, 7), (H,), True, jitter),
            "post_attention_layernorm.weight": synth(seed, layer_tensor(l, 8), (H,), True, jitter),
            "self_attn.q_norm.weight": synth(seed, layer_tensor(l, 9), (d,), True, jitter),
            "self_attn.k_norm.weight": synth(seed, layer_tensor(l, 10), (d,), True, jitter),
        }
        layer.load_state_dict({k: torch.tensor(v) for k, v in sd.items()})
        with torch.no_grad():
            x = layer(x, attention_mask=additive, position_embeddings=pe)
            if isinstance(x, tuple):
                x = x[0]
    h = x.numpy()
    rows = np.concatenate([h[0, length - target:], h[1, :target]])
    ms = np.mean(rows * rows, axis=1, keepdims=True)
    normed = final_norm * (rows / np.sqrt(ms + c["rms_norm_eps"]))
    logits = normed @ heads.T
    return {"seed": seed, "norm_jitter": jitter, "audio_start": text,
            "target": target, "ids": ids.tolist(),
            "logits": np.round(logits, 9).tolist()}


def main():
    out = {"source": "transformers Qwen3DecoderLayer (float64, eager) over "
                     "the reference's CFG batch layout",
           "config": CONFIG,
           "cases": [run_case(*case) for case in CASES]}
    path = os.path.join(HERE, "forward_tiny.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", path, file=sys.stderr)


if __name__ == "__main__":
    main()
