"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on the
CPU (the oracle, the host logic and the C ABI's symbol table)."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def tiny_config(**over):
    """A small model the GPU kernels accept (head_dim 128, 2 q heads per kv
    head) and the oracle runs in milliseconds."""
    cfg = dict(vocab_size=97, hidden_size=256, intermediate_size=384,
               layers=2, heads=4, kv_heads=2, head_dim=128, max_positions=4096,
               rms_norm_eps=1e-6, rope_theta=1e6, audio_codebooks=8,
               audio_vocab_size=1025, audio_mask_id=1024)
    cfg.update(over)
    return cfg


def random_input(rng, cfg, text, reference, target, codes_fill=0.0):
    """A ConditionalInput-shaped id array: text ids, reference codes, then
    target frames (masked, or a `codes_fill` fraction already unmasked)."""
    C = cfg["audio_codebooks"]
    V = cfg["audio_vocab_size"]
    mask = cfg["audio_mask_id"]
    length = text + reference + target
    ids = np.full((C, length), mask, dtype=np.int32)
    tokens = rng.integers(0, cfg["vocab_size"], size=text)
    ids[:, :text] = tokens[None, :]
    if reference:
        ids[:, text:text + reference] = rng.integers(0, V - 1, size=(C, reference))
    if codes_fill > 0:
        fill = rng.random((C, target)) < codes_fill
        vals = rng.integers(0, V - 1, size=(C, target))
        block = ids[:, text + reference:]
        block[fill] = vals[fill]
    return ids


@pytest.fixture(scope="session")
def golden_cases():
    import json
    with open(os.path.join(GOLDEN, "generator_cases.json")) as f:
        return json.load(f)
