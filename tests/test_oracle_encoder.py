"""The oracle's audio encoder pinned before anything is compared with it:
the resampler against the reference's own resampler vectors
(tests/fixtures/audio_golden.json "resample", within the reference's 2e-6,
audio_test.cpp:157-166), and the whole encoder at a small configuration
against transformers' HubertModel and DacEncoder plus torch float64 layers
on the same synthetic weights (tests/golden/encoder_tiny.json)."""
import json
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN


def reference_signal(spec, rate, seed, extra=0):
    """The reference test's integer signal generator (audio_test.cpp:30-58):
    a 31-bit LCG drives uniform noise or a period-55 triangle with small
    noise, clamped to int16 and scaled by 1/32768."""
    state = seed
    out = []
    for ms, kind, amplitude in spec:
        noise_amp = min(amplitude, 64)
        for n in range(ms * rate // 1000):
            state = (state * 1103515245 + 12345) & 0x7FFFFFFF
            if kind == "tone":
                phase = n % 55
                # C++ integer division truncates toward zero and % keeps the
                # dividend's sign; both operands here are non-negative
                noise = (state >> 8) % (2 * noise_amp + 1) - noise_amp
                num = 4 * amplitude * abs(2 * phase - 55)
                value = num // 110 - amplitude + noise
            else:
                value = (state >> 8) % (2 * amplitude + 1) - amplitude
            out.append(min(max(value, -32768), 32767) / 32768.0)
    out.extend([0.25] * extra)
    return np.array(out, dtype=np.float32)


def load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def test_resampler_matches_reference_vectors():
    golden = load("resample_cases.json")
    stride = golden["stride"]
    assert len(golden["cases"]) == 6
    for case in golden["cases"]:
        sig = case["signal"]
        x = reference_signal(sig["spec"], sig["rate"], sig["seed"], sig.get("extra", 0))
        y = oracle.resample(x, sig["rate"], case["target"])
        assert len(y) == case["length"], (sig["rate"], case["target"])
        want = np.array(case["samples"])
        got = y[::stride][:len(want)].astype(np.float64)
        assert len(got) == len(want)
        assert np.abs(got - want).max() <= 2e-6, (sig["rate"], np.abs(got - want).max())


def test_resampler_identity_and_band_limited_tone():
    x = np.random.default_rng(1).standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(oracle.resample(x, 24000, 24000), x)
    # a 300 Hz tone well inside both bands comes out as the same tone at the
    # new rate, away from the edges where the kernel runs off the signal
    t = np.arange(24000)
    y = oracle.resample(np.sin(2 * np.pi * 300 * t / 24000).astype(np.float32), 24000, 16000)
    assert len(y) == 16000
    u = np.arange(16000)
    want = np.sin(2 * np.pi * 300 * u / 16000)
    assert np.abs(y[200:-200] - want[200:-200]).max() < 5e-3


def test_encoder_matches_library_fixture():
    g = load("encoder_tiny.json")
    got = oracle.Encoder(g["config"], g["seed"]).encode(np.array(g["signal"], np.float32))
    for key, tol in (("semantic", 1e-5), ("acoustic", 1e-5), ("embeddings", 1e-5)):
        want = np.array(g[key])
        assert got[key].shape == want.shape, key
        err = np.abs(got[key] - want).max()
        assert err <= tol * max(1.0, np.abs(want).max()), (key, err)
    np.testing.assert_array_equal(got["codes"], np.array(g["codes"]))


def test_encoder_frames_and_determinism():
    cfg = oracle.encoder_tiny_config()
    enc = oracle.Encoder(cfg, 5)
    x = np.random.default_rng(2).standard_normal(24 * 13).astype(np.float32) * 0.1
    a = enc.encode(x)
    assert a["codes"].shape == (3, 13)
    assert a["codes"].min() >= 0 and a["codes"].max() < 16
    b = enc.encode(x)
    for k in a:
        np.testing.assert_array_equal(a[k], b[k])


def test_encoder_quantizer_picks_nearest_entries():
    """Each stage's code is the codebook entry nearest to the projected
    residual (brute force on the oracle's own embeddings: the residual after
    stage q is the embedding minus the decoded entries of stages before)."""
    g = load("encoder_tiny.json")
    c = g["config"]
    got = oracle.Encoder(c, g["seed"]).encode(np.array(g["signal"], np.float32))
    H, D, E = c["width"] + c["latent"], c["codebook_dim"], c["codebook_size"]
    v = lambda tid, n, scale: oracle.codec_values(g["seed"], tid, n, scale, False).astype(np.float64)
    residual = got["embeddings"].astype(np.float64)
    for q in range(c["codebooks"]):
        w_in = v(2900 + 2 * q, D * H, H ** -0.5).reshape(D, H)
        b_in = v(2901 + 2 * q, D, 0.01)
        embed = v(1000 + 4 * q, E * D, 0.35).reshape(E, D)
        proj = residual @ w_in.T + b_in
        dist = ((proj[:, None, :] - embed[None]) ** 2).sum(-1)
        np.testing.assert_array_equal(got["codes"][q], dist.argmin(1))
        w_out = v(1001 + 4 * q, H * D, D ** -0.5).reshape(H, D)
        residual = residual - (embed[got["codes"][q]] @ w_out.T + v(1002 + 4 * q, H, 0.01))


def test_encoder_rejects_partial_frames():
    """Reference audio must be a whole number of frames (codec_encoder.cpp:260)."""
    enc = oracle.Encoder(oracle.encoder_tiny_config(), 5)
    for n in (0, 10, 24 * 3 + 1):
        with pytest.raises(ValueError):
            enc.encode(np.zeros(n, np.float32))
