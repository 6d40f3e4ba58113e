"""Pins of the audio decoder's CPU restatement (oracle/codec.cpp): each
layer against the float64 library routine that defines it
(torch.nn.functional.conv1d / conv_transpose1d on the CPU), the Snake
activation against its closed form, the synthetic values against their
distribution, and the whole decoder against the same composition of torch
layers at a small configuration."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

TINY = dict(codebooks=3, codebook_size=16, codebook_dim=8, hidden=24, latent=12,
            channels=32, ratios=[2, 3, 4])


@pytest.mark.parametrize("cin,cout,length,kernel,dilation",
                         [(5, 7, 37, 7, 1), (6, 4, 50, 7, 3), (3, 5, 80, 7, 9),
                          (8, 8, 19, 1, 1), (4, 1, 33, 7, 1), (2, 3, 5, 7, 9)])
def test_conv1d_matches_torch(cin, cout, length, kernel, dilation):
    rng = np.random.default_rng(cin * 100 + length)
    x = rng.standard_normal((cin, length)).astype(np.float32)
    w = rng.standard_normal((cout, cin, kernel)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    got = oracle.conv1d(x, w, b, dilation)
    want = F.conv1d(torch.from_numpy(x).double()[None], torch.from_numpy(w).double(),
                    torch.from_numpy(b).double(), dilation=dilation,
                    padding=(kernel - 1) * dilation // 2)[0].numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("stride", [2, 3, 4, 5, 8])
def test_conv_transpose1d_matches_torch(stride):
    rng = np.random.default_rng(stride)
    cin, cout, length = 6, 5, 11
    x = rng.standard_normal((cin, length)).astype(np.float32)
    w = rng.standard_normal((cin, cout, 2 * stride)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    got = oracle.conv_transpose1d(x, w, b, stride)
    want = F.conv_transpose1d(torch.from_numpy(x).double()[None],
                              torch.from_numpy(w).double(), torch.from_numpy(b).double(),
                              stride=stride, padding=math.ceil(stride / 2),
                              output_padding=stride % 2)[0].numpy()
    assert got.shape == want.shape == (cout, length * stride)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_snake_closed_form():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((4, 100)) * 3).astype(np.float32)
    alpha = np.exp(rng.standard_normal(4) * 0.5).astype(np.float32)
    got = oracle.snake(x, alpha)
    a = alpha.astype(np.float64)[:, None]
    want = x + np.sin(a * x) ** 2 / (a + 1e-9)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6)
    # snake(0) = 0, so zero padding before or after the activation agree.
    assert (oracle.snake(np.zeros((4, 3), np.float32), alpha) == 0).all()


def test_codec_values_distribution():
    v = oracle.codec_values(1234, 1205, 200000, 0.25)
    assert abs(v.mean()) < 0.25 * 0.01 and abs(v.std() / 0.25 - 1) < 0.01
    a = oracle.codec_values(1234, 1200, 200000, 0.1, exponential=True)
    # log-normal: E[exp(0.1 n)] = exp(0.005)
    assert (a > 0).all() and abs(a.mean() - math.exp(0.005)) < 1e-3
    # distinct tensors and seeds give independent values
    assert abs(np.corrcoef(v, oracle.codec_values(1234, 1206, 200000, 0.25))[0, 1]) < 0.01
    assert abs(np.corrcoef(v, oracle.codec_values(99, 1205, 200000, 0.25))[0, 1]) < 0.01


def _torch_decoder(cfg, seed, codes):
    """The decoder as torch float64 layers, with the synthetic tensors of the
    specification (ids and scales)."""
    def val(tid, shape, scale, exp=False):
        n = int(np.prod(shape))
        return torch.from_numpy(
            oracle.codec_values(seed, tid, n, scale, exp).astype(np.float64)).view(*shape)

    def snake(x, a):
        return x + torch.sin(a.view(1, -1, 1) * x) ** 2 / (a.view(1, -1, 1) + 1e-9)

    C, E, D, H, Lat = (cfg[k] for k in ("codebooks", "codebook_size", "codebook_dim",
                                        "hidden", "latent"))
    q = 0
    for c in range(C):
        table = val(1000 + 4 * c, (E, D), 0.35) @ val(1001 + 4 * c, (H, D), D ** -0.5).T \
            + val(1002 + 4 * c, (H,), 0.01)
        q = q + table[torch.from_numpy(codes[c]).long()]
    x = (q @ val(1100, (Lat, H), H ** -0.5).T + val(1101, (Lat,), 0.01)).T[None]
    ch = cfg["channels"]
    x = F.conv1d(x, val(1102, (ch, Lat, 7), (7 * Lat) ** -0.5), val(1103, (ch,), 0.01),
                 padding=3)
    for i, s in enumerate(cfg["ratios"]):
        base = 1200 + 32 * i
        x = snake(x, val(base, (ch,), 0.1, True))
        x = F.conv_transpose1d(x, val(base + 1, (ch, ch // 2, 2 * s), (2 * ch) ** -0.5),
                               val(base + 2, (ch // 2,), 0.01), stride=s,
                               padding=math.ceil(s / 2), output_padding=s % 2)
        ch //= 2
        for u, d in enumerate((1, 3, 9)):
            uid = base + 4 + 6 * u
            y = F.conv1d(snake(x, val(uid, (ch,), 0.1, True)),
                         val(uid + 1, (ch, ch, 7), (7 * ch) ** -0.5),
                         val(uid + 2, (ch,), 0.01), dilation=d, padding=3 * d)
            y = F.conv1d(snake(y, val(uid + 3, (ch,), 0.1, True)),
                         val(uid + 4, (ch, ch, 1), 0.3 * ch ** -0.5), val(uid + 5, (ch,), 0.01))
            x = x + y
    x = snake(x, val(1400, (ch,), 0.1, True))
    return F.conv1d(x, val(1401, (1, ch, 7), 0.1 * (7 * ch) ** -0.5), val(1402, (1,), 0.01),
                    padding=3)[0, 0].numpy()


@pytest.mark.parametrize("frames", [1, 6])
def test_codec_decode_matches_torch_composition(frames):
    codec = oracle.Codec(TINY, 77)
    codes = np.random.default_rng(frames).integers(0, 16, size=(3, frames)).astype(np.int32)
    got = codec.decode(codes)
    want = _torch_decoder(TINY, 77, codes)
    assert got.shape == want.shape == (frames * 24,)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_codec_decode_matches_transformers_fixture():
    """tests/golden/codec_tiny.json: the installed transformers' DAC decoder
    with HiggsAudioV2's output padding and no tanh, after the RVQ decode and
    fc2, on the synthetic weights (made by tests/golden/make_codec_golden.py)."""
    import json
    import os
    from conftest import GOLDEN
    with open(os.path.join(GOLDEN, "codec_tiny.json")) as f:
        golden = json.load(f)
    codes = np.array(golden["codes"], dtype=np.int32)
    got = oracle.Codec(golden["config"], golden["seed"]).decode(codes)
    want = np.array(golden["audio"])
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-6)
