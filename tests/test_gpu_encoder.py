"""The audio encoder through the C ABI against the oracle: the whole encoder
at a small configuration (intermediate outputs within 1e-4 of their scale,
every code equal), against the transformers fixture, without resampling,
and at the released configuration within the reference's own encode bound
(codec_test.cpp:110-123: at least 90 % of the codes agree); the device entry
point, errors, and a checkpoint written with the reference's tensor
names."""
import json
import os

import numpy as np
import pytest

import omnivoice_amd as ov
import oracle

pytestmark = pytest.mark.gpu


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not _gpu_available():
        pytest.skip("no GPU")


def close(got, want, rtol):
    scale = max(float(np.abs(want).max()), 1e-3)
    err = float(np.abs(got - want).max())
    assert err <= rtol * scale, (err, scale)


def signal(length, seed=0):
    t = np.arange(length)
    rng = np.random.default_rng(seed)
    return (0.3 * np.sin(2 * np.pi * 220 * t / 24000) * (0.5 + 0.5 * np.sin(t / 900))
            + 0.03 * rng.standard_normal(length)).astype(np.float32)


def compare(got, want, rtol=1e-4, codes_equal=True):
    for key in ("semantic", "acoustic", "embeddings"):
        assert got[key].shape == want[key].shape, key
        close(got[key], want[key], rtol)
    if codes_equal:
        np.testing.assert_array_equal(got["codes"], want["codes"])


@pytest.mark.parametrize("frames", [1, 9, 40, 1100])  # 1100: over 2048 HuBERT steps
def test_tiny_encode_matches_oracle(frames):
    cfg = oracle.encoder_tiny_config()
    x = signal(frames * cfg["frame_samples"], frames)
    got = ov.Encoder.synthetic(cfg, 77).encode(x, intermediates=True)
    want = oracle.Encoder(cfg, 77).encode(x)
    compare(got, want)


def test_encode_matches_transformers_fixture():
    """The GPU encoder against transformers' HubertModel and DacEncoder plus
    torch float64 layers on the same synthetic weights
    (tests/golden/encoder_tiny.json)."""
    from conftest import GOLDEN
    with open(os.path.join(GOLDEN, "encoder_tiny.json")) as f:
        g = json.load(f)
    got = ov.Encoder.synthetic(g["config"], g["seed"]).encode(
        np.array(g["signal"], np.float32), intermediates=True)
    want = {k: np.array(g[k]) for k in ("semantic", "acoustic", "embeddings", "codes")}
    compare(got, want)


def test_encode_without_resampling():
    cfg = dict(oracle.encoder_tiny_config(), semantic_rate=24000)
    x = signal(24 * 12, 3)
    got = ov.Encoder.synthetic(cfg, 5).encode(x, intermediates=True)
    compare(got, oracle.Encoder(cfg, 5).encode(x))


@pytest.fixture(scope="module")
def released():
    cfg = ov.encoder_released_config()
    return cfg, ov.Encoder.synthetic(cfg, 1234), oracle.Encoder(oracle.encoder_released_config(),
                                                                1234)


def test_released_encode_within_reference_bound(released):
    cfg, enc, model = released
    x = signal(50 * 960, 11)
    got = enc.encode(x, intermediates=True)
    want = model.encode(x)
    agree = float((got["codes"] == want["codes"]).mean())
    per_book = (got["codes"] == want["codes"]).mean(axis=1)
    print(f"codes agree {agree:.4f} per codebook {np.round(per_book, 3)}")
    for key in ("semantic", "acoustic", "embeddings"):
        err = float(np.abs(got[key] - want[key]).max())
        print(f"{key}: max |d| {err:.2e} of {float(np.abs(want[key]).max()):.3f}")
    compare(got, want, rtol=1e-3, codes_equal=False)
    assert agree >= 0.9
    # the first codebook sees only the encoder's own rounding
    assert per_book[0] >= 0.98


def test_encode_deterministic_and_device_entry(released):
    import torch
    cfg, enc, _ = released
    x = signal(30 * 960, 2)
    a = enc.encode(x)
    np.testing.assert_array_equal(a, enc.encode(x))
    codes = torch.zeros((8, 30), dtype=torch.int32, device="cuda")
    enc.encode_device(torch.from_numpy(x).cuda(), codes)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(codes.cpu().numpy(), a)
    # a shorter encode after a longer one reuses the grown buffers
    short = x[:4 * 960]
    np.testing.assert_array_equal(enc.encode(short), enc.encode(short.copy()))


def test_encode_errors_carry_reference_prefix(released):
    _, enc, _ = released
    with pytest.raises(ov.GeneratorError,
                       match="^OmniVoice encode: reference audio must be a whole number"):
        enc.encode(np.zeros(961, np.float32))
    with pytest.raises(ov.GeneratorError, match="^OmniVoice encode: reference audio must"):
        enc.encode(np.zeros(0, np.float32))


def _synth(seed, tid, shape, scale, offset=0.0, exponential=False):
    n = int(np.prod(shape))
    v = np.array([oracle.lib().orc_synth_normal(seed, tid, e) for e in range(n)])
    out = np.exp(0.1 * v) if exponential else offset + scale * v
    return out.astype(np.float32).reshape(shape)


def _checkpoint_tensors(c, seed):
    """The synthetic encoder under the reference's tensor names and shapes
    (codec_encoder.cpp:74-240)."""
    W, I = c["width"], c["intermediate"]
    H, D, E = W + c["latent"], c["codebook_dim"], c["codebook_size"]
    t = {}
    s = lambda name, tid, shape, scale, offset=0.0: t.__setitem__(
        name, _synth(seed, tid, shape, scale, offset))
    a = lambda name, tid, shape: t.__setitem__(name, _synth(seed, tid, shape, 0.1, 0.0, True))
    sm = "semantic_model."
    cin = 1
    for i, (cd, k) in enumerate(zip(c["conv_dim"], c["conv_kernel"])):
        s(f"{sm}feature_extractor.conv_layers.{i}.conv.weight", 2000 + i, (cd, cin, k),
          (cin * k) ** -0.5)
        cin = cd
    c0 = c["conv_dim"][0]
    s(f"{sm}feature_extractor.conv_layers.0.layer_norm.weight", 2010, (c0,), 0.1, 1.0)
    s(f"{sm}feature_extractor.conv_layers.0.layer_norm.bias", 2011, (c0,), 0.1)
    s(f"{sm}feature_projection.layer_norm.weight", 2012, (cin,), 0.1, 1.0)
    s(f"{sm}feature_projection.layer_norm.bias", 2013, (cin,), 0.1)
    s(f"{sm}feature_projection.projection.weight", 2014, (W, cin), cin ** -0.5)
    s(f"{sm}feature_projection.projection.bias", 2015, (W,), 0.01)
    K, G = c["pos_kernel"], c["pos_groups"]
    p = f"{sm}encoder.pos_conv_embed.conv."
    s(p + "parametrizations.weight.original0", 2016, (1, 1, K), 0.1, 1.0)
    s(p + "parametrizations.weight.original1", 2017, (W, W // G, K), 1.0)
    s(p + "bias", 2018, (W,), 0.01)
    s(f"{sm}encoder.layer_norm.weight", 2019, (W,), 0.1, 1.0)
    s(f"{sm}encoder.layer_norm.bias", 2020, (W,), 0.1)
    for l in range(c["layers"]):
        b, q = 2100 + 16 * l, f"{sm}encoder.layers.{l}."
        for j, name in enumerate(("q_proj", "k_proj", "v_proj")):
            s(q + f"attention.{name}.weight", b + 2 * j, (W, W), W ** -0.5)
            s(q + f"attention.{name}.bias", b + 2 * j + 1, (W,), 0.01)
        s(q + "attention.out_proj.weight", b + 6, (W, W), W ** -0.5)
        s(q + "attention.out_proj.bias", b + 7, (W,), 0.01)
        s(q + "layer_norm.weight", b + 8, (W,), 0.1, 1.0)
        s(q + "layer_norm.bias", b + 9, (W,), 0.1)
        s(q + "feed_forward.intermediate_dense.weight", b + 10, (I, W), W ** -0.5)
        s(q + "feed_forward.intermediate_dense.bias", b + 11, (I,), 0.01)
        s(q + "feed_forward.output_dense.weight", b + 12, (W, I), 0.5 * I ** -0.5)
        s(q + "feed_forward.output_dense.bias", b + 13, (W,), 0.01)
        s(q + "final_layer_norm.weight", b + 14, (W,), 0.1, 1.0)
        s(q + "final_layer_norm.bias", b + 15, (W,), 0.1)
    s("encoder_semantic.conv.weight", 2400, (W, W, 3), (3 * W) ** -0.5)
    for bl in range(2):
        p = f"encoder_semantic.conv_blocks.{bl}"
        for u in range(2):
            s(f"{p}.res_units.{u}.conv1.weight", 2410 + 10 * bl + 2 * u, (W, W, 3),
              (3 * W) ** -0.5)
            s(f"{p}.res_units.{u}.conv2.weight", 2411 + 10 * bl + 2 * u, (W, W, 1),
              0.3 * W ** -0.5)
        s(f"{p}.conv.weight", 2450 + 2 * bl, (W, W, 3), (3 * W) ** -0.5)
        s(f"{p}.conv.bias", 2451 + 2 * bl, (W,), 0.01)
    ch = c["enc_channels"]
    s("acoustic_encoder.conv1.weight", 2500, (ch, 1, 7), 7 ** -0.5)
    s("acoustic_encoder.conv1.bias", 2501, (ch,), 0.01)
    for i, st in enumerate(c["ratios"]):
        b, p = 2600 + 32 * i, f"acoustic_encoder.block.{i}"
        for u in range(3):
            uid, r = b + 4 + 6 * u, f"{p}.res_unit{u + 1}"
            a(r + ".snake1.alpha", uid, (1, ch, 1))
            s(r + ".conv1.weight", uid + 1, (ch, ch, 7), (7 * ch) ** -0.5)
            s(r + ".conv1.bias", uid + 2, (ch,), 0.01)
            a(r + ".snake2.alpha", uid + 3, (1, ch, 1))
            s(r + ".conv2.weight", uid + 4, (ch, ch, 1), 0.3 * ch ** -0.5)
            s(r + ".conv2.bias", uid + 5, (ch,), 0.01)
        a(p + ".snake1.alpha", b, (1, ch, 1))
        s(p + ".conv1.weight", b + 1, (2 * ch, ch, 2 * st), (2 * ch * st) ** -0.5)
        s(p + ".conv1.bias", b + 2, (2 * ch,), 0.01)
        ch *= 2
    a("acoustic_encoder.snake1.alpha", 2800, (1, ch, 1))
    s("acoustic_encoder.conv2.weight", 2801, (c["latent"], ch, 3), (3 * ch) ** -0.5)
    s("acoustic_encoder.conv2.bias", 2802, (c["latent"],), 0.01)
    s("fc.weight", 2810, (H, H), H ** -0.5)
    s("fc.bias", 2811, (H,), 0.01)
    for q in range(c["codebooks"]):
        p = f"quantizer.quantizers.{q}"
        s(p + ".project_in.weight", 2900 + 2 * q, (D, H), H ** -0.5)
        s(p + ".project_in.bias", 2901 + 2 * q, (D,), 0.01)
        s(p + ".codebook.embed", 1000 + 4 * q, (E, D), 0.35)
        s(p + ".project_out.weight", 1001 + 4 * q, (H, D), D ** -0.5)
        s(p + ".project_out.bias", 1002 + 4 * q, (H,), 0.01)
    return t


def test_checkpoint_matches_synthetic_encoder(tmp_path):
    from safetensors.numpy import save_file
    cfg = oracle.encoder_tiny_config()
    os.makedirs(tmp_path / "audio_tokenizer")
    path = str(tmp_path / "audio_tokenizer" / "model.safetensors")
    tensors = _checkpoint_tensors(cfg, 99)
    save_file(tensors, path)
    x = signal(24 * 7, 4)
    from_file = ov.Encoder.load(cfg, str(tmp_path)).encode(x, intermediates=True)
    synthetic = ov.Encoder.synthetic(cfg, 99).encode(x, intermediates=True)
    for key in synthetic:
        np.testing.assert_array_equal(from_file[key], synthetic[key])
    # a tensor of the wrong shape is named
    tensors["fc.bias"] = np.zeros(5, dtype=np.float32)
    save_file(tensors, path)
    with pytest.raises(ov.GeneratorError, match="^OmniVoice audio tokenizer: .*fc.bias"):
        ov.Encoder.load(cfg, str(tmp_path))
