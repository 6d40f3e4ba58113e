"""The audio decoder through the C ABI against the oracle: each convolution
kernel (with and without the fused Snake, residual accumulation, every tile
shape, ragged channel counts and signal edges), the whole decoder at a tiny
and at the released configuration within the reference's own decode bounds
(codec_test.cpp:60-62: RMS within 1e-4, samples within 1e-3), determinism,
the device entry point, errors, and a checkpoint written with the
reference's tensor names."""
import math
import os

import numpy as np
import pytest

import omnivoice_amd as ov
import oracle

pytestmark = pytest.mark.gpu

TINY = dict(codebooks=3, codebook_size=16, codebook_dim=8, hidden=24, latent=12,
            channels=32, ratios=[2, 3, 4])


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


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def close(got, want, rtol=1e-4):
    scale = max(float(np.abs(want).max()), 1e-3)
    err = float(np.abs(got - want).max())
    assert err <= rtol * scale, (err, scale)


@pytest.mark.parametrize("cin,cout,length,kernel,dilation,snake,accumulate", [
    (16, 32, 300, 7, 1, False, False),    # 32 x 128 tiles
    (48, 64, 150, 7, 3, True, False),     # 64 x 64 tiles
    (32, 96, 97, 7, 9, True, True),       # ragged output channels and positions
    (21, 40, 64, 1, 1, True, True),       # ragged input channels, one tap
    (256, 1024, 25, 7, 1, False, False),  # the decoder's input convolution shape
    (64, 64, 5, 7, 9, True, False),       # signal shorter than the taps' spread
    (128, 128, 40000, 7, 1, True, True),  # long signals: hundreds of tiles
    (64, 64, 40000, 7, 3, True, False),
    (48, 96, 40000, 1, 1, True, True),    # long, one tap, ragged channels
])
def test_conv1d_matches_oracle(cin, cout, length, kernel, dilation, snake, accumulate):
    rng = np.random.default_rng(cin + cout + length)
    x = rng.standard_normal((cin, length)).astype(np.float32)
    w = (rng.standard_normal((cout, cin, kernel)) / math.sqrt(cin * kernel)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    alpha = np.exp(0.3 * rng.standard_normal(cin)).astype(np.float32) if snake else None
    y0 = rng.standard_normal((cout, length)).astype(np.float32)
    y = dev(y0)
    ov.op_conv1d(dev(x), w, b, y, alpha=dev(alpha) if snake else None, dilation=dilation,
                 accumulate=accumulate)
    xin = oracle.snake(x, alpha) if snake else x
    want = oracle.conv1d(xin, w, b, dilation) + (y0 if accumulate else 0)
    close(y.cpu().numpy(), want)


@pytest.mark.parametrize("cin,cout,length,stride,snake", [
    (64, 32, 40, 8, True), (32, 16, 33, 5, True), (128, 64, 70, 4, False),
    (16, 8, 9, 2, True), (48, 24, 31, 3, True), (1024, 512, 25, 8, True),
    (256, 128, 10000, 4, True)])  # long signal over four phases
def test_conv_transpose1d_matches_oracle(cin, cout, length, stride, snake):
    rng = np.random.default_rng(cin * stride + length)
    x = rng.standard_normal((cin, length)).astype(np.float32)
    w = (rng.standard_normal((cin, cout, 2 * stride)) / math.sqrt(2 * cin)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    alpha = np.exp(0.3 * rng.standard_normal(cin)).astype(np.float32) if snake else None
    y = dev(np.zeros((cout, length * stride)))
    ov.op_conv_transpose1d(dev(x), w, b, y, stride, alpha=dev(alpha) if snake else None)
    xin = oracle.snake(x, alpha) if snake else x
    close(y.cpu().numpy(), oracle.conv_transpose1d(xin, w, b, stride))


def test_synthetic_values_match_oracle():
    for tensor, scale, exp in [(1000, 0.35, False), (1205, 0.25, False), (1200, 0.1, True)]:
        np.testing.assert_array_equal(
            ov.codec_synthetic_values(1234, tensor, 17, 5000, scale, exp),
            oracle.codec_values(1234, tensor, 5000, scale, exp, first=17))


@pytest.mark.parametrize("frames", [1, 7, 40])
def test_tiny_decode_matches_oracle(frames):
    codec = ov.Codec.synthetic(TINY, 77)
    codes = np.random.default_rng(frames).integers(0, 16, size=(3, frames)).astype(np.int32)
    got = codec.decode(codes)
    want = oracle.Codec(TINY, 77).decode(codes)
    assert got.shape == want.shape == (frames * 24,)
    close(got, want, rtol=2e-4)


def test_decode_matches_transformers_fixture():
    """The GPU decoder against transformers' DAC decoder (HiggsAudioV2's
    output padding, no tanh) on the same synthetic weights
    (tests/golden/codec_tiny.json)."""
    import json
    from conftest import GOLDEN
    with open(os.path.join(GOLDEN, "codec_tiny.json")) as f:
        golden = json.load(f)
    codec = ov.Codec.synthetic(golden["config"], golden["seed"])
    got = codec.decode(np.array(golden["codes"], dtype=np.int32))
    close(got, np.array(golden["audio"]), rtol=2e-4)


@pytest.fixture(scope="module")
def released():
    cfg = ov.codec_released_config()
    return cfg, ov.Codec.synthetic(cfg, 1234), oracle.Codec(oracle.codec_released_config(), 1234)


@pytest.mark.parametrize("frames", [3, 25])
def test_released_decode_within_reference_bounds(released, frames):
    cfg, codec, model = released
    codes = np.random.default_rng(frames).integers(0, 1024, size=(8, frames)).astype(np.int32)
    got = codec.decode(codes)
    want = model.decode(codes)
    assert got.shape == want.shape == (frames * 960,)
    rms_got = float(np.sqrt(np.mean(got.astype(np.float64) ** 2)))
    rms_want = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    worst = float(np.abs(got - want).max())
    print(f"rms {rms_got:.6f} vs {rms_want:.6f}, max |d sample| {worst:.2e}")
    assert abs(rms_got - rms_want) < 1e-4
    assert worst < 1e-3


def test_decode_deterministic_and_device_entry(released):
    import torch
    cfg, codec, _ = released
    codes = np.random.default_rng(5).integers(0, 1024, size=(8, 50)).astype(np.int32)
    a = codec.decode(codes)
    b = codec.decode(codes)
    np.testing.assert_array_equal(a, b)
    codes_dev = torch.from_numpy(codes).cuda()
    audio = torch.empty(codec.samples(50), dtype=torch.float32, device="cuda")
    codec.decode_device(codes_dev, audio)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(audio.cpu().numpy(), a)
    # a shorter decode after a longer one reuses the grown buffers
    short = codec.decode(codes[:, :4])
    np.testing.assert_array_equal(short, codec.decode(codes[:, :4].copy()))


def test_decode_errors_carry_reference_prefix(released):
    _, codec, _ = released
    bad = np.zeros((8, 3), dtype=np.int32)
    bad[2, 1] = 1024
    with pytest.raises(ov.GeneratorError, match="^OmniVoice decode: code outside the codebook"):
        codec.decode(bad)
    with pytest.raises(ov.GeneratorError, match="^OmniVoice decode: no frames"):
        codec.decode(np.zeros((8, 0), dtype=np.int32))


def _checkpoint_tensors(cfg, seed):
    """The synthetic decoder written under the reference's tensor names and
    shapes (codec.cpp:112-181)."""
    v = lambda tid, shape, scale, exp=False: ov.codec_synthetic_values(
        seed, tid, 0, int(np.prod(shape)), scale, exp).reshape(shape)
    C, E, D, H, Lat = (cfg[k] for k in ("codebooks", "codebook_size", "codebook_dim",
                                        "hidden", "latent"))
    t = {}
    for c in range(C):
        p = f"quantizer.quantizers.{c}"
        t[p + ".codebook.embed"] = v(1000 + 4 * c, (E, D), 0.35)
        t[p + ".project_out.weight"] = v(1001 + 4 * c, (H, D), D ** -0.5)
        t[p + ".project_out.bias"] = v(1002 + 4 * c, (H,), 0.01)
    t["fc2.weight"] = v(1100, (Lat, H), H ** -0.5)
    t["fc2.bias"] = v(1101, (Lat,), 0.01)
    ch = cfg["channels"]
    t["acoustic_decoder.conv1.weight"] = v(1102, (ch, Lat, 7), (7 * Lat) ** -0.5)
    t["acoustic_decoder.conv1.bias"] = v(1103, (ch,), 0.01)
    for i, s in enumerate(cfg["ratios"]):
        p, base, out = f"acoustic_decoder.block.{i}", 1200 + 32 * i, ch // 2
        t[p + ".snake1.alpha"] = v(base, (1, ch, 1), 0.1, True)
        t[p + ".conv_t1.weight"] = v(base + 1, (ch, out, 2 * s), (2 * ch) ** -0.5)
        t[p + ".conv_t1.bias"] = v(base + 2, (out,), 0.01)
        for u in range(3):
            q, uid = f"{p}.res_unit{u + 1}", base + 4 + 6 * u
            t[q + ".snake1.alpha"] = v(uid, (1, out, 1), 0.1, True)
            t[q + ".conv1.weight"] = v(uid + 1, (out, out, 7), (7 * out) ** -0.5)
            t[q + ".conv1.bias"] = v(uid + 2, (out,), 0.01)
            t[q + ".snake2.alpha"] = v(uid + 3, (1, out, 1), 0.1, True)
            t[q + ".conv2.weight"] = v(uid + 4, (out, out, 1), 0.3 * out ** -0.5)
            t[q + ".conv2.bias"] = v(uid + 5, (out,), 0.01)
        ch = out
    t["acoustic_decoder.snake1.alpha"] = v(1400, (1, ch, 1), 0.1, True)
    t["acoustic_decoder.conv2.weight"] = v(1401, (1, ch, 7), 0.1 * (7 * ch) ** -0.5)
    t["acoustic_decoder.conv2.bias"] = v(1402, (1,), 0.01)
    return t


def test_checkpoint_matches_synthetic_decoder(tmp_path):
    from safetensors.numpy import save_file
    os.makedirs(tmp_path / "audio_tokenizer")
    save_file(_checkpoint_tensors(TINY, 99), str(tmp_path / "audio_tokenizer" /
                                                 "model.safetensors"))
    codes = np.random.default_rng(3).integers(0, 16, size=(3, 11)).astype(np.int32)
    from_file = ov.Codec.load(TINY, str(tmp_path)).decode(codes)
    np.testing.assert_array_equal(from_file, ov.Codec.synthetic(TINY, 99).decode(codes))
    # a tensor of the wrong shape is named
    t = _checkpoint_tensors(TINY, 99)
    t["fc2.bias"] = np.zeros(5, dtype=np.float32)
    save_file(t, str(tmp_path / "audio_tokenizer" / "model.safetensors"))
    with pytest.raises(ov.GeneratorError, match="^OmniVoice audio tokenizer: .*fc2.bias"):
        ov.Codec.load(TINY, str(tmp_path))
