"""Pins the oracle's forward pass: each piece against a float64 formulation
of the textbook operation at tiny shapes, and the whole forward against the
committed fixture computed with transformers' Qwen3 decoder layers."""
import json
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN


def _p(a):
    return a.ctypes.data


def test_rmsnorm_matches_float64():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((9, 256)).astype(np.float32) * 3
    w = rng.standard_normal(256).astype(np.float32)
    y = np.zeros_like(x)
    oracle.lib().orc_rmsnorm(_p(x), _p(w), _p(y), 9, 256, 1e-6)
    x64 = x.astype(np.float64)
    want = w * x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(y, want, rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("rows,k,n", [(7, 72, 13), (16, 128, 64), (5, 1024, 9)])
def test_linear_matches_float64(rows, k, n):
    rng = np.random.default_rng(rows)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    y = np.ones((rows, n), dtype=np.float32)
    oracle.lib().orc_linear(_p(x), _p(w), _p(y), rows, k, n, 1)
    want = 1.0 + x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(y, want, rtol=1e-4, atol=1e-4)


def test_qk_norm_rope_matches_complex_rotation():
    """Rotate-half RoPE is multiplication of (x_i + i x_{i+64}) by
    exp(i pos theta^(-2i/d)); q and k heads are RMS-normalised with their own
    weights, v heads pass through."""
    rng = np.random.default_rng(1)
    heads, kv, d, rows = 4, 2, 128, 6
    width = (heads + 2 * kv) * d
    x = rng.standard_normal((rows, width)).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    pos = np.array([0, 1, 5, 77, 300, 4000], dtype=np.int32)
    out = np.zeros_like(x)
    oracle.lib().orc_qk_norm_rope(_p(x), _p(qn), _p(kn), _p(pos), _p(out),
                                  rows, heads, kv, d, 1e-6, 1e6)
    half = d // 2
    # Hugging Face forms inv_freq and the angle in float32 (the reference's
    # kernel does the same); the rotation itself is then exact.
    freq = (np.float32(1.0) / np.float32(1e6) ** (np.arange(half, dtype=np.float32)
                                                 * np.float32(2.0 / d)))
    for r in range(rows):
        for s in range(heads + 2 * kv):
            v = x[r, s * d:(s + 1) * d].astype(np.float64)
            got = out[r, s * d:(s + 1) * d]
            if s >= heads + kv:
                np.testing.assert_array_equal(got, x[r, s * d:(s + 1) * d])
                continue
            w = qn if s < heads else kn
            v = w * v / np.sqrt((v ** 2).mean() + 1e-6)
            angle = (np.float32(pos[r]) * freq).astype(np.float64)
            z = (v[:half] + 1j * v[half:]) * np.exp(1j * angle)
            want = np.concatenate([z.real, z.imag])
            # One float32 ulp of inv_freq or of the angle moves the angle by
            # up to ~1e-7 * pos rad; a wrong sign, half or frequency is O(1).
            atol = 3e-5 + 3e-7 * pos[r] * np.abs(v).max()
            np.testing.assert_allclose(got, want, rtol=0, atol=atol)


def test_attention_matches_float64_with_gqa():
    rng = np.random.default_rng(4)
    heads, kv, d = 4, 2, 128
    seqs = [(0, 11), (16, 5)]
    rows = 21
    width = (heads + 2 * kv) * d
    qkv = rng.standard_normal((rows, width)).astype(np.float32)
    out = np.zeros((rows, heads * d), dtype=np.float32)
    s = np.array(seqs, dtype=np.int64).ravel()
    oracle.lib().orc_attention(_p(qkv), _p(out), rows, heads, kv, d, _p(s),
                               len(seqs), 0)
    x = qkv.astype(np.float64)
    for first, length in seqs:
        for h in range(heads):
            g = h // (heads // kv)
            q = x[first:first + length, h * d:(h + 1) * d]
            k = x[first:first + length, (heads + g) * d:(heads + g + 1) * d]
            v = x[first:first + length, (heads + kv + g) * d:(heads + kv + g + 1) * d]
            a = q @ k.T / np.sqrt(d)
            p = np.exp(a - a.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            np.testing.assert_allclose(out[first:first + length, h * d:(h + 1) * d],
                                       p @ v, rtol=1e-4, atol=1e-5)


def test_forward_matches_transformers_fixture():
    with open(os.path.join(GOLDEN, "forward_tiny.json")) as f:
        golden = json.load(f)
    cfg = golden["config"]
    for case in golden["cases"]:
        model = oracle.Model(cfg, seed=case["seed"],
                             norm_jitter=case["norm_jitter"])
        ids = np.array(case["ids"], dtype=np.int32)
        got = model.forward(ids, case["audio_start"], case["target"])
        want = np.array(case["logits"])
        assert np.abs(got - want).max() < 5e-6
        assert np.linalg.norm(got - want) / np.linalg.norm(want) < 5e-6


def test_emulated_fp16_stays_close_to_float32():
    """Rounding at the reference's fp16 points moves the tiny model's logits
    by far less than the parity tolerance."""
    with open(os.path.join(GOLDEN, "forward_tiny.json")) as f:
        golden = json.load(f)
    case = golden["cases"][0]
    model = oracle.Model(golden["config"], seed=case["seed"],
                         norm_jitter=case["norm_jitter"])
    ids = np.array(case["ids"], dtype=np.int32)
    a = model.forward(ids, case["audio_start"], case["target"], emulate=False)
    b = model.forward(ids, case["audio_start"], case["target"], emulate=True)
    assert 0 < np.abs(a - b).max() < 5e-3


def _host_tensors(cfg, seed, jitter):
    """The synthetic model's values as host float32 tensors in the layout
    orc_model_from_host takes (the reference's Load order: text, audio
    embeddings, audio heads, final norm, then per layer q, k, v, o, gate, up,
    down, input norm, post norm, q norm, k norm), drawn with the oracle's own
    generator."""
    h, i = cfg["hidden_size"], cfg["intermediate_size"]
    q, kv, d = cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"], cfg["head_dim"]
    audio_rows = cfg["audio_codebooks"] * cfg["audio_vocab_size"]

    def values(tensor, shape, norm=False):
        out = np.zeros(int(np.prod(shape)), dtype=np.float32)
        oracle.lib().orc_synth_values(seed, tensor, 0, out.size, int(norm), jitter,
                                      out.ctypes.data)
        return out.reshape(shape)

    shapes = [(q, h), (kv, h), (kv, h), (h, q), (i, h), (i, h), (h, i),
              (h,), (h,), (d,), (d,)]
    layers = [[values(100 + 16 * l + k, shape, k >= 7) for k, shape in enumerate(shapes)]
              for l in range(cfg["layers"])]
    return {"text": values(1, (cfg["vocab_size"], h)),
            "audio_embeddings": values(2, (audio_rows, h)),
            "audio_heads": values(3, (audio_rows, h)),
            "final_norm": values(4, (h,), True), "layers": layers}


def test_model_from_host_matches_synthetic_model():
    """orc_model_from_host (generator.cpp:364-425 layout: q|k|v and gate|up
    fused in that order) given the synthetic model's tensors gives the
    synthetic model's logits bit for bit; the synthetic model is pinned by
    the transformers fixture above. Swapping gate and up, or k and v, moves
    the logits, so the fused order is what is checked."""
    from conftest import random_input, tiny_config
    cfg = tiny_config()
    host = _host_tensors(cfg, 21, 0.1)
    synthetic = oracle.Model(cfg, 21, 0.1)
    loaded = oracle.Model(cfg, host=host)
    rng = np.random.default_rng(3)
    ids = random_input(rng, cfg, 7, 5, 19, 0.3)
    for emulate in (False, True):
        a = synthetic.forward(ids, 7, 19, emulate=emulate)
        b = loaded.forward(ids, 7, 19, emulate=emulate)
        assert a.tobytes() == b.tobytes()
    for x, y in [(4, 5), (1, 2)]:
        bad = dict(host, layers=[list(layer) for layer in host["layers"]])
        bad["layers"][0][x], bad["layers"][0][y] = bad["layers"][0][y], bad["layers"][0][x]
        swapped = oracle.Model(cfg, host=bad).forward(ids, 7, 19)
        assert np.abs(swapped - synthetic.forward(ids, 7, 19)).max() > 1e-3


@pytest.mark.parametrize("temperature,seed,target", [(0.0, 0, 12), (5.0, 42, 12), (5.0, 7, 3)])
def test_closed_loop_generate_matches_stepwise_loop(temperature, seed, target):
    """orc_generate (the closed loop of generator.cpp:486-543) equals the loop
    spelled out step by step from pinned pieces: the forward, the score and
    the reference's own compiled PositionSelector (oracle/_ref, when built;
    the oracle's selector, pinned against it, otherwise), writing each step's
    chosen codes into the conditional target frames (generator.cpp:526-535)
    and skipping zero-count steps."""
    from conftest import random_input, tiny_config
    cfg = tiny_config()
    model = oracle.Model(cfg, 21, 0.1)
    rng = np.random.default_rng(seed + 5)
    text, ref = 6, 4
    ids = random_input(rng, cfg, text, ref, target)
    codes, at = model.generate(ids, text, target, temperature=temperature, seed=seed)
    sel = oracle.Selector(5.0, temperature, seed, use_ref=oracle.ref_available())
    current = ids.copy()
    expect = np.full(8 * target, 1024, dtype=np.int32)
    expect_at = np.full(8 * target, -1, dtype=np.int32)
    steps = 0
    for step, count in enumerate(oracle.unmask_schedule(8 * target, 32, 0.1)):
        if count == 0:
            continue
        steps += 1
        logits = model.forward(current, text, target)
        pred, conf = oracle.score(logits, target, 8, 1025, 1024, 2.0)
        for i in sel.fill(count, 8, target, pred, conf, 1024, expect):
            expect_at[i] = step
        current[:, -target:] = expect.reshape(8, target)
    assert steps == (32 if target == 12 else 24)  # 24 positions leave 8 steps empty
    np.testing.assert_array_equal(codes.ravel(), expect)
    np.testing.assert_array_equal(at.ravel(), expect_at)
    assert (codes != 1024).all()


# ------------------------------------------------------------------ fp16 rounding points
#
# The reference rounds to fp16 where its kernels write half outputs
# (kernels/generator_kernels.hip:85-200 and generator.cpp:161-176): the
# RMSNorm outputs (input, post-attention and final norm), the q/k/v heads
# after QkNormRope (v passed through), the softmax probabilities, the merged
# heads and the SwiGLU output. The oracle's emulating forward must round at
# exactly those points and nowhere else.
#
# An end-to-end float64 forward cannot pin that by tolerance: rounding is
# discontinuous, so a float32-vs-float64 difference of one part in 1e7 before
# a rounding point flips a few half-ulp decisions, and the flips compound
# through the fourteen rounding stages of even a two-layer model until two
# correctly rounded forwards differ by the rounding noise itself (~3e-4
# rel-L2 here, the same as rounding versus not rounding). The pin is
# therefore structural and bit-exact: orc_forward equals the composition of
# its separately pinned pieces (RMSNorm, linear, QkNormRope, attention,
# SwiGLU: float64 tests above and below) with fp16 rounding at exactly the
# listed points, for both modes.

ROUNDING_POINTS = ("input_norm", "qkv", "probabilities", "merged", "post_norm",
                   "swiglu", "final_norm")


def _f16(x):
    return x.astype(np.float16).astype(np.float32)


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_round_half_is_round_to_nearest_even():
    """orc_round_half equals numpy's float32 -> float16 conversion (round to
    nearest, ties to even) over normal, subnormal, tie and overflow values."""
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(3),
        (rng.standard_normal(1000) * 1e-6).astype(np.float32),   # fp16 subnormals
        (np.arange(-2048, 2048, dtype=np.float32) + np.float32(0.5)),  # ties above 1024
        np.float32([65504, 65519, 65520, 1e6, -1e6, 0.0, -0.0, 6.1035156e-05]),
    ]).astype(np.float32)
    got = np.array([oracle.lib().orc_round_half(float(v)) for v in x], dtype=np.float32)
    want = _f16(x)
    assert got.tobytes() == want.tobytes()


def test_swiglu_matches_float64():
    rng = np.random.default_rng(6)
    rows, inter = 5, 96
    gu = (rng.standard_normal((rows, 2 * inter)) * 4).astype(np.float32)
    out = np.zeros((rows, inter), dtype=np.float32)
    oracle.lib().orc_swiglu(_p(gu), _p(out), rows, inter)
    g, u = gu[:, :inter].astype(np.float64), gu[:, inter:].astype(np.float64)
    np.testing.assert_allclose(out, g / (1 + np.exp(-g)) * u, rtol=3e-6, atol=1e-7)


def _composed_forward(cfg, host, ids, audio_start, frames, rounded):
    """Generator::Forward (generator.cpp:175-301) composed from the oracle's
    pinned pieces, rounding to fp16 at the points in `rounded`."""
    L = oracle.lib()
    eps, theta = cfg["rms_norm_eps"], cfg["rope_theta"]
    C, V = cfg["audio_codebooks"], cfg["audio_vocab_size"]
    heads, kv, d = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    hs, inter = cfg["hidden_size"], cfg["intermediate_size"]
    qkv_width = (heads + 2 * kv) * d
    rnd = {p: (_f16 if p in rounded else (lambda x: x)) for p in ROUNDING_POINTS}
    f16 = lambda a: np.ascontiguousarray(_f16(a))  # the reference loads matrices as fp16
    length = ids.shape[1]
    rows = length + frames
    packed = np.concatenate([ids, ids[:, length - frames:]], axis=1)
    h = np.zeros((rows, hs), dtype=np.float32)
    for r in range(rows):
        if r < audio_start:
            h[r] = host["text"][packed[0, r]]
        else:
            acc = np.zeros(hs, dtype=np.float32)
            for c in range(C):   # float32, codebook order, from +0
                acc = acc + host["audio_embeddings"][c * V + packed[c, r]]
            h[r] = acc
    positions = np.concatenate([np.arange(length), np.arange(frames)]).astype(np.int32)
    seqs = np.array([0, length, length, frames], dtype=np.int64)

    def norm(x, w):
        y = np.zeros_like(x)
        L.orc_rmsnorm(_p(x), _p(w), _p(y), x.shape[0], x.shape[1], eps)
        return y

    for wq, wk, wv, wo, wg, wu, wd, n_in, n_post, n_q, n_k in host["layers"]:
        x = np.ascontiguousarray(rnd["input_norm"](norm(h, n_in)))
        wqkv = f16(np.concatenate([wq, wk, wv]))
        qkv = np.zeros((rows, qkv_width), dtype=np.float32)
        L.orc_linear(_p(x), _p(wqkv), _p(qkv), rows, hs, qkv_width, 0)
        roped = np.zeros_like(qkv)
        L.orc_qk_norm_rope(_p(qkv), _p(n_q), _p(n_k), _p(positions), _p(roped), rows,
                           heads, kv, d, eps, theta)
        roped = np.ascontiguousarray(rnd["qkv"](roped))
        merged = np.zeros((rows, heads * d), dtype=np.float32)
        L.orc_attention(_p(roped), _p(merged), rows, heads, kv, d, _p(seqs), 2,
                        int("probabilities" in rounded))
        merged = np.ascontiguousarray(rnd["merged"](merged))
        wo16 = f16(wo)
        L.orc_linear(_p(merged), _p(wo16), _p(h), rows, heads * d, hs, 1)
        x = np.ascontiguousarray(rnd["post_norm"](norm(h, n_post)))
        wgu = f16(np.concatenate([wg, wu]))
        gu = np.zeros((rows, 2 * inter), dtype=np.float32)
        L.orc_linear(_p(x), _p(wgu), _p(gu), rows, hs, 2 * inter, 0)
        act = np.zeros((rows, inter), dtype=np.float32)
        L.orc_swiglu(_p(gu), _p(act), rows, inter)
        act = np.ascontiguousarray(rnd["swiglu"](act))
        wd16 = f16(wd)
        L.orc_linear(_p(act), _p(wd16), _p(h), rows, inter, hs, 1)
    target = np.ascontiguousarray(np.concatenate([h[length - frames:length], h[length:]]))
    x = np.ascontiguousarray(rnd["final_norm"](norm(target, host["final_norm"])))
    heads_w = f16(host["audio_heads"])
    logits = np.zeros((2 * frames, C * V), dtype=np.float32)
    L.orc_linear(_p(x), _p(heads_w), _p(logits), 2 * frames, hs, C * V, 0)
    return logits


def test_forward_rounds_exactly_at_the_reference_points():
    """orc_forward(emulate=1) is bit for bit the composition of the pinned
    pieces rounding at the seven points, orc_forward(emulate=0) the one
    rounding nowhere; leaving out any single point changes the bits."""
    from conftest import random_input, tiny_config
    cfg = tiny_config()
    host = _host_tensors(cfg, 21, 0.1)
    model = oracle.Model(cfg, host=host)
    rng = np.random.default_rng(17)
    text, ref, frames = 7, 5, 19
    ids = random_input(rng, cfg, text, ref, frames, 0.3)
    emulated = model.forward(ids, text, frames, emulate=True)
    plain = model.forward(ids, text, frames, emulate=False)
    every = _composed_forward(cfg, host, ids, text, frames, set(ROUNDING_POINTS))
    assert emulated.tobytes() == every.tobytes()
    assert plain.tobytes() == _composed_forward(cfg, host, ids, text, frames, set()).tobytes()
    for point in ROUNDING_POINTS:
        without = _composed_forward(cfg, host, ids, text, frames,
                                    set(ROUNDING_POINTS) - {point})
        assert without.tobytes() != emulated.tobytes(), point


def test_attention_rounded_probabilities_match_float64():
    """orc_attention(round_p=1) is the float64 attention with the
    probabilities rounded to fp16 before P V (the reference's SoftmaxKernel
    writes half probabilities, kernels/generator_kernels.hip:161-176); the
    unrounded mode is the plain float64 attention."""
    rng = np.random.default_rng(9)
    heads, kv, d = 4, 2, 128
    seqs = [(0, 37), (48, 23)]
    rows = 71
    width = (heads + 2 * kv) * d
    qkv = (rng.standard_normal((rows, width)) * 2).astype(np.float32)
    s = np.array(seqs, dtype=np.int64).ravel()
    got = {}
    for round_p in (0, 1):
        out = np.zeros((rows, heads * d), dtype=np.float32)
        oracle.lib().orc_attention(_p(qkv), _p(out), rows, heads, kv, d, _p(s),
                                   len(seqs), round_p)
        got[round_p] = out
    x = qkv.astype(np.float64)
    f16 = lambda a: a.astype(np.float16).astype(np.float64)
    want = {0: np.zeros((rows, heads * d)), 1: np.zeros((rows, heads * d))}
    for first, length in seqs:
        for h in range(heads):
            g = h // (heads // kv)
            q = x[first:first + length, h * d:(h + 1) * d]
            k = x[first:first + length, (heads + g) * d:(heads + g + 1) * d]
            v = x[first:first + length, (heads + kv + g) * d:(heads + kv + g + 1) * d]
            a = q @ k.T / np.sqrt(d)
            p = np.exp(a - a.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            want[0][first:first + length, h * d:(h + 1) * d] = p @ v
            want[1][first:first + length, h * d:(h + 1) * d] = f16(p) @ v
    live = np.concatenate([np.arange(f, f + n) for f, n in seqs])
    moved = _rel(want[1][live], want[0][live])
    for round_p in (0, 1):
        d = _rel(got[round_p][live], want[round_p][live])
        print(f"round_p={round_p}: {d:.2e} (rounding moves {moved:.2e})")
        assert d < moved / 20
