"""Pins the CPU oracle (test infrastructure) before it is trusted as the
checker: the reference's golden vectors and known answers, the reference's
own decoding.cpp compiled into oracle/_ref, and closed forms."""
import json
import math
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN

ref_only = pytest.mark.skipif(not oracle.ref_available(),
                              reason="oracle/_ref not built (needs /root/reference)")


# ------------------------------------------------------------ schedule / build

def test_schedule_matches_reference_fixture(golden_cases):
    steps = golden_cases["config"]["num_step"]
    t_shift = golden_cases["config"]["t_shift"]
    for case in golden_cases["generate"]:
        got = oracle.unmask_schedule(8 * case["target"], steps, t_shift)
        assert got == case["schedule"], case["text"]


def test_schedule_invariants():
    for total in [0, 1, 7, 400, 2000, 3000, 16384]:
        for steps in [1, 2, 16, 32, 64]:
            s = oracle.unmask_schedule(total, steps, 0.1)
            assert sum(s) == total and min(s) >= 0 and len(s) == steps


@ref_only
def test_schedule_matches_compiled_reference():
    R = oracle.ref()
    for total in [1, 8, 400, 520, 2000, 2999, 3000, 12345]:
        for steps in [1, 5, 16, 32, 33]:
            for t_shift in [0.1, 0.5, 1.0]:
                out = np.zeros(steps, dtype=np.int64)
                R.ref_unmask_schedule(total, steps, t_shift, out.ctypes.data)
                assert oracle.unmask_schedule(total, steps, t_shift) == out.tolist()


def test_build_matches_reference_fixture(golden_cases):
    for case in golden_cases["generate"]:
        ids = np.array(case["input_ids"], dtype=np.int32)
        a = case["audio_start"]
        refc = case["reference_codes"]
        rf = 0 if refc is None else len(refc[0])
        built = oracle.build_input(ids[0, :a], refc, rf, case["target"])
        np.testing.assert_array_equal(built, ids)


@ref_only
def test_build_matches_compiled_reference():
    rng = np.random.default_rng(3)
    R = oracle.ref()
    for text, rf, target in [(0, 0, 1), (5, 0, 7), (12, 9, 30), (1, 40, 2)]:
        t = rng.integers(0, 151936, size=max(text, 1)).astype(np.uint32)[:text]
        refc = rng.integers(0, 1024, size=(8, max(rf, 1))).astype(np.int32)[:, :rf]
        mine = oracle.build_input(t, refc, rf, target)
        ref_ids = np.zeros(8 * (text + rf + target), dtype=np.int32)
        tt = np.ascontiguousarray(t) if text else np.zeros(1, dtype=np.uint32)
        rr = np.ascontiguousarray(refc) if rf else np.zeros(1, dtype=np.int32)
        n = R.ref_build_input(tt.ctypes.data, text, rr.ctypes.data, rf, target,
                              8, 1024, ref_ids.ctypes.data)
        assert n == text + rf + target
        np.testing.assert_array_equal(mine.ravel(), ref_ids)


# ------------------------------------------------------------ selector

def _kat(golden_cases):
    return golden_cases["greedy_kat"]


@pytest.mark.parametrize("use_ref", [False, pytest.param(True, marks=ref_only)])
def test_selector_greedy_kat(golden_cases, use_ref):
    k = _kat(golden_cases)
    sel = oracle.Selector(k["layer_penalty"], 0.0, 0, use_ref=use_ref)
    codes = np.array(k["codes"], dtype=np.int32)
    chosen = sel.fill(k["count"], k["codebooks"], k["frames"], k["prediction"],
                      k["confidence"], k["mask_id"], codes)
    assert chosen == k["chosen"]
    assert codes.tolist() == k["codes_after"]


def test_mt19937_64_known_answer():
    # The C++ standard's required value of the 10000th draw of a
    # default-constructed std::mt19937_64 (seed 5489).
    assert oracle.lib().orc_mt19937_64_nth(5489, 10000) == 9981545732273789042


@ref_only
@pytest.mark.parametrize("temperature", [0.0, 5.0, 1.0])
def test_selector_matches_compiled_reference(temperature):
    rng = np.random.default_rng(int(temperature * 10) + 1)
    C, F = 8, 57
    mine = oracle.Selector(5.0, temperature, 1234)
    theirs = oracle.Selector(5.0, temperature, 1234, use_ref=True)
    codes_a = np.full(C * F, 1024, dtype=np.int32)
    codes_b = codes_a.copy()
    for count in oracle.unmask_schedule(C * F, 32, 0.1):
        if count == 0:
            continue
        pred = rng.integers(0, 1024, size=C * F).astype(np.int32)
        conf = (-rng.exponential(2.0, size=C * F)).astype(np.float32)
        conf[rng.random(C * F) < 0.05] = -1.5  # ties
        a = mine.fill(count, C, F, pred, conf, 1024, codes_a)
        b = theirs.fill(count, C, F, pred, conf, 1024, codes_b)
        assert a == b
        np.testing.assert_array_equal(codes_a, codes_b)
    assert (codes_a != 1024).all()


def test_selector_greedy_bruteforce():
    """Greedy selection is the top `count` of float32 scores
    conf - c * penalty over masked entries, ties to the lower index."""
    rng = np.random.default_rng(5)
    C, F = 8, 33
    for trial in range(20):
        codes = np.full(C * F, 1024, dtype=np.int32)
        done = rng.random(C * F) < 0.3
        codes[done] = 5
        pred = rng.integers(0, 1024, size=C * F).astype(np.int32)
        conf = np.round(-rng.exponential(1.0, size=C * F), 1).astype(np.float32)
        count = int(rng.integers(1, (~done).sum() + 1))
        c_idx = np.repeat(np.arange(C), F).astype(np.float32)
        score = conf - c_idx * np.float32(5.0)
        score[done] = -np.inf
        order = np.lexsort((np.arange(C * F), -score.astype(np.float64)))
        expect = order[:count].tolist()
        sel = oracle.Selector(5.0, 0.0, 0)
        got = sel.fill(count, C, F, pred, conf, 1024, codes)
        assert got == expect


# ------------------------------------------------------------ exp / log / score

def _ulps(got, exact):
    got = np.asarray(got, dtype=np.float32)
    spacing = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - exact) / spacing


def test_exp_within_one_ulp():
    L = oracle.lib()
    xs = np.concatenate([np.linspace(-87.0, 0.0, 40001, dtype=np.float32),
                         np.linspace(0.0, 88.0, 4001, dtype=np.float32),
                         np.float32([-1e-8, 1e-8, -0.5, -86.99])])
    got = np.array([L.orc_exp(float(x)) for x in xs])
    assert _ulps(got, np.exp(xs.astype(np.float64))).max() <= 1.0
    assert L.orc_exp(-100.0) == 0.0 and L.orc_exp(0.0) == 1.0
    assert math.isinf(L.orc_exp(100.0)) and math.isnan(L.orc_exp(float("nan")))


def test_log_within_two_ulp():
    L = oracle.lib()
    ys = np.concatenate([np.exp(np.linspace(-100, 80, 40001)).astype(np.float32),
                         np.float32([1.0, 2.0, 1025.0, 1.0000001, 0.9999999,
                                     1e-40, 3e-39])])
    got = np.array([L.orc_log(float(y)) for y in ys])
    exact = np.log(ys.astype(np.float64))
    nz = exact != 0
    assert _ulps(got[nz], exact[nz]).max() <= 2.0
    assert L.orc_log(1.0) == 0.0 and L.orc_log(0.0) == -math.inf


def _score64(logits, F, C, V, mask, w):
    pred = np.zeros((C, F), dtype=np.int64)
    conf = np.zeros((C, F))
    x = logits.astype(np.float64)
    for f in range(F):
        for c in range(C):
            cr = x[f, c * V:(c + 1) * V]
            ur = x[F + f, c * V:(c + 1) * V]
            lc = cr - np.logaddexp.reduce(cr)
            lu = ur - np.logaddexp.reduce(ur)
            g = lc + w * (lc - lu)
            lg = g - np.logaddexp.reduce(g)
            lg_m = lg.copy()
            lg_m[mask] = -np.inf
            pred[c, f] = int(np.argmax(lg_m))
            conf[c, f] = lg_m[pred[c, f]]
    return pred, conf


@pytest.mark.parametrize("guidance", [0.0, 2.0, 3.5])
def test_score_matches_float64_closed_form(guidance):
    rng = np.random.default_rng(int(guidance * 10))
    F, C, V = 6, 8, 1025
    logits = (rng.standard_normal((2 * F, C * V)) * 2.0).astype(np.float32)
    pred, conf = oracle.score(logits, F, C, V, 1024, guidance)
    p64, c64 = _score64(logits, F, C, V, 1024, guidance)
    np.testing.assert_array_equal(pred, p64)
    np.testing.assert_allclose(conf, c64, atol=2e-5, rtol=0)
    assert (pred != 1024).all() and (conf <= 1e-6).all()


def test_score_mask_is_excluded_and_ties_take_lowest_index():
    F, C, V = 2, 8, 1025
    logits = np.zeros((2 * F, C * V), dtype=np.float32)
    for c in range(C):
        logits[:F, c * V + 1024] = 50.0          # the mask dominates ...
        logits[:F, c * V + 17] = 3.0             # ... then a tie between
        logits[:F, c * V + 900] = 3.0            # entries 17 and 900
    pred, conf = oracle.score(logits, F, C, V, 1024, 2.0)
    assert (pred == 17).all()
    # mask excluded from the argmax but not from the normaliser: conf << 0
    assert (conf < -40).all()


# ------------------------------------------------------------ fp16 / synthetic

def test_round_half_matches_numpy():
    rng = np.random.default_rng(9)
    x = np.concatenate([
        (rng.standard_normal(50000) * 0.02).astype(np.float32),
        (rng.standard_normal(50000) * 1e-6).astype(np.float32),
        (rng.standard_normal(20000) * 3e4).astype(np.float32),
        np.float32([65504, 65519.99, 65520, 6.1035e-5, 2.9802322e-8,
                    2.9802326e-8, 5.9604645e-8, 0.0, -0.0])])
    L = oracle.lib()
    got = np.array([L.orc_round_half(float(v)) for v in x], dtype=np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got, want)


def test_synthetic_normal_moments_and_rounding():
    L = oracle.lib()
    n = 200000
    z = np.array([L.orc_synth_normal(42, 7, e) for e in range(0, n, 4)])
    assert abs(z.mean()) < 0.02 and abs(z.std() - 1.0) < 0.02
    assert abs((np.abs(z) < 1.0).mean() - 0.6827) < 0.01
    w = np.zeros(4096, dtype=np.float32)
    L.orc_synth_values(42, 7, 0, 4096, 0, 0.0, w.ctypes.data)
    np.testing.assert_array_equal(w, w.astype(np.float16).astype(np.float32))
    assert abs(w.std() - 0.02) < 0.002
    other = np.zeros(4096, dtype=np.float32)
    L.orc_synth_values(42, 8, 0, 4096, 0, 0.0, other.ctypes.data)
    assert abs(np.corrcoef(w, other)[0, 1]) < 0.05
    norms = np.zeros(64, dtype=np.float32)
    L.orc_synth_values(42, 9, 0, 64, 1, 0.0, norms.ctypes.data)
    assert (norms == 1.0).all()


def test_generate_from_logits_consistent_with_stepwise_selector():
    """The teacher-forced loop equals score + Fill per executed step."""
    rng = np.random.default_rng(2)
    C, F, V = 8, 9, 1025
    sched = oracle.unmask_schedule(C * F, 32, 0.1)
    executed = sum(1 for s in sched if s)
    trace = rng.standard_normal((executed, 2 * F, C * V)).astype(np.float32)
    codes, at = oracle.generate_from_logits(trace, C, F, V, 1024,
                                            temperature=5.0, seed=77)
    sel = oracle.Selector(5.0, 5.0, 77)
    expect = np.full(C * F, 1024, dtype=np.int32)
    expect_at = np.full(C * F, -1, dtype=np.int32)
    e = 0
    for step, count in enumerate(sched):
        if not count:
            continue
        pred, conf = oracle.score(trace[e], F, C, V, 1024, 2.0)
        for i in sel.fill(count, C, F, pred, conf, 1024, expect):
            expect_at[i] = step
        e += 1
    np.testing.assert_array_equal(codes.ravel(), expect)
    np.testing.assert_array_equal(at.ravel(), expect_at)
    for step, count in enumerate(sched):
        assert (at == step).sum() == count
