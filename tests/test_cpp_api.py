"""The reference-shaped C++ interface (include/omnivoice/*.hpp) through the
test programs under tests/cpp, built by __graft_entry__.build() (make -C
tests/cpp). The decoding program mirrors the reference's
tests/decoding_test.cpp on the committed fixture; the generator program
checks Generate / Forward / Score, cancellation and error reporting on a
small synthetic model."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CPP = os.path.join(HERE, "cpp")


def program(name):
    path = os.path.join(CPP, name)
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built: run __graft_entry__.build() "
                    "(make -C tests/cpp)")
    return path


def write_fixture(golden_cases, path):
    steps = golden_cases["config"]["num_step"]
    t_shift = golden_cases["config"]["t_shift"]
    lines = []
    for case in golden_cases["generate"]:
        target = case["target"]
        lines.append(" ".join(["schedule", str(8 * target), str(steps), repr(t_shift)]
                              + [str(c) for c in case["schedule"]]))
        ids = case["input_ids"]
        start = case["audio_start"]
        text = ids[0][:start]
        ref = case["reference_codes"] or []
        ref_frames = len(ref[0]) if ref else 0
        flat_ref = [v for row in ref for v in row]
        length = len(ids[0])
        flat_ids = [v for row in ids for v in row]
        lines.append(" ".join(
            ["input", "8", "1024", str(len(text))] + [str(t) for t in text]
            + [str(ref_frames)] + [str(v) for v in flat_ref]
            + [str(target), str(length)] + [str(v) for v in flat_ids]))
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def test_decoding_interface_matches_reference_fixture(golden_cases, tmp_path):
    fixture = tmp_path / "decoding_fixture.txt"
    write_fixture(golden_cases, fixture)
    run = subprocess.run([program("decoding_test"), str(fixture)],
                         capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stdout + run.stderr
    assert f"{2 * len(golden_cases['generate'])} fixture cases, 0 failures" in run.stdout


@pytest.mark.gpu
def test_generator_interface_contract():
    run = subprocess.run([program("generator_test")], capture_output=True,
                         text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
