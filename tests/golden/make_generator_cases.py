#!/usr/bin/env python3
"""Writes tests/golden/generator_cases.json: the CPU-usable vectors of the
reference's tests/fixtures/generator_golden.json (gufo-extensions/omnivoice)
and the greedy-selection known answer of its tests/decoding_test.cpp:67-80.

Kept: the decoding config, and per generate case the schedule, input_ids,
audio_start, target and reference codes (tests/decoding_test.cpp:43-65 checks
exactly these). The real-checkpoint statistics (forward.*, generate.*.tokens
and unmasked_at) need the OmniVoice weights and are left out.
"""
import json
import os
import sys

REFERENCE = "/root/reference/tests/fixtures/generator_golden.json"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)),
                   "generator_cases.json")


def main():
    with open(REFERENCE) as f:
        golden = json.load(f)
    cases = []
    for entry in golden["generate"]:
        cases.append({k: entry[k] for k in (
            "text", "audio_start", "target", "schedule", "input_ids",
            "reference_codes")})
    out = {
        "source": "gufo-extensions/omnivoice tests/fixtures/generator_golden.json"
                  " and tests/decoding_test.cpp:67-80",
        "config": golden["config"],
        "generate": cases,
        "greedy_kat": {
            "codebooks": 2, "frames": 3, "count": 2, "mask_id": 1024,
            "codes": [1024, 7, 1024, 1024, 1024, 1024],
            "prediction": [10, 11, 12, 13, 14, 15],
            "confidence": [-0.5, -0.1, -2.0, -0.2, -0.3, -9.0],
            "layer_penalty": 5.0,
            "chosen": [0, 2],
            "codes_after": [10, 7, 12, 1024, 1024, 1024],
        },
    }
    with open(OUT, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", OUT, file=sys.stderr)


if __name__ == "__main__":
    main()
