"""Writes tests/golden/resample_cases.json: the reference's own resampler
vectors (the "resample" entries of its tests/fixtures/audio_golden.json, with
the fixture's sample stride), copied as data: signal recipe (segments, rate,
seed), target rate, output length and every stride-th output sample.

Run in the container that holds the reference tree:
python3 tests/golden/make_audio_golden.py
"""
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
SOURCE = "/root/reference/tests/fixtures/audio_golden.json"


def main():
    with open(SOURCE) as f:
        golden = json.load(f)
    out = {"source": "gufo-extensions/omnivoice tests/fixtures/audio_golden.json (resample)",
           "stride": golden["stride"], "cases": golden["resample"]}
    path = os.path.join(ROOT, "tests", "golden", "resample_cases.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print(path, len(out["cases"]))


if __name__ == "__main__":
    main()
