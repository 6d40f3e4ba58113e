"""The C ABI without a GPU: the library loads and exports every function
include/omnivoice_mi355x.h declares; its host-only helpers agree with the
reference's fixtures and the oracle; configuration errors are reported the
reference's way."""
import ctypes
import os
import re

import numpy as np
import pytest

import omnivoice_amd as ov
import oracle
from conftest import ROOT


def declared_functions():
    names = set()
    for header in ("omnivoice_mi355x.h", "omnivoice_codec_mi355x.h"):
        with open(os.path.join(ROOT, "include", header)) as f:
            text = f.read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(ov[gc]_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) >= 28
    lib = ctypes.CDLL(ov.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(ov.EXPORTS), set(names) ^ set(ov.EXPORTS)


def test_schedule_and_build_match_reference_fixture(golden_cases):
    for case in golden_cases["generate"]:
        assert ov.unmask_schedule(8 * case["target"], 32, 0.1) == case["schedule"]
        ids = np.array(case["input_ids"], dtype=np.int32)
        a = case["audio_start"]
        refc = case["reference_codes"]
        rf = 0 if refc is None else len(refc[0])
        built = ov.ConditionalInput.build(ids[0, :a], refc, rf, case["target"])
        np.testing.assert_array_equal(built.ids, ids)
        assert built.audio_start == a and built.length == ids.shape[1]


def test_schedule_matches_oracle_everywhere():
    for total in [1, 3, 64, 400, 2000, 3000, 8192]:
        for steps in [1, 7, 32]:
            for t_shift in [0.1, 0.3, 1.0]:
                assert (ov.unmask_schedule(total, steps, t_shift) ==
                        oracle.unmask_schedule(total, steps, t_shift))


@pytest.mark.parametrize("tensor,norm,jitter", [(1, False, 0.0), (3, False, 0.0),
                                                (100 + 16 * 27 + 6, False, 0.0),
                                                (4, True, 0.0), (109, True, 0.25)])
def test_synthetic_weights_match_oracle(tensor, norm, jitter):
    first, count = 12345, 70001
    mine = ov.synthetic_values(1234, tensor, first, count, norm, jitter)
    theirs = np.zeros(count, dtype=np.float32)
    oracle.lib().orc_synth_values(1234, tensor, first, count, int(norm), jitter,
                                  theirs.ctypes.data)
    np.testing.assert_array_equal(mine, theirs)


def test_bad_config_is_rejected_with_reference_prefix():
    cfg = ov.released_config()
    cfg["head_dim"] = 64
    with pytest.raises(ov.GeneratorError) as e:
        ov.Generator.synthetic(cfg)
    assert str(e.value) == "OmniVoice generator: head_dim must be 128"


def test_missing_checkpoint_directory_is_an_error():
    with pytest.raises(ov.GeneratorError) as e:
        ov.Generator.load(ov.released_config(), "/nonexistent")
    assert str(e.value).startswith("OmniVoice generator: ")


@pytest.mark.parametrize("root", [None, ""])
def test_empty_checkpoint_root_is_an_error(root, tmp_path, monkeypatch):
    """An empty model root names model.safetensors in the working directory,
    as the reference's Load joins model_root / "model.safetensors"
    (generator.cpp:371-374): with no such file every loader fails with its
    prefix instead of building synthetic weights."""
    monkeypatch.chdir(tmp_path)
    with pytest.raises(ov.GeneratorError,
                       match="^OmniVoice generator: cannot open model.safetensors"):
        ov.Generator.load(ov.released_config(), root)
    with pytest.raises(ov.GeneratorError,
                       match="^OmniVoice audio tokenizer: cannot open "
                             "audio_tokenizer/model.safetensors"):
        ov.Codec.load(ov.codec_released_config(), root)
    with pytest.raises(ov.GeneratorError,
                       match="^OmniVoice audio tokenizer: cannot open "
                             "audio_tokenizer/model.safetensors"):
        ov.Encoder.load(ov.encoder_released_config(), root)


def test_build_input_rejects_bad_arguments():
    ids = np.zeros(8, dtype=np.int32)
    assert ov.lib().ovg_build_input(None, -1, None, 0, 1, 8, 1024,
                                    ids.ctypes.data) == -1


def test_codec_config_and_file_errors_before_the_gpu():
    """Configuration and checkpoint errors are reported with the reference's
    prefix before any device work (codec.cpp:143-145)."""
    cfg = ov.codec_released_config()
    with pytest.raises(ov.GeneratorError,
                       match="^OmniVoice audio tokenizer: config: 1 to 8 upsampling blocks"):
        ov.Codec.load(dict(cfg, ratios=[]))
    with pytest.raises(ov.GeneratorError, match="can't be halved"):
        ov.Codec.load(dict(cfg, channels=1000))
    with pytest.raises(ov.GeneratorError,
                       match="^OmniVoice audio tokenizer: .*audio_tokenizer/model.safetensors"):
        ov.Codec.load(cfg, "/nonexistent")


def test_encoder_config_and_file_errors_before_the_gpu():
    """The encoder's configuration and checkpoint errors carry the reference's
    prefix and come before any device work (codec_encoder.cpp:74-240)."""
    cfg = ov.encoder_released_config()
    prefix = "^OmniVoice audio tokenizer: "
    with pytest.raises(ov.GeneratorError, match=prefix + "ratios must multiply to frame_samples"):
        ov.Encoder.load(dict(cfg, ratios=[8, 5, 4, 2, 2]))
    with pytest.raises(ov.GeneratorError, match=prefix + "width must split into heads"):
        ov.Encoder.load(dict(cfg, heads=7))
    with pytest.raises(ov.GeneratorError, match=prefix + "width must split into positional"):
        ov.Encoder.load(dict(cfg, pos_groups=7))
    with pytest.raises(ov.GeneratorError, match=prefix + "HuBERT widths above 1024"):
        ov.Encoder.load(dict(cfg, width=1536, heads=12, pos_groups=16))
    with pytest.raises(ov.GeneratorError, match=prefix + "1 to 8 feature convolutions"):
        ov.Encoder.load(dict(cfg, conv_dim=[], conv_kernel=[], conv_stride=[]))
    with pytest.raises(ov.GeneratorError, match=prefix + ".*audio_tokenizer/model.safetensors"):
        ov.Encoder.load(cfg, "/nonexistent")
