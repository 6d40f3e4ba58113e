"""Loading a checkpoint directory (model_root/model.safetensors) with the
reference's tensor names, float32 dtype and shapes (reference
generator.cpp:364-434). Format and naming errors are reported before the
GPU is touched, so those run on the CPU; the GPU test checks that a
checkpoint holding the synthetic model's values gives the synthetic model's
logits bit for bit."""
import os

import numpy as np
import pytest
from safetensors.numpy import save_file

import omnivoice_amd as ov
from conftest import tiny_config as small_config

LAYER_TENSORS = [  # (name, rows, columns or None, synthetic kind, is norm)
    ("self_attn.q_proj.weight", "q", "h", 0, False),
    ("self_attn.k_proj.weight", "kv", "h", 1, False),
    ("self_attn.v_proj.weight", "kv", "h", 2, False),
    ("self_attn.o_proj.weight", "h", "q", 3, False),
    ("mlp.gate_proj.weight", "i", "h", 4, False),
    ("mlp.up_proj.weight", "i", "h", 5, False),
    ("mlp.down_proj.weight", "h", "i", 6, False),
    ("input_layernorm.weight", "h", None, 7, True),
    ("post_attention_layernorm.weight", "h", None, 8, True),
    ("self_attn.q_norm.weight", "d", None, 9, True),
    ("self_attn.k_norm.weight", "d", None, 10, True),
]


def checkpoint_tensors(cfg, seed, jitter):
    """The synthetic model's values under the checkpoint's names."""
    dims = {"h": cfg["hidden_size"], "i": cfg["intermediate_size"],
            "q": cfg["heads"] * cfg["head_dim"], "kv": cfg["kv_heads"] * cfg["head_dim"],
            "d": cfg["head_dim"]}
    audio_rows = cfg["audio_codebooks"] * cfg["audio_vocab_size"]
    h = cfg["hidden_size"]

    def values(tensor, shape, norm=False):
        n = int(np.prod(shape))
        return ov.synthetic_values(seed, tensor, 0, n, norm, jitter).reshape(shape)

    out = {
        "llm.embed_tokens.weight": values(1, (cfg["vocab_size"], h)),
        "audio_embeddings.weight": values(2, (audio_rows, h)),
        "audio_heads.weight": values(3, (audio_rows, h)),
        "llm.norm.weight": values(4, (h,), True),
    }
    for layer in range(cfg["layers"]):
        for name, rows, cols, kind, norm in LAYER_TENSORS:
            shape = (dims[rows], dims[cols]) if cols else (dims[rows],)
            out[f"llm.layers.{layer}.{name}"] = values(100 + 16 * layer + kind, shape, norm)
    return out


@pytest.fixture
def tiny_config():
    return small_config()


def write(directory, tensors):
    os.makedirs(directory, exist_ok=True)
    save_file(tensors, os.path.join(directory, "model.safetensors"))


def load_error(cfg, directory):
    with pytest.raises(ov.GeneratorError) as e:
        ov.Generator.load(cfg, str(directory))
    message = str(e.value)
    assert message.startswith("OmniVoice generator: "), message
    return message


def test_missing_checkpoint_is_reported(tiny_config, tmp_path):
    message = load_error(tiny_config, tmp_path / "absent")
    assert "model.safetensors" in message


def test_missing_tensor_is_reported(tiny_config, tmp_path):
    tensors = checkpoint_tensors(tiny_config, 3, 0.0)
    del tensors["llm.norm.weight"]
    write(tmp_path, tensors)
    assert "model.safetensors lacks llm.norm.weight" in load_error(tiny_config, tmp_path)


def test_wrong_dtype_and_shape_are_reported(tiny_config, tmp_path):
    tensors = checkpoint_tensors(tiny_config, 3, 0.0)
    name = "llm.layers.1.self_attn.k_norm.weight"
    tensors[name] = tensors[name].astype(np.float16)
    write(tmp_path / "dtype", tensors)
    assert f"{name} is F16 [128], expected F32 [128]" in load_error(tiny_config, tmp_path / "dtype")
    tensors[name] = np.ones(64, dtype=np.float32)
    write(tmp_path / "shape", tensors)
    assert f"{name} is F32 [64], expected F32 [128]" in load_error(tiny_config, tmp_path / "shape")


def test_corrupt_files_are_reported(tiny_config, tmp_path):
    write(tmp_path, {"llm.norm.weight": np.ones(256, dtype=np.float32)})
    path = tmp_path / "model.safetensors"
    data = path.read_bytes()
    path.write_bytes(data[:20])
    assert "header" in load_error(tiny_config, tmp_path)
    path.write_bytes((10 ** 12).to_bytes(8, "little") + data[8:])
    assert "implausible header length" in load_error(tiny_config, tmp_path)


@pytest.mark.gpu
def test_checkpoint_matches_synthetic_model(tiny_config, tmp_path):
    write(tmp_path, checkpoint_tensors(tiny_config, 11, 0.1))
    loaded = ov.Generator.load(tiny_config, str(tmp_path))
    synthetic = ov.Generator.synthetic(tiny_config, 11, 0.1)
    rng = np.random.default_rng(4)
    x = ov.ConditionalInput.build(rng.integers(0, tiny_config["vocab_size"], size=9),
                                  None, 0, 30)
    a, b = loaded.forward(x), synthetic.forward(x)
    assert a.tobytes() == b.tobytes()
    r1 = loaded.generate(x, ov.DecodingConfig(), 7)
    r2 = synthetic.generate(x, ov.DecodingConfig(), 7)
    assert (r1.codes == r2.codes).all() and (r1.unmasked_at == r2.unmasked_at).all()


def random_checkpoint(cfg, seed):
    """Float32 tensors under the checkpoint's names whose values are not
    fp16-exact (N(0, 0.02) matrices and embeddings, norms around 1)."""
    rng = np.random.default_rng(seed)
    dims = {"h": cfg["hidden_size"], "i": cfg["intermediate_size"],
            "q": cfg["heads"] * cfg["head_dim"], "kv": cfg["kv_heads"] * cfg["head_dim"],
            "d": cfg["head_dim"]}
    audio_rows = cfg["audio_codebooks"] * cfg["audio_vocab_size"]
    h = cfg["hidden_size"]

    def draw(shape, norm=False):
        x = 1.0 + 0.1 * rng.standard_normal(shape) if norm else 0.02 * rng.standard_normal(shape)
        return x.astype(np.float32)

    out = {"llm.embed_tokens.weight": draw((cfg["vocab_size"], h)),
           "audio_embeddings.weight": draw((audio_rows, h)),
           "audio_heads.weight": draw((audio_rows, h)),
           "llm.norm.weight": draw((h,), True)}
    for layer in range(cfg["layers"]):
        for name, rows, cols, _, norm in LAYER_TENSORS:
            shape = (dims[rows], dims[cols]) if cols else (dims[rows],)
            out[f"llm.layers.{layer}.{name}"] = draw(shape, norm)
    return out


def oracle_host(cfg, tensors):
    """The same tensors in the oracle's host layout (the reference's Load
    order, generator.cpp:377-425)."""
    return {"text": tensors["llm.embed_tokens.weight"],
            "audio_embeddings": tensors["audio_embeddings.weight"],
            "audio_heads": tensors["audio_heads.weight"],
            "final_norm": tensors["llm.norm.weight"],
            "layers": [[tensors[f"llm.layers.{layer}.{name}"] for name, *_ in LAYER_TENSORS]
                       for layer in range(cfg["layers"])]}


@pytest.mark.gpu
def test_checkpoint_of_arbitrary_values_matches_oracle(tiny_config, tmp_path):
    """A checkpoint of float32 values that fp16 cannot hold exactly: the
    matrices are rounded to fp16 on the GPU while being packed, as the
    reference's ConvertToHalf rounds them on the host (generator.cpp:31-49,
    364-434), so the loaded model's logits are within the parity bound of the
    float32 oracle built from the same tensors (which rounds its matrices the
    same way), and identical to the same tensors given through the host
    entry point."""
    import oracle
    tensors = random_checkpoint(tiny_config, 5)
    assert any((t != t.astype(np.float16).astype(np.float32)).any()
               for t in tensors.values())
    write(tmp_path, tensors)
    loaded = ov.Generator.load(tiny_config, str(tmp_path))
    host = oracle_host(tiny_config, tensors)
    model = oracle.Model(tiny_config, host=host)
    from_host = ov.Generator.from_host(tiny_config, host)
    rng = np.random.default_rng(9)
    for text, target in [(9, 30), (23, 61)]:
        x = ov.ConditionalInput.build(rng.integers(0, tiny_config["vocab_size"], size=text),
                                      None, 0, target)
        got = loaded.forward(x)
        want = model.forward(x.ids, text, target)
        rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
        print(f"({text}, {target}): max-abs {np.abs(got - want).max():.3e} rel-l2 {rel:.3e}")
        assert np.abs(got - want).max() < 2e-2
        assert rel < 1e-3
        assert got.tobytes() == from_host.forward(x).tobytes()
    loaded.close()
    from_host.close()
