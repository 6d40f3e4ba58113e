"""ORACLE — test infrastructure, not product code.

ctypes bindings of the CPU restatement (liboracle.so, built by
oracle/Makefile) and of the reference's own decoding.cpp compiled into
oracle/_ref/. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this package, to check the product's results or as
the timed CPU baseline; the product package never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_decoding.so")

_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_ptr = ctypes.c_void_p


class OrcConfig(ctypes.Structure):
    _fields_ = [("vocab_size", _i64), ("hidden_size", _i64),
                ("intermediate_size", _i64), ("layers", _i64),
                ("heads", _i64), ("kv_heads", _i64), ("head_dim", _i64),
                ("max_positions", _i64), ("rms_norm_eps", _f32),
                ("rope_theta", _f32), ("audio_codebooks", _i64),
                ("audio_vocab_size", _i64), ("audio_mask_id", _u32)]


class OrcCodecConfig(ctypes.Structure):
    _fields_ = [("codebooks", _i64), ("codebook_size", _i64),
                ("codebook_dim", _i64), ("hidden", _i64), ("latent", _i64),
                ("channels", _i64), ("blocks", _i64), ("ratios", _i64 * 8)]


class OrcEncoderConfig(ctypes.Structure):
    _fields_ = [("sample_rate", _i64), ("semantic_rate", _i64), ("frame_samples", _i64),
                ("semantic_stride", _i64), ("feat_layers", _i64), ("conv_dim", _i64 * 8),
                ("conv_kernel", _i64 * 8), ("conv_stride", _i64 * 8), ("width", _i64),
                ("intermediate", _i64), ("heads", _i64), ("layers", _i64),
                ("pos_kernel", _i64), ("pos_groups", _i64), ("eps", _f32),
                ("enc_channels", _i64), ("latent", _i64), ("blocks", _i64),
                ("ratios", _i64 * 8), ("codebooks", _i64), ("codebook_size", _i64),
                ("codebook_dim", _i64)]


def build(reference: bool = True) -> None:
    """Compiles liboracle.so and, when the reference tree is present,
    _ref/libref_decoding.so."""
    subprocess.run(["make", "-B", "-C", HERE, "-j8", "all"], check=True,
                   stdout=subprocess.DEVNULL)
    if reference and os.path.isdir("/root/reference"):
        subprocess.run(["make", "-B", "-C", HERE, "ref"], check=True,
                       stdout=subprocess.DEVNULL)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built (run make -C oracle)")
    L = ctypes.CDLL(LIB_PATH)
    sig = {
        "orc_unmask_schedule": (None, [_i64, _i64, _f32, _ptr]),
        "orc_build_input": (_i64, [_ptr, _i64, _ptr, _i64, _i64, _i64, _u32, _ptr]),
        "orc_exp": (_f32, [_f32]),
        "orc_log": (_f32, [_f32]),
        "orc_score": (None, [_ptr, _i64, _i64, _i64, _u32, _f32, _ptr, _ptr]),
        "orc_selector_create": (_ptr, [_f32, _f32, _u64]),
        "orc_selector_destroy": (None, [_ptr]),
        "orc_selector_fill": (_i64, [_ptr, _i64, _i64, _i64, _ptr, _ptr, _u32, _ptr, _ptr]),
        "orc_selector_noise": (None, [_ptr, _i64, _ptr]),
        "orc_mt19937_64_nth": (_u64, [_u64, _i64]),
        "orc_generate_from_logits": (_i64, [_ptr, _i64, _i64, _i64, _i64, _u32, _i64,
                                            _f32, _f32, _f32, _f32, _u64, _ptr, _ptr]),
        "orc_synth_normal": (ctypes.c_double, [_u64, _u64, _u64]),
        "orc_round_half": (_f32, [_f32]),
        "orc_synth_values": (None, [_u64, _u64, _u64, _i64, ctypes.c_int, _f32, _ptr]),
        "orc_model_synthetic": (_ptr, [ctypes.POINTER(OrcConfig), _u64, _f32]),
        "orc_model_from_host": (_ptr, [ctypes.POINTER(OrcConfig), _ptr, _ptr, _ptr, _ptr, _ptr]),
        "orc_model_destroy": (None, [_ptr]),
        "orc_set_threads": (None, [ctypes.c_int]),
        "orc_forward": (None, [_ptr, _ptr, _i64, _i64, _i64, ctypes.c_int, _ptr]),
        "orc_generate": (None, [_ptr, _ptr, _i64, _i64, _i64, ctypes.c_int, _i64, _f32,
                                _f32, _f32, _f32, _u64, _ptr, _ptr]),
        "orc_rmsnorm": (None, [_ptr, _ptr, _ptr, _i64, _i64, _f32]),
        "orc_linear": (None, [_ptr, _ptr, _ptr, _i64, _i64, _i64, ctypes.c_int]),
        "orc_qk_norm_rope": (None, [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64,
                                    _f32, _f32]),
        "orc_attention": (None, [_ptr, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, ctypes.c_int]),
        "orc_swiglu": (None, [_ptr, _ptr, _i64, _i64]),
        "orc_snake": (None, [_ptr, _i64, _i64, _ptr, _ptr]),
        "orc_conv1d": (None, [_ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _i64, _ptr]),
        "orc_conv_transpose1d": (None, [_ptr, _i64, _i64, _ptr, _ptr, _i64, _i64, _ptr]),
        "orc_codec_values": (None, [_u64, _u64, _u64, _i64, ctypes.c_double, ctypes.c_int,
                                    _ptr]),
        "orc_codec_synthetic": (_ptr, [ctypes.POINTER(OrcCodecConfig), _u64]),
        "orc_codec_destroy": (None, [_ptr]),
        "orc_codec_decode": (_i64, [_ptr, _ptr, _i64, _ptr]),
        "orc_resample": (_i64, [_ptr, _i64, _u32, _u32, _ptr]),
        "orc_encoder_synthetic": (_ptr, [ctypes.POINTER(OrcEncoderConfig), _u64]),
        "orc_encoder_destroy": (None, [_ptr]),
        "orc_encoder_encode": (_i64, [_ptr, _ptr, _i64, _ptr, _ptr, _ptr, _ptr]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


_ref: Optional[ctypes.CDLL] = None


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> ctypes.CDLL:
    """The reference's decoding.cpp (oracle/_ref)."""
    global _ref
    if _ref is not None:
        return _ref
    R = ctypes.CDLL(REF_PATH)
    R.ref_unmask_schedule.argtypes = [_i64, _i64, _f32, _ptr]
    R.ref_unmask_schedule.restype = None
    R.ref_build_input.argtypes = [_ptr, _i64, _ptr, _i64, _i64, _i64, _u32, _ptr]
    R.ref_build_input.restype = _i64
    R.ref_selector_create.argtypes = [_f32, _f32, _u64]
    R.ref_selector_create.restype = _ptr
    R.ref_selector_destroy.argtypes = [_ptr]
    R.ref_selector_destroy.restype = None
    R.ref_selector_fill.argtypes = [_ptr, _i64, _i64, _i64, _ptr, _ptr, _u32, _ptr, _ptr]
    R.ref_selector_fill.restype = _i64
    _ref = R
    return R


# ---------------------------------------------------------------- wrappers

def unmask_schedule(total: int, steps: int, t_shift: float) -> list:
    out = np.zeros(steps, dtype=np.int64)
    lib().orc_unmask_schedule(total, steps, t_shift, _p(out))
    return out.tolist()


def build_input(text_ids, reference_codes, reference_frames, target_frames,
                codebooks=8, mask_id=1024) -> np.ndarray:
    text = np.ascontiguousarray(text_ids, dtype=np.uint32)
    refc = (np.ascontiguousarray(reference_codes, dtype=np.int32)
            if reference_frames else np.zeros(1, dtype=np.int32))
    length = len(text) + reference_frames + target_frames
    ids = np.zeros(codebooks * length, dtype=np.int32)
    lib().orc_build_input(_p(text), len(text), _p(refc), reference_frames,
                          target_frames, codebooks, mask_id, _p(ids))
    return ids.reshape(codebooks, length)


def score(logits: np.ndarray, frames: int, codebooks: int, vocab: int,
          mask_id: int, guidance: float):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    pred = np.zeros(codebooks * frames, dtype=np.int32)
    conf = np.zeros(codebooks * frames, dtype=np.float32)
    lib().orc_score(_p(logits), frames, codebooks, vocab, mask_id, guidance,
                    _p(pred), _p(conf))
    return pred.reshape(codebooks, frames), conf.reshape(codebooks, frames)


class Selector:
    """PositionSelector (decoding.cpp:64-107) restated; `use_ref` runs the
    reference's own compiled decoding.cpp instead."""

    def __init__(self, layer_penalty: float, temperature: float, seed: int,
                 use_ref: bool = False):
        self._L = ref() if use_ref else lib()
        self._pre = "ref_" if use_ref else "orc_"
        self._h = getattr(self._L, self._pre + "selector_create")(
            layer_penalty, temperature, seed)

    def fill(self, count, codebooks, frames, prediction, confidence, mask_id,
             codes: np.ndarray):
        pred = np.ascontiguousarray(prediction, dtype=np.int32).ravel()
        conf = np.ascontiguousarray(confidence, dtype=np.float32).ravel()
        assert codes.dtype == np.int32 and codes.flags.c_contiguous
        chosen = np.zeros(codebooks * frames, dtype=np.int64)
        n = getattr(self._L, self._pre + "selector_fill")(
            self._h, count, codebooks, frames, _p(pred), _p(conf), mask_id,
            _p(codes), _p(chosen))
        return chosen[:n].tolist()

    def noise(self, total: int) -> np.ndarray:
        assert self._pre == "orc_"
        out = np.zeros(total, dtype=np.float32)
        lib().orc_selector_noise(self._h, total, _p(out))
        return out

    def __del__(self):
        try:
            getattr(self._L, self._pre + "selector_destroy")(self._h)
        except Exception:
            pass


def config_struct(cfg: dict) -> OrcConfig:
    return OrcConfig(**{k: cfg[k] for k, _ in OrcConfig._fields_})


class Model:
    """The CPU model: synthetic (seeded) or from host float32 tensors."""

    def __init__(self, cfg: dict, seed: int = 1234, norm_jitter: float = 0.0,
                 host: Optional[dict] = None):
        self.cfg = dict(cfg)
        self._c = config_struct(cfg)
        if host is None:
            self._h = lib().orc_model_synthetic(ctypes.byref(self._c), seed,
                                                norm_jitter)
        else:
            self._keep = host
            layers = host["layers"]
            ptrs = (ctypes.c_void_p * (len(layers) * 11))()
            for l, tensors in enumerate(layers):
                for k in range(11):
                    ptrs[l * 11 + k] = _p(tensors[k])
            self._ptrs = ptrs
            self._h = lib().orc_model_from_host(
                ctypes.byref(self._c), _p(host["text"]),
                _p(host["audio_embeddings"]), _p(host["audio_heads"]),
                _p(host["final_norm"]), ctypes.cast(ptrs, ctypes.c_void_p))

    def forward(self, ids: np.ndarray, audio_start: int, target_frames: int,
                emulate: bool = False) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        C, length = ids.shape
        V = self.cfg["audio_vocab_size"]
        out = np.zeros((2 * target_frames, C * V), dtype=np.float32)
        lib().orc_forward(self._h, _p(ids), length, audio_start, target_frames,
                          int(emulate), _p(out))
        return out

    def generate(self, ids, audio_start, target_frames, steps=32,
                 guidance=2.0, t_shift=0.1, layer_penalty=5.0,
                 temperature=0.0, seed=0, emulate=False):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        C, length = ids.shape
        codes = np.zeros(C * target_frames, dtype=np.int32)
        at = np.zeros(C * target_frames, dtype=np.int32)
        lib().orc_generate(self._h, _p(ids), length, audio_start,
                           target_frames, int(emulate), steps, guidance,
                           t_shift, layer_penalty, temperature, seed,
                           _p(codes), _p(at))
        return codes.reshape(C, target_frames), at.reshape(C, target_frames)

    def __del__(self):
        try:
            lib().orc_model_destroy(self._h)
        except Exception:
            pass


def generate_from_logits(logits_trace: np.ndarray, codebooks, frames, vocab,
                         mask_id, steps=32, guidance=2.0, t_shift=0.1,
                         layer_penalty=5.0, temperature=0.0, seed=0):
    trace = np.ascontiguousarray(logits_trace, dtype=np.float32)
    executed = trace.shape[0]
    codes = np.zeros(codebooks * frames, dtype=np.int32)
    at = np.zeros(codebooks * frames, dtype=np.int32)
    n = lib().orc_generate_from_logits(
        _p(trace), executed, codebooks, frames, vocab, mask_id, steps,
        guidance, t_shift, layer_penalty, temperature, seed, _p(codes), _p(at))
    if n < 0:
        raise ValueError("logits trace shorter than the executed steps")
    return codes.reshape(codebooks, frames), at.reshape(codebooks, frames)


def released_config(vocab_size: int = 151936) -> dict:
    """Dimensions of the released checkpoint (tests/config_samples.hpp:15-31
    of the reference), with the benchmark's text vocabulary."""
    return dict(vocab_size=vocab_size, hidden_size=1024, intermediate_size=3072,
                layers=28, heads=16, kv_heads=8, head_dim=128,
                max_positions=40960, rms_norm_eps=1e-6, rope_theta=1e6,
                audio_codebooks=8, audio_vocab_size=1025, audio_mask_id=1024)


# ------------------------------------------------------------------ codec

def codec_released_config() -> dict:
    """The audio tokenizer's decoder dimensions (tests/config_samples.hpp:34-70
    of the reference): 8 codebooks of 1024 x 64, RVQ output 768 + 256, fc2 to
    256 latent channels, 1024 decoder channels, upsampling 8, 5, 4, 2, 3
    (960 samples per frame)."""
    return dict(codebooks=8, codebook_size=1024, codebook_dim=64, hidden=1024,
                latent=256, channels=1024, ratios=[8, 5, 4, 2, 3])


def codec_config_struct(cfg: dict) -> OrcCodecConfig:
    ratios = (_i64 * 8)(*cfg["ratios"])
    return OrcCodecConfig(cfg["codebooks"], cfg["codebook_size"],
                          cfg["codebook_dim"], cfg["hidden"], cfg["latent"],
                          cfg["channels"], len(cfg["ratios"]), ratios)


def snake(x: np.ndarray, alpha: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    alpha = np.ascontiguousarray(alpha, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_snake(_p(x), x.shape[0], x.shape[1], _p(alpha), _p(y))
    return y


def conv1d(x, w, b, dilation=1) -> np.ndarray:
    """x [in][L], w [out][in][k]: nn.Conv1d, 'same' padding."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out, cin, k = w.shape
    y = np.empty((out, x.shape[1]), dtype=np.float32)
    lib().orc_conv1d(_p(x), cin, x.shape[1], _p(w), _p(b), out, k, dilation, _p(y))
    return y


def conv_transpose1d(x, w, b, stride) -> np.ndarray:
    """x [in][L], w [in][out][2 stride]: the decoder's upsampling layer."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    cin, out, _ = w.shape
    y = np.empty((out, x.shape[1] * stride), dtype=np.float32)
    lib().orc_conv_transpose1d(_p(x), cin, x.shape[1], _p(w), _p(b), out, stride,
                               _p(y))
    return y


def codec_values(seed, tensor, count, scale, exponential=False, first=0):
    out = np.empty(count, dtype=np.float32)
    lib().orc_codec_values(seed, tensor, first, count, scale, int(exponential),
                           _p(out))
    return out


class Codec:
    """The CPU audio decoder with synthetic (seeded) weights."""

    def __init__(self, cfg: dict, seed: int = 1234):
        self.cfg = dict(cfg)
        self._c = codec_config_struct(cfg)
        self._h = lib().orc_codec_synthetic(ctypes.byref(self._c), seed)

    def decode(self, codes: np.ndarray) -> np.ndarray:
        codes = np.ascontiguousarray(codes, dtype=np.int32)
        frames = codes.shape[1]
        audio = np.empty(frames * int(np.prod(self.cfg["ratios"])), dtype=np.float32)
        n = lib().orc_codec_decode(self._h, _p(codes), frames, _p(audio))
        assert n == audio.size
        return audio

    def __del__(self):
        try:
            lib().orc_codec_destroy(self._h)
        except Exception:
            pass


# ------------------------------------------------------------------ encoder

def encoder_released_config() -> dict:
    """The released audio tokenizer's encoder (tests/config_samples.hpp:34-70
    of the reference): HuBERT base at 16 kHz (7 feature convolutions of 512
    channels, 12 layers of 768 x 3072, 12 heads, positional convolution 128
    taps in 16 groups), semantic stride 2, DAC encoder 64 channels doubling
    over strides 8 5 4 2 3 to latent 256, 8 codebooks of 1024 x 64."""
    return dict(sample_rate=24000, semantic_rate=16000, frame_samples=960, semantic_stride=2,
                conv_dim=[512] * 7, conv_kernel=[10, 3, 3, 3, 3, 2, 2],
                conv_stride=[5, 2, 2, 2, 2, 2, 2], width=768, intermediate=3072, heads=12,
                layers=12, pos_kernel=128, pos_groups=16, eps=1e-5, enc_channels=64,
                latent=256, ratios=[8, 5, 4, 2, 3], codebooks=8, codebook_size=1024,
                codebook_dim=64)


def encoder_tiny_config() -> dict:
    """A small encoder of the same structure: 24 samples per frame (ratios
    2 3 4), HuBERT strides 2 2 2 at 16 kHz (two steps per frame)."""
    return dict(sample_rate=24000, semantic_rate=16000, frame_samples=24, semantic_stride=2,
                conv_dim=[16, 16, 16], conv_kernel=[4, 3, 2], conv_stride=[2, 2, 2], width=32,
                intermediate=48, heads=4, layers=2, pos_kernel=8, pos_groups=4, eps=1e-5,
                enc_channels=4, latent=12, ratios=[2, 3, 4], codebooks=3, codebook_size=16,
                codebook_dim=8)


def encoder_config_struct(cfg: dict) -> OrcEncoderConfig:
    def arr(v):
        return (_i64 * 8)(*v)
    return OrcEncoderConfig(cfg["sample_rate"], cfg["semantic_rate"], cfg["frame_samples"],
                            cfg["semantic_stride"], len(cfg["conv_dim"]), arr(cfg["conv_dim"]),
                            arr(cfg["conv_kernel"]), arr(cfg["conv_stride"]), cfg["width"],
                            cfg["intermediate"], cfg["heads"], cfg["layers"], cfg["pos_kernel"],
                            cfg["pos_groups"], cfg["eps"], cfg["enc_channels"], cfg["latent"],
                            len(cfg["ratios"]), arr(cfg["ratios"]), cfg["codebooks"],
                            cfg["codebook_size"], cfg["codebook_dim"])


def resample(samples, from_rate: int, to_rate: int) -> np.ndarray:
    x = np.ascontiguousarray(samples, dtype=np.float32)
    out = np.empty(int(np.ceil(to_rate * len(x) / from_rate)) + 1, dtype=np.float32)
    n = lib().orc_resample(_p(x), len(x), from_rate, to_rate, _p(out))
    return out[:n]


class Encoder:
    """The CPU audio encoder with synthetic (seeded) weights."""

    def __init__(self, cfg: dict, seed: int = 1234):
        self.cfg = dict(cfg)
        self._c = encoder_config_struct(cfg)
        self._h = lib().orc_encoder_synthetic(ctypes.byref(self._c), seed)

    def encode(self, samples) -> dict:
        x = np.ascontiguousarray(samples, dtype=np.float32)
        c = self.cfg
        count = len(x) // c["frame_samples"]
        hidden = c["width"] + c["latent"]
        codes = np.zeros((c["codebooks"], count), dtype=np.int32)
        sem = np.zeros((count, c["width"]), dtype=np.float32)
        ac = np.zeros((count, c["latent"]), dtype=np.float32)
        emb = np.zeros((count, hidden), dtype=np.float32)
        n = lib().orc_encoder_encode(self._h, _p(x), len(x), _p(codes), _p(sem), _p(ac), _p(emb))
        if n < 0:
            raise ValueError(f"encode failed ({n})")
        return dict(codes=codes, semantic=sem, acoustic=ac, embeddings=emb)

    def __del__(self):
        try:
            lib().orc_encoder_destroy(self._h)
        except Exception:
            pass
