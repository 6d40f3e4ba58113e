"""MI355X (gfx950) OmniVoice unmasking generator.

Python bindings of the C ABI in include/omnivoice_mi355x.h (ctypes over
libomnivoice_mi355x.so, built in-tree by omnivoice_amd/csrc/Makefile). The
names mirror the reference's C++ surface (generator.hpp / decoding.hpp of
gufo-extensions/omnivoice): DecodingConfig, ConditionalInput.build,
unmask_schedule, Generator.forward / score / generate.

Every call runs the HIP kernels; there is no CPU fallback. If the library is
not built, or no GPU is visible, the calls raise.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libomnivoice_mi355x.so")
CSRC = os.path.join(HERE, "csrc")

OVG_OK, OVG_ERROR, OVG_CANCELLED = 0, 1, 2

_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_ptr = ctypes.c_void_p
_err = ctypes.c_char_p
_sz = ctypes.c_size_t


class GeneratorError(RuntimeError):
    pass


class Cancelled(GeneratorError):
    pass


class _Config(ctypes.Structure):
    _fields_ = [("vocab_size", _i64), ("hidden_size", _i64),
                ("intermediate_size", _i64), ("layers", _i64),
                ("heads", _i64), ("kv_heads", _i64), ("head_dim", _i64),
                ("max_positions", _i64), ("rms_norm_eps", _f32),
                ("rope_theta", _f32), ("audio_codebooks", _i64),
                ("audio_vocab_size", _i64), ("audio_mask_id", _u32)]


class _Input(ctypes.Structure):
    _fields_ = [("codebooks", _i64), ("length", _i64), ("audio_start", _i64),
                ("target_frames", _i64), ("ids", _ptr)]


class _Decoding(ctypes.Structure):
    _fields_ = [("steps", _i64), ("guidance", _f32), ("t_shift", _f32),
                ("layer_penalty", _f32), ("position_temperature", _f32)]


class _HostWeights(ctypes.Structure):
    _fields_ = [("text_embeddings", _ptr), ("audio_embeddings", _ptr),
                ("audio_heads", _ptr), ("final_norm", _ptr), ("layers", _ptr)]


class _KernelStat(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("launches", _i64),
                ("total_ms", ctypes.c_double), ("flops", ctypes.c_double),
                ("bytes", ctypes.c_double)]


class _CodecConfig(ctypes.Structure):
    _fields_ = [("codebooks", _i64), ("codebook_size", _i64), ("codebook_dim", _i64),
                ("hidden", _i64), ("latent", _i64), ("channels", _i64),
                ("blocks", _i64), ("ratios", _i64 * 8)]


class _EncoderConfig(ctypes.Structure):
    _fields_ = [("sample_rate", _i64), ("semantic_rate", _i64), ("frame_samples", _i64),
                ("semantic_stride", _i64), ("feature_layers", _i64), ("conv_dim", _i64 * 8),
                ("conv_kernel", _i64 * 8), ("conv_stride", _i64 * 8), ("width", _i64),
                ("intermediate", _i64), ("heads", _i64), ("layers", _i64),
                ("pos_kernel", _i64), ("pos_groups", _i64), ("eps", ctypes.c_double),
                ("enc_channels", _i64), ("latent", _i64), ("blocks", _i64),
                ("ratios", _i64 * 8), ("codebooks", _i64), ("codebook_size", _i64),
                ("codebook_dim", _i64)]


_CANCEL_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)

EXPORTS = {
    "ovg_create": (ctypes.c_int, [ctypes.POINTER(_Config), ctypes.c_char_p, _u64,
                                  ctypes.POINTER(_ptr), _err, _sz]),
    "ovg_create_synthetic": (ctypes.c_int, [ctypes.POINTER(_Config), _u64, _f32,
                                            ctypes.POINTER(_ptr), _err, _sz]),
    "ovg_create_from_host": (ctypes.c_int, [ctypes.POINTER(_Config),
                                            ctypes.POINTER(_HostWeights),
                                            ctypes.POINTER(_ptr), _err, _sz]),
    "ovg_destroy": (None, [_ptr]),
    "ovg_forward": (ctypes.c_int, [_ptr, ctypes.POINTER(_Input), _ptr, _err, _sz]),
    "ovg_score": (ctypes.c_int, [_ptr, ctypes.POINTER(_Input), _f32, _ptr, _ptr,
                                 _err, _sz]),
    "ovg_generate": (ctypes.c_int, [_ptr, ctypes.POINTER(_Input),
                                    ctypes.POINTER(_Decoding), _u64, _CANCEL_FN,
                                    _ptr, _ptr, _ptr, _err, _sz]),
    "ovg_generate_batch": (ctypes.c_int, [_ptr, _i64, _ptr, ctypes.POINTER(_Decoding),
                                          _ptr, _CANCEL_FN, _ptr, _ptr, _ptr, _err, _sz]),
    "ovg_generate_trace_batch": (ctypes.c_int, [_ptr, _i64, _ptr, ctypes.POINTER(_Decoding),
                                                _ptr, _ptr, _ptr, _ptr, _ptr, _err, _sz]),
    "ovg_generate_chunks": (ctypes.c_int, [_ptr, _i64, _ptr, _ptr, _ptr, _i64, _ptr,
                                           ctypes.POINTER(_Decoding), _u64, _CANCEL_FN, _ptr,
                                           _ptr, _ptr, _err, _sz]),
    "ovg_generate_trace": (ctypes.c_int, [_ptr, ctypes.POINTER(_Input),
                                          ctypes.POINTER(_Decoding), _u64, _ptr, _ptr,
                                          _ptr, ctypes.POINTER(_i64), _err, _sz]),
    "ovg_profile_step": (ctypes.c_int, [_ptr, ctypes.POINTER(_Input), _i64, _ptr, _i64,
                                        ctypes.POINTER(_i64), _err, _sz]),
    "ovg_profile_batch": (ctypes.c_int, [_ptr, _i64, ctypes.POINTER(_Input), _i64, _ptr,
                                         _i64, ctypes.POINTER(_i64), _err, _sz]),
    "ovg_device_bytes": (_i64, [_ptr]),
    "ovg_synthetic_values": (None, [_u64, _u64, _u64, _i64, ctypes.c_int, _f32, _ptr]),
    "ovg_unmask_schedule": (ctypes.c_int, [_i64, _i64, _f32, _ptr]),
    "ovg_build_input": (_i64, [_ptr, _i64, _ptr, _i64, _i64, _i64, _u32, _ptr]),
    "ovg_op_score": (ctypes.c_int, [_ptr, _ptr, _ptr, _i64, _i64, _i64, _u32, _f32,
                                    _ptr, _err, _sz]),
    "ovg_op_select": (ctypes.c_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64,
                                     ctypes.c_int32, _f32, _f32, _u32, _ptr, _err, _sz]),
    "ovg_op_linear": (ctypes.c_int, [_ptr, _ptr, _ptr, _i64, _i64, _i64, ctypes.c_int,
                                     _ptr, _err, _sz]),
    "ovg_op_linear_packed": (ctypes.c_int, [_ptr, _ptr, _ptr, _i64, _i64, _i64,
                                            ctypes.c_int, _i64, _i64, _ptr, _err, _sz]),
    "ovg_op_linear_noalloc": (ctypes.c_int, [_ptr, _ptr, _ptr, _i64, _i64, _i64,
                                             ctypes.c_int, _ptr, _err, _sz]),
    "ovg_op_rmsnorm": (ctypes.c_int, [_ptr, _ptr, _ptr, _i64, _i64, _f32, _ptr, _err,
                                      _sz]),
    "ovg_op_attention": (ctypes.c_int, [_ptr, _ptr, _i64, _i64, _i64, _ptr, _i64,
                                        _ptr, _err, _sz]),
    # the audio decoder (include/omnivoice_codec_mi355x.h)
    "ovc_create": (ctypes.c_int, [ctypes.POINTER(_CodecConfig), ctypes.c_char_p, _u64,
                                  ctypes.POINTER(_ptr), _err, _sz]),
    "ovc_create_synthetic": (ctypes.c_int, [ctypes.POINTER(_CodecConfig), _u64,
                                            ctypes.POINTER(_ptr), _err, _sz]),
    "ovc_destroy": (None, [_ptr]),
    "ovc_samples": (_i64, [_ptr, _i64]),
    "ovc_decode": (ctypes.c_int, [_ptr, _ptr, _i64, _ptr, _err, _sz]),
    "ovc_decode_device": (ctypes.c_int, [_ptr, _ptr, _i64, _ptr, _ptr, _err, _sz]),
    "ovc_profile_decode": (ctypes.c_int, [_ptr, _i64, _i64, _ptr, _i64,
                                          ctypes.POINTER(_i64), _err, _sz]),
    "ovc_synthetic_values": (None, [_u64, _u64, _u64, _i64, ctypes.c_double, ctypes.c_int,
                                    _ptr]),
    "ovc_op_conv1d": (ctypes.c_int, [_ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _i64,
                                     ctypes.c_int, _ptr, _ptr, _err, _sz]),
    "ovc_op_conv_transpose1d": (ctypes.c_int, [_ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64,
                                               _i64, _ptr, _ptr, _err, _sz]),
    # the audio encoder (include/omnivoice_codec_mi355x.h)
    "ovc_encoder_create": (ctypes.c_int, [ctypes.POINTER(_EncoderConfig), ctypes.c_char_p,
                                          _u64, ctypes.POINTER(_ptr), _err, _sz]),
    "ovc_encoder_create_synthetic": (ctypes.c_int, [ctypes.POINTER(_EncoderConfig), _u64,
                                                    ctypes.POINTER(_ptr), _err, _sz]),
    "ovc_encoder_destroy": (None, [_ptr]),
    "ovc_encoder_frames": (_i64, [_ptr, _i64]),
    "ovc_encode": (ctypes.c_int, [_ptr, _ptr, _i64, _ptr, _ptr, _ptr, _ptr, _err, _sz]),
    "ovc_encode_device": (ctypes.c_int, [_ptr, _ptr, _i64, _ptr, _ptr, _err, _sz]),
    "ovc_profile_encode": (ctypes.c_int, [_ptr, _i64, _i64, _ptr, _i64,
                                          ctypes.POINTER(_i64), _err, _sz]),
}

_lib: Optional[ctypes.CDLL] = None


def build(jobs: int = 8) -> None:
    """Compiles libomnivoice_mi355x.so for gfx950 (always recompiles)."""
    subprocess.run(["make", "-B", "-C", CSRC, f"-j{jobs}"], check=True,
                   stdout=subprocess.DEVNULL)


def lib() -> ctypes.CDLL:
    """The HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise GeneratorError(
            f"{LIB_PATH} is not built: run omnivoice_amd.build() or "
            f"make -C {CSRC}")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in EXPORTS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _buf() -> ctypes.Array:
    return ctypes.create_string_buffer(1024)


def _check(status: int, err) -> int:
    if status == OVG_OK:
        return status
    message = err.value.decode(errors="replace")
    if status == OVG_CANCELLED:
        raise Cancelled(message)
    raise GeneratorError(message)


# --------------------------------------------------------------- decoding.hpp

@dataclass
class DecodingConfig:
    """OmniVoiceGenerationConfig's decoding parameters (decoding.hpp:14-21)."""
    steps: int = 32
    guidance: float = 2.0
    t_shift: float = 0.1
    layer_penalty: float = 5.0
    position_temperature: float = 5.0

    def _c(self) -> _Decoding:
        return _Decoding(self.steps, self.guidance, self.t_shift,
                         self.layer_penalty, self.position_temperature)


def unmask_schedule(total: int, steps: int, t_shift: float) -> List[int]:
    """UnmaskSchedule (decoding.hpp:23-27)."""
    out = np.zeros(steps, dtype=np.int64)
    if lib().ovg_unmask_schedule(total, steps, t_shift, _p(out)) != OVG_OK:
        raise GeneratorError("bad schedule arguments")
    return out.tolist()


@dataclass
class ConditionalInput:
    """[text tokens | reference frames | target frames] x codebooks
    (decoding.hpp:32-47); ids is int32 [codebooks][length]."""
    codebooks: int
    length: int
    audio_start: int
    target_frames: int
    ids: np.ndarray

    @staticmethod
    def build(text_ids: Sequence[int], reference_codes: Optional[np.ndarray],
              reference_frames: int, target_frames: int, codebooks: int = 8,
              mask_id: int = 1024) -> "ConditionalInput":
        text = np.ascontiguousarray(text_ids, dtype=np.uint32)
        refc = (np.ascontiguousarray(reference_codes, dtype=np.int32)
                if reference_frames else np.zeros(1, dtype=np.int32))
        length = len(text) + reference_frames + target_frames
        ids = np.zeros(codebooks * length, dtype=np.int32)
        n = lib().ovg_build_input(_p(text), len(text), _p(refc),
                                  reference_frames, target_frames, codebooks,
                                  mask_id, _p(ids))
        if n != length:
            raise GeneratorError("bad input arguments")
        return ConditionalInput(codebooks, length, len(text), target_frames,
                                ids.reshape(codebooks, length))

    def _c(self) -> _Input:
        ids = np.ascontiguousarray(self.ids, dtype=np.int32)
        self._keep = ids
        return _Input(self.codebooks, self.length, self.audio_start,
                      self.target_frames, _p(ids))


@dataclass
class GenerationResult:
    """codes and unmasked_at, int32 [codebooks][frames] (decoding.hpp:49-54)."""
    codes: np.ndarray
    unmasked_at: np.ndarray
    executed_steps: int = 0
    logits_trace: Optional[np.ndarray] = field(default=None, repr=False)


def synthetic_values(seed: int, tensor: int, first: int, count: int,
                     norm: bool = False, jitter: float = 0.0) -> np.ndarray:
    """The synthetic model's values of one tensor's elements (host only)."""
    out = np.zeros(count, dtype=np.float32)
    lib().ovg_synthetic_values(seed, tensor, first, count, int(norm), jitter,
                               _p(out))
    return out


def released_config(vocab_size: int = 151936, layers: int = 28) -> dict:
    """The released checkpoint's dimensions (reference
    tests/config_samples.hpp:15-31); the synthetic benchmark model uses a
    151936-entry text vocabulary."""
    return dict(vocab_size=vocab_size, hidden_size=1024, intermediate_size=3072,
                layers=layers, heads=16, kv_heads=8, head_dim=128,
                max_positions=40960, rms_norm_eps=1e-6, rope_theta=1e6,
                audio_codebooks=8, audio_vocab_size=1025, audio_mask_id=1024)


def _config(cfg: dict) -> _Config:
    return _Config(**{k: cfg[k] for k, _ in _Config._fields_})


# --------------------------------------------------------------- generator.hpp

class Generator:
    """The bidirectional Qwen3 backbone with its audio embeddings and heads
    in HBM, and the unmasking loop on the GPU (generator.hpp:17-56). Not
    thread-safe."""

    def __init__(self, handle: int, cfg: dict, keep=None):
        self._h = handle
        self.cfg = dict(cfg)
        self._keep = keep

    @classmethod
    def synthetic(cls, cfg: dict, seed: int = 1234,
                  norm_jitter: float = 0.0) -> "Generator":
        c = _config(cfg)
        h = _ptr()
        err = _buf()
        _check(lib().ovg_create_synthetic(ctypes.byref(c), seed, norm_jitter,
                                          ctypes.byref(h), err, len(err)), err)
        return cls(h.value, cfg)

    @classmethod
    def load(cls, cfg: dict, model_root: Optional[str] = None) -> "Generator":
        """Generator::Load: model_root/model.safetensors (None or "" names
        the working directory, as the reference joins the path; a missing
        file is an error)."""
        c = _config(cfg)
        h = _ptr()
        err = _buf()
        root = (model_root or "").encode()
        _check(lib().ovg_create(ctypes.byref(c), root, 0, ctypes.byref(h),
                                err, len(err)), err)
        return cls(h.value, cfg)

    @classmethod
    def from_host(cls, cfg: dict, tensors: dict) -> "Generator":
        """tensors: text, audio_embeddings, audio_heads, final_norm (float32)
        and layers: [layers][11] float32 arrays in OVG_LAYER_* order."""
        keep = {k: np.ascontiguousarray(v, dtype=np.float32)
                for k, v in tensors.items() if k != "layers"}
        layers = [[np.ascontiguousarray(t, dtype=np.float32) for t in layer]
                  for layer in tensors["layers"]]
        ptrs = (_ptr * (len(layers) * 11))()
        for l, layer in enumerate(layers):
            for k in range(11):
                ptrs[l * 11 + k] = _p(layer[k])
        w = _HostWeights(_p(keep["text"]), _p(keep["audio_embeddings"]),
                         _p(keep["audio_heads"]), _p(keep["final_norm"]),
                         ctypes.cast(ptrs, _ptr).value)
        c = _config(cfg)
        h = _ptr()
        err = _buf()
        _check(lib().ovg_create_from_host(ctypes.byref(c), ctypes.byref(w),
                                          ctypes.byref(h), err, len(err)), err)
        return cls(h.value, cfg)

    def close(self) -> None:
        if self._h:
            lib().ovg_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def device_bytes(self) -> int:
        return int(lib().ovg_device_bytes(self._h))

    def _width(self) -> int:
        return self.cfg["audio_codebooks"] * self.cfg["audio_vocab_size"]

    def forward(self, inp: ConditionalInput) -> np.ndarray:
        """Generator::Forward: logits [2 F][codebooks * vocab], conditional
        target rows first."""
        out = np.zeros((2 * inp.target_frames, self._width()), dtype=np.float32)
        c = inp._c()
        err = _buf()
        _check(lib().ovg_forward(self._h, ctypes.byref(c), _p(out), err,
                                 len(err)), err)
        return out

    def score(self, inp: ConditionalInput, guidance: float = 2.0
              ) -> Tuple[np.ndarray, np.ndarray]:
        """Generator::Score: prediction int32 / confidence float32
        [codebooks][frames]."""
        n = inp.codebooks * inp.target_frames
        pred = np.zeros(n, dtype=np.int32)
        conf = np.zeros(n, dtype=np.float32)
        c = inp._c()
        err = _buf()
        _check(lib().ovg_score(self._h, ctypes.byref(c), guidance, _p(pred),
                               _p(conf), err, len(err)), err)
        shape = (inp.codebooks, inp.target_frames)
        return pred.reshape(shape), conf.reshape(shape)

    def generate(self, inp: ConditionalInput,
                 decoding: DecodingConfig = DecodingConfig(), seed: int = 0,
                 cancelled: Optional[Callable[[], bool]] = None
                 ) -> GenerationResult:
        """Generator::Generate: the whole unmasking loop on the GPU."""
        return self.generate_batch([inp], decoding, [seed], cancelled)[0]

    def generate_batch(self, inputs: Sequence[ConditionalInput],
                       decoding: DecodingConfig = DecodingConfig(),
                       seeds: Optional[Sequence[int]] = None,
                       cancelled: Optional[Callable[[], bool]] = None
                       ) -> List[GenerationResult]:
        n = len(inputs)
        seeds = list(seeds) if seeds is not None else list(range(n))
        cs = (_Input * n)(*[i._c() for i in inputs])
        seed_arr = (_u64 * n)(*seeds)
        codes = [np.zeros((i.codebooks, i.target_frames), dtype=np.int32)
                 for i in inputs]
        ats = [np.zeros_like(c) for c in codes]
        code_ptrs = (_ptr * n)(*[_p(c) for c in codes])
        at_ptrs = (_ptr * n)(*[_p(a) for a in ats])
        cb = _CANCEL_FN(lambda _user: int(bool(cancelled())) if cancelled else 0)
        d = decoding._c()
        err = _buf()
        _check(lib().ovg_generate_batch(
            self._h, n, ctypes.cast(cs, _ptr), ctypes.byref(d),
            ctypes.cast(seed_arr, _ptr), cb, None, ctypes.cast(code_ptrs, _ptr),
            ctypes.cast(at_ptrs, _ptr), err, len(err)), err)
        return [GenerationResult(c, a) for c, a in zip(codes, ats)]

    def generate_trace(self, inp: ConditionalInput,
                       decoding: DecodingConfig = DecodingConfig(),
                       seed: int = 0) -> GenerationResult:
        """generate, launched eagerly, also returning every executed step's
        logits [executed][2 F][codebooks * vocab]."""
        steps = sum(1 for s in unmask_schedule(
            inp.codebooks * inp.target_frames, decoding.steps,
            decoding.t_shift) if s > 0)
        trace = np.zeros((steps, 2 * inp.target_frames, self._width()),
                         dtype=np.float32)
        codes = np.zeros((inp.codebooks, inp.target_frames), dtype=np.int32)
        at = np.zeros_like(codes)
        executed = _i64()
        c = inp._c()
        d = decoding._c()
        err = _buf()
        _check(lib().ovg_generate_trace(self._h, ctypes.byref(c), ctypes.byref(d),
                                        seed, _p(codes), _p(at), _p(trace),
                                        ctypes.byref(executed), err, len(err)), err)
        return GenerationResult(codes, at, executed.value, trace)

    def generate_trace_batch(self, inputs: Sequence[ConditionalInput],
                             decoding: DecodingConfig = DecodingConfig(),
                             seeds: Optional[Sequence[int]] = None,
                             trace: Optional[Sequence[bool]] = None
                             ) -> List[GenerationResult]:
        """generate_batch launched eagerly, also returning each item's logits
        at every step it executes ([executed][2 F][codebooks * vocab]) for
        the items whose `trace` flag is set (all by default)."""
        n = len(inputs)
        seeds = list(seeds) if seeds is not None else list(range(n))
        trace = list(trace) if trace is not None else [True] * n
        cs = (_Input * n)(*[i._c() for i in inputs])
        seed_arr = (_u64 * n)(*seeds)
        codes = [np.zeros((i.codebooks, i.target_frames), dtype=np.int32) for i in inputs]
        ats = [np.zeros_like(c) for c in codes]
        traces = []
        for i, want in zip(inputs, trace):
            steps = sum(1 for s in unmask_schedule(i.codebooks * i.target_frames,
                                                   decoding.steps, decoding.t_shift) if s > 0)
            traces.append(np.zeros((steps, 2 * i.target_frames, self._width()),
                                   dtype=np.float32) if want else None)
        code_ptrs = (_ptr * n)(*[_p(c) for c in codes])
        at_ptrs = (_ptr * n)(*[_p(a) for a in ats])
        trace_ptrs = (_ptr * n)(*[_p(t) if t is not None else None for t in traces])
        executed = (_i64 * n)()
        d = decoding._c()
        err = _buf()
        _check(lib().ovg_generate_trace_batch(
            self._h, n, ctypes.cast(cs, _ptr), ctypes.byref(d), ctypes.cast(seed_arr, _ptr),
            ctypes.cast(code_ptrs, _ptr), ctypes.cast(at_ptrs, _ptr),
            ctypes.cast(trace_ptrs, _ptr), ctypes.cast(executed, _ptr), err, len(err)), err)
        return [GenerationResult(c, a, executed[k], t)
                for k, (c, a, t) in enumerate(zip(codes, ats, traces))]

    def generate_chunks(self, text_ids: Sequence[Sequence[int]],
                        target_frames: Sequence[int],
                        decoding: DecodingConfig = DecodingConfig(), seed: int = 0,
                        reference_codes=None,
                        cancelled: Optional[Callable[[], bool]] = None
                        ) -> List[GenerationResult]:
        """The reference's chunk loop (synthesizer.cpp:179-201): chunk i is
        ConditionalInput.build(text_ids[i], reference, target_frames[i]) with
        one seed; without reference codes, chunk 0 runs first and its codes
        are the reference of the rest, which run as one batch."""
        n = len(text_ids)
        texts = [np.ascontiguousarray(t, dtype=np.uint32) for t in text_ids]
        counts = (_i64 * n)(*[len(t) for t in texts])
        text_ptrs = (_ptr * n)(*[_p(t) if len(t) else None for t in texts])
        frames = (_i64 * n)(*[int(f) for f in target_frames])
        C = self.cfg["audio_codebooks"]
        ref = (np.ascontiguousarray(reference_codes, dtype=np.int32)
               if reference_codes is not None else None)
        ref_frames = ref.shape[1] if ref is not None else 0
        codes = [np.zeros((C, int(f)), dtype=np.int32) for f in target_frames]
        ats = [np.zeros_like(c) for c in codes]
        code_ptrs = (_ptr * n)(*[_p(c) for c in codes])
        at_ptrs = (_ptr * n)(*[_p(a) for a in ats])
        cb = _CANCEL_FN(lambda _user: int(bool(cancelled())) if cancelled else 0)
        d = decoding._c()
        err = _buf()
        _check(lib().ovg_generate_chunks(
            self._h, n, ctypes.cast(text_ptrs, _ptr), ctypes.cast(counts, _ptr),
            _p(ref) if ref is not None else None, ref_frames, ctypes.cast(frames, _ptr),
            ctypes.byref(d), seed, cb, None, ctypes.cast(code_ptrs, _ptr),
            ctypes.cast(at_ptrs, _ptr), err, len(err)), err)
        return [GenerationResult(c, a) for c, a in zip(codes, ats)]

    def profile(self, inp, repeats: int = 3) -> dict:
        """Per-kernel HIP-event timings of eager forward + score + select of
        one input, or of a list of inputs packed as one batch."""
        items = list(inp) if isinstance(inp, (list, tuple)) else [inp]
        cap = 64
        stats = (_KernelStat * cap)()
        count = _i64()
        cs = (_Input * len(items))(*[i._c() for i in items])
        err = _buf()
        _check(lib().ovg_profile_batch(self._h, len(items), cs, repeats,
                                       ctypes.cast(stats, _ptr), cap,
                                       ctypes.byref(count), err, len(err)), err)
        out = {}
        for i in range(min(count.value, cap)):
            s = stats[i]
            out[s.name.decode()] = dict(launches=s.launches, total_ms=s.total_ms,
                                        flops=s.flops, bytes=s.bytes)
        return out


# --------------------------------------------------------------- device ops

def _dev(t) -> int:
    """Device pointer of a torch tensor (torch is only plumbing here)."""
    return t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream


def op_score(logits, prediction, confidence, frames: int, codebooks: int,
             vocab: int, mask_id: int, guidance: float, stream=None) -> None:
    err = _buf()
    _check(lib().ovg_op_score(_dev(logits), _dev(prediction), _dev(confidence),
                              frames, codebooks, vocab, mask_id, guidance,
                              _stream(stream), err, len(err)), err)


def op_select(prediction, confidence, noise, codes, unmasked_at,
              codebooks: int, frames: int, count: int, step: int,
              layer_penalty: float, temperature: float, mask_id: int,
              stream=None) -> None:
    err = _buf()
    _check(lib().ovg_op_select(_dev(prediction), _dev(confidence),
                               _dev(noise) if noise is not None else None,
                               _dev(codes), _dev(unmasked_at), codebooks, frames,
                               count, step, layer_penalty, temperature, mask_id,
                               _stream(stream), err, len(err)), err)


def op_linear(x, w, y, accumulate: bool = False, stream=None) -> None:
    rows, k = x.shape
    n = w.shape[0]
    err = _buf()
    _check(lib().ovg_op_linear(_dev(x), _dev(w), _dev(y), rows, k, n,
                               int(accumulate), _stream(stream), err, len(err)), err)


def op_linear_packed(x, w, y, accumulate: bool = False, tile_rows: int = 0,
                     tile_cols: int = 0, stream=None) -> None:
    """op_linear through the generator's packed-weight kernel (tile forced
    when tile_rows and tile_cols are given)."""
    rows, k = x.shape
    n = w.shape[0]
    err = _buf()
    _check(lib().ovg_op_linear_packed(_dev(x), _dev(w), _dev(y), rows, k, n, int(accumulate),
                                      tile_rows, tile_cols, _stream(stream), err, len(err)),
           err)


def op_linear_noalloc(x, w, y, accumulate: bool = False, stream=None) -> None:
    """op_linear without device allocation (a static split-K scratch); returns
    without waiting for the stream."""
    rows, k = x.shape
    n = w.shape[0]
    err = _buf()
    _check(lib().ovg_op_linear_noalloc(_dev(x), _dev(w), _dev(y), rows, k, n,
                                       int(accumulate), _stream(stream), err, len(err)),
           err)


def op_rmsnorm(x, weight, out, eps: float, stream=None) -> None:
    rows, width = x.shape
    err = _buf()
    _check(lib().ovg_op_rmsnorm(_dev(x), _dev(weight), _dev(out), rows, width,
                                eps, _stream(stream), err, len(err)), err)


def op_attention(qkv, out, heads: int, kv_heads: int,
                 sequences: Sequence[Tuple[int, int]], stream=None) -> None:
    rows = qkv.shape[0]
    seq = np.ascontiguousarray(np.array(sequences, dtype=np.int64).ravel())
    err = _buf()
    _check(lib().ovg_op_attention(_dev(qkv), _dev(out), rows, heads, kv_heads,
                                  _p(seq), len(sequences), _stream(stream),
                                  err, len(err)), err)


# --------------------------------------------------------------- audio decoder

def codec_released_config() -> dict:
    """The released audio tokenizer's decoder (tests/config_samples.hpp:34-70
    of the reference): 8 codebooks of 1024 x 64, RVQ output 768 + 256, fc2 to
    256 latent channels, 1024 decoder channels, upsampling 8, 5, 4, 2, 3
    (960 samples per frame at 24 kHz)."""
    return dict(codebooks=8, codebook_size=1024, codebook_dim=64, hidden=1024,
                latent=256, channels=1024, ratios=[8, 5, 4, 2, 3])


def _codec_config(cfg: dict) -> _CodecConfig:
    ratios = list(cfg["ratios"])
    return _CodecConfig(cfg["codebooks"], cfg["codebook_size"], cfg["codebook_dim"],
                        cfg["hidden"], cfg["latent"], cfg["channels"], len(ratios),
                        (_i64 * 8)(*ratios))


def codec_synthetic_values(seed: int, tensor: int, first: int, count: int,
                           scale: float, exponential: bool = False) -> np.ndarray:
    out = np.zeros(count, dtype=np.float32)
    lib().ovc_synthetic_values(seed, tensor, first, count, scale, int(exponential),
                               _p(out))
    return out


class Codec:
    """The audio tokenizer's decoder on the GPU: codes [codebooks][frames] to
    24 kHz float32 audio (codec.hpp:16-45 of the reference, Decode). Not
    thread-safe."""

    def __init__(self, handle: int, cfg: dict):
        self._h = handle
        self.cfg = dict(cfg)

    @classmethod
    def load(cls, cfg: dict, model_root: Optional[str] = None) -> "Codec":
        """model_root/audio_tokenizer/model.safetensors (None or "" names the
        working directory, as the reference joins the path)."""
        c = _codec_config(cfg)
        h = _ptr()
        err = _buf()
        root = (model_root or "").encode()
        _check(lib().ovc_create(ctypes.byref(c), root, 0, ctypes.byref(h), err,
                                len(err)), err)
        return cls(h.value, cfg)

    @classmethod
    def synthetic(cls, cfg: dict, seed: int = 1234) -> "Codec":
        """The seeded synthetic decoder."""
        c = _codec_config(cfg)
        h = _ptr()
        err = _buf()
        _check(lib().ovc_create_synthetic(ctypes.byref(c), seed, ctypes.byref(h), err,
                                          len(err)), err)
        return cls(h.value, cfg)

    def samples(self, frames: int) -> int:
        return int(lib().ovc_samples(self._h, frames))

    def decode(self, codes) -> np.ndarray:
        codes = np.ascontiguousarray(codes, dtype=np.int32)
        frames = codes.shape[1]
        audio = np.zeros(self.samples(frames), dtype=np.float32)
        err = _buf()
        _check(lib().ovc_decode(self._h, _p(codes), frames, _p(audio), err, len(err)),
               err)
        return audio

    def decode_device(self, codes, audio, stream=None) -> None:
        """codes: int32 device tensor [codebooks][frames]; audio: float32
        device tensor of samples(frames). Enqueued on `stream`."""
        err = _buf()
        _check(lib().ovc_decode_device(self._h, _dev(codes), codes.shape[1], _dev(audio),
                                       _stream(stream), err, len(err)), err)

    def profile(self, frames: int, repeats: int = 3) -> dict:
        cap = 32
        stats = (_KernelStat * cap)()
        count = _i64()
        err = _buf()
        _check(lib().ovc_profile_decode(self._h, frames, repeats, ctypes.cast(stats, _ptr),
                                        cap, ctypes.byref(count), err, len(err)), err)
        out = {}
        for i in range(min(count.value, cap)):
            s = stats[i]
            out[s.name.decode()] = dict(launches=s.launches, total_ms=s.total_ms,
                                        flops=s.flops, bytes=s.bytes)
        return out

    def close(self) -> None:
        if self._h:
            lib().ovc_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def op_conv1d(x, w, b, y, alpha=None, dilation: int = 1, accumulate: bool = False,
              stream=None) -> None:
    """x [in][L], y [out][L], alpha [in]: float32 device tensors; w [out][in][k]
    and b [out]: host float32 arrays."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out, cin, k = w.shape
    err = _buf()
    _check(lib().ovc_op_conv1d(_dev(x), cin, x.shape[1],
                               _dev(alpha) if alpha is not None else None, _p(w), _p(b),
                               out, k, dilation, int(accumulate), _dev(y), _stream(stream),
                               err, len(err)), err)


def op_conv_transpose1d(x, w, b, y, stride: int, alpha=None, stream=None) -> None:
    """x [in][L], y [out][L stride], alpha [in]: float32 device tensors;
    w [in][out][2 stride] and b [out]: host float32 arrays."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    cin, out, _ = w.shape
    err = _buf()
    _check(lib().ovc_op_conv_transpose1d(_dev(x), cin, x.shape[1],
                                         _dev(alpha) if alpha is not None else None,
                                         _p(w), _p(b), out, stride, _dev(y),
                                         _stream(stream), err, len(err)), err)


# --------------------------------------------------------------- audio encoder

def encoder_released_config() -> dict:
    """The released audio tokenizer's encoder (tests/config_samples.hpp:34-70
    of the reference): HuBERT base at 16 kHz (7 feature convolutions of 512
    channels, 12 layers of 768 x 3072, 12 heads, positional convolution of
    128 taps in 16 groups), semantic stride 2, the DAC encoder from 64
    channels doubling over strides 8 5 4 2 3 to 256 latent channels, 8
    codebooks of 1024 x 64."""
    return dict(sample_rate=24000, semantic_rate=16000, frame_samples=960, semantic_stride=2,
                conv_dim=[512] * 7, conv_kernel=[10, 3, 3, 3, 3, 2, 2],
                conv_stride=[5, 2, 2, 2, 2, 2, 2], width=768, intermediate=3072, heads=12,
                layers=12, pos_kernel=128, pos_groups=16, eps=1e-5, enc_channels=64,
                latent=256, ratios=[8, 5, 4, 2, 3], codebooks=8, codebook_size=1024,
                codebook_dim=64)


def _encoder_config(cfg: dict) -> _EncoderConfig:
    def arr(v):
        return (_i64 * 8)(*v)
    return _EncoderConfig(cfg["sample_rate"], cfg["semantic_rate"], cfg["frame_samples"],
                          cfg["semantic_stride"], len(cfg["conv_dim"]), arr(cfg["conv_dim"]),
                          arr(cfg["conv_kernel"]), arr(cfg["conv_stride"]), cfg["width"],
                          cfg["intermediate"], cfg["heads"], cfg["layers"], cfg["pos_kernel"],
                          cfg["pos_groups"], cfg["eps"], cfg["enc_channels"], cfg["latent"],
                          len(cfg["ratios"]), arr(cfg["ratios"]), cfg["codebooks"],
                          cfg["codebook_size"], cfg["codebook_dim"])


class Encoder:
    """The audio tokenizer's encoder on the GPU: 24 kHz mono float32 audio, a
    whole number of frames, to codes [codebooks][frames] (codec.hpp:16-45 of
    the reference, Encode). Not thread-safe."""

    def __init__(self, handle: int, cfg: dict):
        self._h = handle
        self.cfg = dict(cfg)

    @classmethod
    def load(cls, cfg: dict, model_root: Optional[str] = None) -> "Encoder":
        """The encoder half of model_root/audio_tokenizer/model.safetensors
        (None or "" names the working directory, as the reference joins the
        path)."""
        c = _encoder_config(cfg)
        h = _ptr()
        err = _buf()
        root = (model_root or "").encode()
        _check(lib().ovc_encoder_create(ctypes.byref(c), root, 0, ctypes.byref(h), err,
                                        len(err)), err)
        return cls(h.value, cfg)

    @classmethod
    def synthetic(cls, cfg: dict, seed: int = 1234) -> "Encoder":
        """The seeded synthetic encoder."""
        c = _encoder_config(cfg)
        h = _ptr()
        err = _buf()
        _check(lib().ovc_encoder_create_synthetic(ctypes.byref(c), seed, ctypes.byref(h),
                                                  err, len(err)), err)
        return cls(h.value, cfg)

    def frames(self, samples: int) -> int:
        return int(lib().ovc_encoder_frames(self._h, samples))

    def encode(self, samples, intermediates: bool = False):
        """Codes [codebooks][frames] (int32); with `intermediates`, a dict
        that also holds the averaged HuBERT features [frames][width], the
        DAC encoder output [frames][latent] and fc's output [frames][hidden]."""
        x = np.ascontiguousarray(samples, dtype=np.float32)
        c = self.cfg
        n = max(self.frames(len(x)), 1)
        codes = np.zeros((c["codebooks"], n), dtype=np.int32)
        extra = None
        if intermediates:
            extra = dict(semantic=np.zeros((n, c["width"]), np.float32),
                         acoustic=np.zeros((n, c["latent"]), np.float32),
                         embeddings=np.zeros((n, c["width"] + c["latent"]), np.float32))
        err = _buf()
        _check(lib().ovc_encode(self._h, _p(x), len(x), _p(codes),
                                _p(extra["semantic"]) if extra else None,
                                _p(extra["acoustic"]) if extra else None,
                                _p(extra["embeddings"]) if extra else None, err, len(err)),
               err)
        if extra is None:
            return codes
        return dict(codes=codes, **extra)

    def encode_device(self, samples, codes, stream=None) -> None:
        """samples: float32 device tensor; codes: int32 device tensor
        [codebooks][frames]. Enqueued on `stream`."""
        err = _buf()
        _check(lib().ovc_encode_device(self._h, _dev(samples), samples.numel(), _dev(codes),
                                       _stream(stream), err, len(err)), err)

    def profile(self, samples: int, repeats: int = 3) -> dict:
        cap = 64
        stats = (_KernelStat * cap)()
        count = _i64()
        err = _buf()
        _check(lib().ovc_profile_encode(self._h, samples, repeats, ctypes.cast(stats, _ptr),
                                        cap, ctypes.byref(count), err, len(err)), err)
        out = {}
        for i in range(min(count.value, cap)):
            s = stats[i]
            out[s.name.decode()] = dict(launches=s.launches, total_ms=s.total_ms,
                                        flops=s.flops, bytes=s.bytes)
        return out

    def close(self) -> None:
        if self._h:
            lib().ovc_encoder_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
