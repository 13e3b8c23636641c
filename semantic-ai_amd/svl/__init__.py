"""Python binding of libsvl (the MI355X streaming-transformer step, C ABI in include/svl.h).

The classes mirror the reference crate's step API (crates/semantic-voice-local/src = SVL):

  * ``Model``                       Transformer::new + LanguageModel::new / FlowLm::new
  * ``Model.init_state``            Transformer::init_state          (SVL/nn/transformer.rs:127-136)
  * ``State.duplicate``             TransformerState::duplicate      (SVL/nn/transformer.rs:64-73)
  * ``Model.state_from_layer_caches`` TransformerState::from_layer_caches (transformer.rs:81-103)
  * ``State.layer_caches``          TransformerState::layer_caches   (transformer.rs:76-78)
  * ``Model.forward``               Transformer::forward             (transformer.rs:139-154)
  * ``Model.step``                  LanguageModel::step              (SVL/stt/model.rs:239-276)
  * ``Model.recognize``             Recognizer::step's token loop    (SVL/stt/mod.rs:551-566)
  * ``Model.backbone_step``         FlowLm::step, backbone part      (SVL/tts/flow_lm.rs:162-181)
  * ``Model.tts_step``              FlowLm::step with the sampler's noise (SVL/tts/flow_lm.rs:162-185)

Errors raise ``SvlError`` carrying the library's status code (the reference's
``Result<_, Error>``, SVL/error.rs).  There is no CPU fallback: without the built library or a
GPU every call fails.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_PATH = os.environ.get("SVL_LIBRARY") or os.path.join(PKG, "lib", "libsvl.so")

F32, BF16, F16, Q8_0, Q4K, Q4_0, I64 = 0, 1, 2, 3, 4, 5, 6
NORM_LAYER, NORM_RMS = 0, 1
FF_PLAIN_GELU, FF_GATED_SILU, FF_PLAIN_GELU_ERF = 0, 1, 2
MODEL_TRANSFORMER, MODEL_STT, MODEL_TTS = 0, 1, 2
FLOW_LSD, FLOW_MATCHING, FLOW_DRIFTING, FLOW_POINTWISE = 0, 1, 2, 3

ERR_CONFIG, ERR_INVALID_INPUT, ERR_DEVICE, ERR_IO = -1, -2, -3, -4
UNSUPPORTED = 1  # valid for the reference, outside these kernels: run the reference's path

EXPORTS = [
    "svl_last_error", "svl_device_count", "svl_model_create", "svl_model_destroy",
    "svl_model_linear_weight", "svl_state_create", "svl_state_duplicate", "svl_state_load_stream",
    "svl_state_layer_cache", "svl_state_positions", "svl_state_reset", "svl_state_destroy",
    "svl_state_synchronize", "svl_state_stream", "svl_transformer_forward", "svl_stt_step",
    "svl_stt_recognize", "svl_stt_recognize_async", "svl_stt_step_heads", "svl_stt_recognize_heads",
    "svl_stt_recognize_heads_async", "svl_tts_backbone_step",
    "svl_stt_recognize_noalloc", "svl_bench_copy", "svl_bench_read", "svl_bench_row_stats", "svl_bench_phase", "svl_bench_activation",
    "svl_tts_step", "svl_tts_step_async", "svl_stt_recognize_turns", "svl_stt_recognize_turns_async",
    "svl_state_load_voice", "svl_rvq_create", "svl_rvq_destroy", "svl_rvq_encode", "svl_rvq_encode_async",
    "svl_rvq_synchronize",
]


class SvlError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class SvlUnsupported(SvlError):
    """The request is valid but outside what the GPU kernels cover (svl.h SVL_UNSUPPORTED): the
    reference's kernels return None in that case and the caller runs the reference's own path
    (SVL/nn/kernels/matvec.rs:12-17)."""


class Config(C.Structure):
    _fields_ = [
        ("kind", C.c_int32),
        ("d_model", C.c_int32), ("num_layers", C.c_int32), ("num_heads", C.c_int32),
        ("num_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("ff_kind", C.c_int32), ("ff_hidden", C.c_int32),
        ("norm_kind", C.c_int32), ("norm_eps", C.c_float),
        ("layer_scale", C.c_int32), ("context", C.c_int32), ("max_period", C.c_double),
        ("quantize", C.c_int32),
        ("card", C.c_int32), ("n_q", C.c_int32), ("text_card", C.c_int32),
        ("latent_dim", C.c_int32), ("z_dim", C.c_int32),
        ("kv_dtype", C.c_int32),
        ("extra_heads_num", C.c_int32), ("extra_heads_dim", C.c_int32),
        ("flow_dim", C.c_int32), ("flow_depth", C.c_int32), ("flow_kind", C.c_int32),
    ]


class TurnConfig(C.Structure):
    """TurnDetector's parameters (SVL/stt/mod.rs:283-325)."""
    _fields_ = [("threshold", C.c_float), ("frames", C.c_int32), ("head", C.c_int32)]


class Tensor(C.Structure):
    _fields_ = [
        ("name", C.c_char_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
        ("shape", C.c_int64 * 5), ("data", C.c_void_p),
    ]


_lib = None


def load_library(path: str = LIB_PATH):
    """Loads libsvl.so (built by ``make -C semantic-ai_amd``); raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise SvlError(ERR_IO, f"{path} is not built (run: make -C {PKG})")
    L = C.CDLL(path)
    vp, i32, i64, sz = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t
    L.svl_last_error.restype = C.c_char_p
    L.svl_device_count.argtypes = [C.POINTER(C.c_int)]
    L.svl_model_create.argtypes = [C.POINTER(Config), C.POINTER(Tensor), sz, C.c_int, C.POINTER(vp)]
    L.svl_model_destroy.argtypes = [vp]
    L.svl_model_destroy.restype = None
    L.svl_model_linear_weight.argtypes = [vp, C.c_char_p, vp, sz, vp, sz]
    L.svl_state_create.argtypes = [vp, i32, i32, C.POINTER(vp)]
    L.svl_state_duplicate.argtypes = [vp, C.POINTER(vp)]
    L.svl_state_load_stream.argtypes = [vp, i32, i64, C.POINTER(vp), C.POINTER(vp)]
    L.svl_state_layer_cache.argtypes = [vp, i32, i32, vp, vp, C.POINTER(i64), C.POINTER(i64)]
    L.svl_state_load_voice.argtypes = [vp, i32, C.POINTER(Tensor), sz]
    L.svl_state_positions.argtypes = [vp, vp]
    L.svl_state_reset.argtypes = [vp]
    L.svl_state_destroy.argtypes = [vp]
    L.svl_state_destroy.restype = None
    L.svl_state_synchronize.argtypes = [vp]
    L.svl_state_stream.argtypes = [vp]
    L.svl_state_stream.restype = vp
    L.svl_transformer_forward.argtypes = [vp, vp, vp, i64, vp]
    L.svl_stt_step.argtypes = [vp, vp, vp, vp, vp, vp]
    L.svl_stt_recognize.argtypes = [vp, vp, i64, vp, vp]
    L.svl_stt_step_heads.argtypes = [vp, vp, vp, vp, vp, vp, vp]
    L.svl_stt_recognize_heads.argtypes = [vp, vp, i64, vp, vp, vp]
    L.svl_stt_recognize_heads_async.argtypes = [vp, vp, i64, vp, vp, vp]
    L.svl_stt_recognize_async.argtypes = [vp, vp, i64, vp, vp]
    L.svl_tts_backbone_step.argtypes = [vp, vp, vp, vp]
    L.svl_stt_recognize_noalloc.argtypes = [vp, vp, i64, vp, vp]
    L.svl_tts_step.argtypes = [vp, vp, vp, vp, i32, C.c_float, vp, vp, vp]
    L.svl_stt_recognize_turns.argtypes = [vp, vp, i64, vp, C.POINTER(TurnConfig), vp, vp, vp]
    L.svl_stt_recognize_turns_async.argtypes = [vp, vp, i64, vp, C.POINTER(TurnConfig), vp, vp, vp]
    L.svl_tts_step_async.argtypes = [vp, vp, vp, vp, i32, vp, vp]
    L.svl_rvq_create.argtypes = [C.POINTER(Tensor), sz, i32, i32, C.c_int, C.POINTER(vp)]
    L.svl_rvq_destroy.argtypes = [vp]
    L.svl_rvq_destroy.restype = None
    L.svl_rvq_encode.argtypes = [vp, i32, i32, vp, vp]
    L.svl_rvq_encode_async.argtypes = [vp, i32, i32, vp, vp]
    L.svl_rvq_synchronize.argtypes = [vp]
    L.svl_bench_phase.argtypes = [vp, vp, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_int)]
    L.svl_bench_copy.argtypes = [C.c_int, vp, vp, sz, vp]
    L.svl_bench_read.argtypes = [C.c_int, vp, sz, C.c_int, C.c_int, vp, vp]
    L.svl_bench_row_stats.argtypes = [C.c_int, vp, C.c_int, C.c_int, C.c_int, vp, vp]
    L.svl_bench_activation.argtypes = [C.c_int, C.c_int, vp, sz, vp, vp]
    for name in EXPORTS:
        if name not in ("svl_last_error", "svl_model_destroy", "svl_state_destroy", "svl_state_stream",
                        "svl_rvq_destroy"):
            getattr(L, name).restype = C.c_int
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc == UNSUPPORTED:
        raise SvlUnsupported(rc, load_library().svl_last_error().decode())
    if rc != 0:
        raise SvlError(rc, load_library().svl_last_error().decode())


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def activation(kind: int, x, device: int = 0) -> np.ndarray:
    """The step kernels' exp (0), SiLU (1), GELU-tanh (2) or erf GELU (3) of x on the GPU
    (svl_bench_activation)."""
    from . import hip
    v = np.ascontiguousarray(x, dtype=np.float32).ravel()
    dx = hip.DeviceBuffer.from_array(v)
    dy = hip.DeviceBuffer(v.nbytes)
    _check(load_library().svl_bench_activation(device, kind, C.c_void_p(dx.address), v.size, C.c_void_p(dy.address),
                                                None))
    hip.synchronize()
    return dy.to_array(np.float32, v.size).reshape(np.shape(x))


def row_stats(x: np.ndarray, norm: int, device: int = 0) -> np.ndarray:
    """[rows, 2] = (sum of x^2, sum of x) of every row of x [rows, k] as the decode step's norm
    prologues compute them (svl_bench_row_stats)."""
    from . import hip

    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    dx = hip.DeviceBuffer.from_array(x)
    dout = hip.DeviceBuffer(rows * 2 * 4)
    _check(load_library().svl_bench_row_stats(device, C.c_void_p(dx.address), rows, k, norm,
                                              C.c_void_p(dout.address), None))
    hip.synchronize()
    return dout.to_array(np.float32, rows * 2).reshape(rows, 2)


def device_count() -> int:
    n = C.c_int(0)
    _check(load_library().svl_device_count(C.byref(n)))
    return n.value


def make_config(cfg: dict) -> Config:
    c = Config()
    for k, v in cfg.items():
        setattr(c, k, v)
    return c


def _tensor_array(tensors: dict):
    keep = []
    arr = (Tensor * len(tensors))()
    for i, (name, (dtype, shape, data)) in enumerate(tensors.items()):
        data = np.ascontiguousarray(data)
        nm = name.encode()
        keep += [data, nm]
        arr[i].name = nm
        arr[i].dtype = dtype
        arr[i].ndim = len(shape)
        for j, s in enumerate(shape):
            arr[i].shape[j] = s
        arr[i].data = data.ctypes.data
    return arr, keep


class Rvq:
    """Mimi's split residual vector quantizer on one GPU (svl_rvq_*, SVL/stt/model.rs:84-174).
    ``tensors``: name -> (dtype code, shape, ndarray), the names of svl.h."""

    def __init__(self, tensors: dict, n_q: int, bins: int, device: int = 0):
        L = load_library()
        arr, keep = _tensor_array(tensors)
        h = C.c_void_p()
        _check(L.svl_rvq_create(arr, len(tensors), n_q, bins, device, C.byref(h)))
        self.h, self.n_q, self.bins = h, n_q, bins

    def close(self):
        if getattr(self, "h", None):
            load_library().svl_rvq_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def encode(self, latents) -> np.ndarray:
        """latents [batch, 512, frames] -> codes [batch, frames, n_q] (uint32)."""
        x = np.ascontiguousarray(latents, dtype=np.float32)
        b, c, t = x.shape
        if c != 512:
            raise ValueError("512 latent channels expected")
        codes = np.empty((b, t, self.n_q), np.uint32)
        _check(load_library().svl_rvq_encode(self.h, b, t, _p(x), _p(codes)))
        return codes

    def encode_async(self, batch: int, frames: int, d_latents: int, d_codes: int) -> None:
        """Device-pointer variant: enqueues on the quantizer's stream and returns."""
        _check(load_library().svl_rvq_encode_async(self.h, batch, frames, C.c_void_p(d_latents), C.c_void_p(d_codes)))

    def synchronize(self) -> None:
        _check(load_library().svl_rvq_synchronize(self.h))


class Model:
    """A model on one GPU.  ``tensors``: name -> (dtype code, shape, ndarray)."""

    def __init__(self, cfg: dict, tensors: dict, device: int = 0, kv_dtype: int = F32):
        L = load_library()
        self.cfg = dict(cfg)
        self.cfg["kv_dtype"] = kv_dtype
        keep = []
        arr = (Tensor * len(tensors))()
        for i, (name, (dtype, shape, data)) in enumerate(tensors.items()):
            data = np.ascontiguousarray(data)
            nm = name.encode()
            keep += [data, nm]
            arr[i].name = nm
            arr[i].dtype = dtype
            arr[i].ndim = len(shape)
            for j, s in enumerate(shape):
                arr[i].shape[j] = s
            arr[i].data = data.ctypes.data
        c = make_config(self.cfg)
        h = C.c_void_p()
        _check(L.svl_model_create(C.byref(c), arr, len(tensors), device, C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            load_library().svl_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def linear_weight(self, name: str):
        """(dequantized f32 [out, in], candle Q8_0, Q4_0 or Q4K block bytes [out, ...] or None)
        as held on the GPU."""
        out, inp = self._linear_shape(name)
        w = np.empty((out, inp), dtype=np.float32)
        L = load_library()
        _check(L.svl_model_linear_weight(self.h, name.encode(), _p(w), w.size, None, 0))
        for values, nbytes in ((32, 34), (32, 18), (256, 144)):  # Q8_0, Q4_0, Q4K
            if inp % values:
                continue
            b = np.empty(out * inp // values * nbytes, dtype=np.uint8)
            try:
                _check(L.svl_model_linear_weight(self.h, name.encode(), None, 0, _p(b), b.size))
            except SvlError:
                continue
            return w, b.reshape(out, inp // values * nbytes)
        return w, None

    def _linear_shape(self, name: str):
        c = self.cfg
        d, hd = c["d_model"], c["head_dim"]
        if name == "text_linear":
            return c["text_card"], d
        if name == "input_linear":
            return d, c["latent_dim"]
        if name == "z_proj":
            return c["z_dim"], d
        layer, which = name.split(".")
        qkv = (c["num_heads"] + 2 * c["num_kv_heads"]) * hd
        F = c["ff_hidden"]
        gated = c["ff_kind"] == FF_GATED_SILU
        return {"in_proj": (qkv, d), "out_proj": (d, c["num_heads"] * hd),
                "ff1": (2 * F if gated else F, d), "ff2": (d, F)}[which]

    def init_state(self, batch: int = 1, capacity: int = 0) -> "State":
        h = C.c_void_p()
        _check(load_library().svl_state_create(self.h, batch, capacity, C.byref(h)))
        return State(self, h, batch)

    def state_from_layer_caches(self, keys, values, capacity: int = 0) -> "State":
        """keys/values: per layer [1, kvh, len, hd] (or [kvh, len, hd])."""
        st = self.init_state(1, capacity)
        st.load_stream(0, keys, values)
        return st

    # -- steps ----------------------------------------------------------------------------------
    def forward(self, xs, state: "State") -> np.ndarray:
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        ys = np.empty_like(xs)
        _check(load_library().svl_transformer_forward(self.h, state.h, _p(xs), xs.shape[1], _p(ys)))
        return ys

    def step(self, text_tokens, audio_tokens, state: "State", want_logits: bool = False,
             want_probs: bool = False):
        """LanguageModel::step for every stream -> tokens [batch] (+ logits [batch, text_card])
        (+ the extra heads' first-class probabilities [batch, extra_heads_num])."""
        t = np.ascontiguousarray(np.atleast_1d(text_tokens), dtype=np.uint32)
        a = np.ascontiguousarray(audio_tokens, dtype=np.uint32)
        out = np.empty(state.batch, dtype=np.uint32)
        logits = np.empty((state.batch, self.cfg["text_card"]), dtype=np.float32) if want_logits else None
        probs = (np.empty((state.batch, self.cfg.get("extra_heads_num", 0)), dtype=np.float32)
                 if want_probs else None)
        _check(load_library().svl_stt_step_heads(self.h, state.h, _p(t), _p(a), _p(out),
                                                 None if logits is None else _p(logits),
                                                 None if probs is None else _p(probs)))
        res = (out,) + ((logits,) if want_logits else ()) + ((probs,) if want_probs else ())
        return res if len(res) > 1 else out

    def recognize(self, audio_tokens, state: "State", want_probs: bool = False):
        """audio_tokens [n_steps, batch, n_q] -> tokens [n_steps, batch] (+ the extra heads'
        probabilities [n_steps, batch, extra_heads_num])."""
        a = np.ascontiguousarray(audio_tokens, dtype=np.uint32)
        n = a.shape[0]
        out = np.empty((n, state.batch), dtype=np.uint32)
        if not want_probs:
            _check(load_library().svl_stt_recognize(self.h, state.h, n, _p(a), _p(out)))
            return out
        probs = np.empty((n, state.batch, self.cfg.get("extra_heads_num", 0)), dtype=np.float32)
        _check(load_library().svl_stt_recognize_heads(self.h, state.h, n, _p(a), _p(out), _p(probs)))
        return out, probs

    def recognize_turns(self, audio_tokens, state: "State", threshold: float = 0.5, frames: int = 1,
                        head: int = 2):
        """audio_tokens [n_steps, batch, n_q] -> (tokens [n_steps, batch], the extra heads'
        probabilities [n_steps, batch, extra_heads_num], turn ends [n_steps, batch])."""
        a = np.ascontiguousarray(audio_tokens, dtype=np.uint32)
        n = a.shape[0]
        out = np.empty((n, state.batch), dtype=np.uint32)
        nh = self.cfg.get("extra_heads_num", 0)
        probs = np.empty((n, state.batch, nh), dtype=np.float32)
        ends = np.empty((n, state.batch), dtype=np.int32)
        cfg = TurnConfig(threshold, frames, head)
        _check(load_library().svl_stt_recognize_turns(self.h, state.h, n, _p(a), C.byref(cfg), _p(out),
                                                      _p(probs) if nh else None, _p(ends)))
        return out, probs, ends

    def recognize_async(self, n_steps: int, d_audio: int, d_out: int, state: "State") -> None:
        """Device-pointer variant: enqueues on the state's stream and returns."""
        _check(load_library().svl_stt_recognize_async(self.h, state.h, n_steps, C.c_void_p(d_audio),
                                                      C.c_void_p(d_out)))

    def backbone_step(self, latent, state: "State") -> np.ndarray:
        zd = self.cfg.get("z_dim", 0) or self.cfg["d_model"]
        z = np.empty((state.batch, zd), dtype=np.float32)
        lat = None if latent is None else np.ascontiguousarray(latent, dtype=np.float32)
        _check(load_library().svl_tts_backbone_step(self.h, state.h, None if lat is None else _p(lat), _p(z)))
        return z

    def tts_step(self, latent, noise, state: "State", decode_steps: int = 1, eos_threshold: float = -4.0):
        """FlowLm::step for every stream with the sampler's noise [batch, latent_dim] ->
        (latents [batch, latent_dim], eos logits [batch], eos flags [batch])."""
        ld = self.cfg["latent_dim"]
        nz = np.ascontiguousarray(noise, dtype=np.float32).reshape(state.batch, ld)
        lat = None if latent is None else np.ascontiguousarray(latent, dtype=np.float32).reshape(state.batch, ld)
        out = np.empty((state.batch, ld), dtype=np.float32)
        logits = np.empty(state.batch, dtype=np.float32)
        flags = np.empty(state.batch, dtype=np.int32)
        _check(load_library().svl_tts_step(self.h, state.h, None if lat is None else _p(lat), _p(nz), decode_steps,
                                           eos_threshold, _p(out), _p(logits), _p(flags)))
        return out, logits, flags

    def tts_step_async(self, d_latent: int, d_noise: int, decode_steps: int, d_out: int, d_eos: int,
                       state: "State") -> None:
        """Device-pointer variant (d_latent 0: bos); enqueues on the state's stream."""
        _check(load_library().svl_tts_step_async(self.h, state.h, C.c_void_p(d_latent or None), C.c_void_p(d_noise),
                                                 decode_steps, C.c_void_p(d_out), C.c_void_p(d_eos or None)))


class State:
    def __init__(self, model: Model, h, batch: int):
        self.model = model
        self.h = h
        self.batch = batch

    def close(self):
        if getattr(self, "h", None):
            load_library().svl_state_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def duplicate(self) -> "State":
        h = C.c_void_p()
        _check(load_library().svl_state_duplicate(self.h, C.byref(h)))
        return State(self.model, h, self.batch)

    def load_stream(self, stream: int, keys, values) -> None:
        ks = [np.ascontiguousarray(np.asarray(k, dtype=np.float32).reshape(-1)) for k in keys]
        vs = [np.ascontiguousarray(np.asarray(v, dtype=np.float32).reshape(-1)) for v in values]
        c = self.model.cfg
        n = ks[0].size // (c["num_kv_heads"] * c["head_dim"]) if ks else 0
        kp = (C.c_void_p * len(ks))(*[k.ctypes.data for k in ks])
        vp = (C.c_void_p * len(vs))(*[v.ctypes.data for v in vs])
        _check(load_library().svl_state_load_stream(self.h, stream, n, kp, vp))

    def load_voice(self, tensors: dict, stream: int = 0) -> None:
        """Voice::load (SVL/tts/voice.rs:103-143) from name -> (dtype code, shape, ndarray)."""
        keep = []
        arr = (Tensor * len(tensors))()
        for i, (name, (dtype, shape, data)) in enumerate(tensors.items()):
            data = np.ascontiguousarray(data)
            nm = name.encode()
            keep += [data, nm]
            arr[i].name = nm
            arr[i].dtype = dtype
            arr[i].ndim = len(shape)
            for j, d in enumerate(shape):
                arr[i].shape[j] = d
            arr[i].data = data.ctypes.data
        _check(load_library().svl_state_load_voice(self.h, stream, arr, len(tensors)))

    def layer_caches(self, stream: int = 0):
        """Per layer (keys, values, first) with keys/values [kvh, len, hd]."""
        c = self.model.cfg
        out = []
        L = load_library()
        for layer in range(c["num_layers"]):
            n, first = C.c_int64(), C.c_int64()
            _check(L.svl_state_layer_cache(self.h, stream, layer, None, None, C.byref(n), C.byref(first)))
            k = np.empty((c["num_kv_heads"], n.value, c["head_dim"]), dtype=np.float32)
            v = np.empty_like(k)
            _check(L.svl_state_layer_cache(self.h, stream, layer, _p(k), _p(v), C.byref(n), C.byref(first)))
            out.append((k, v, first.value))
        return out

    @property
    def positions(self) -> np.ndarray:
        p = np.empty(self.batch, dtype=np.int64)
        _check(load_library().svl_state_positions(self.h, _p(p)))
        return p

    def reset(self) -> None:
        _check(load_library().svl_state_reset(self.h))

    def synchronize(self) -> None:
        _check(load_library().svl_state_synchronize(self.h))

    @property
    def stream(self) -> int:
        return load_library().svl_state_stream(self.h) or 0
