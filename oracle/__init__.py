"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()`` and by the CPU
baseline leg of ``bench.py``.  The product library (``libsvl.so``) never loads it.

The oracle restates the reference's CPU path of the streaming-transformer step
(crates/semantic-voice-local/src/nn/transformer.rs, nn/kernels/*, nn/mod.rs:55-100,
stt/model.rs:239-276, tts/flow_lm.rs:162-181) in plain C; see svl_oracle.h for the per-function
citations.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, BF16, F16, Q8_0, Q4K, Q4_0 = 0, 1, 2, 3, 4, 5
NORM_LAYER, NORM_RMS = 0, 1
FF_PLAIN, FF_GATED, FF_PLAIN_ERF = 0, 1, 2
MODEL_TRANSFORMER, MODEL_STT, MODEL_TTS = 0, 1, 2
FLOW_LSD, FLOW_MATCHING, FLOW_DRIFTING, FLOW_POINTWISE = 0, 1, 2, 3

Q8_0_BLOCK_BYTES = 34
Q4_0_BLOCK_BYTES = 18
Q4K_BLOCK_BYTES = 144
Q8K_BLOCK_BYTES = 292

_lock = threading.Lock()
_lib = None


def build(force: bool = False) -> str:
    """Compiles liboracle.so with the Makefile beside this file."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else []), check=True)
    return LIB_PATH


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
        ("extra_heads_num", C.c_int32), ("extra_heads_dim", C.c_int32),
        ("flow_dim", C.c_int32), ("flow_depth", C.c_int32), ("flow_kind", C.c_int32),
    ]


class Tensor(C.Structure):
    _fields_ = [
        ("name", C.c_char_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
        ("shape", C.c_int64 * 4), ("data", C.c_void_p),
    ]


def lib():
    global _lib
    with _lock:
        if _lib is None:
            build()
            L = C.CDLL(LIB_PATH)
            vp, sz, f32p = C.c_void_p, C.c_size_t, C.POINTER(C.c_float)
            L.svlo_f32_to_f16.restype = C.c_uint16
            L.svlo_f32_to_f16.argtypes = [C.c_float]
            L.svlo_f16_to_f32.restype = C.c_float
            L.svlo_f16_to_f32.argtypes = [C.c_uint16]
            L.svlo_f32_to_bf16.restype = C.c_uint16
            L.svlo_f32_to_bf16.argtypes = [C.c_float]
            for name in ["svlo_f32_to_f16_n", "svlo_f32_to_bf16_n", "svlo_bf16_to_f32_n",
                         "svlo_quantize_q8_0", "svlo_dequantize_q8_0", "svlo_quantize_q4k",
                         "svlo_dequantize_q4k", "svlo_quantize_q8k", "svlo_quantize_q4_0",
                         "svlo_dequantize_q4_0"]:
                getattr(L, name).argtypes = [vp, vp, sz]
                getattr(L, name).restype = None
            L.svlo_vec_dot_q8_0.argtypes = [sz, vp, vp]
            L.svlo_vec_dot_q8_0.restype = C.c_float
            L.svlo_vec_dot_q4k_q8k.argtypes = [sz, vp, vp]
            L.svlo_vec_dot_q4k_q8k.restype = C.c_float
            L.svlo_vec_dot_q4_0_q8_0.argtypes = [sz, vp, vp]
            L.svlo_vec_dot_q4_0_q8_0.restype = C.c_float
            L.svlo_set_fma.argtypes = [C.c_int]
            L.svlo_set_threads.argtypes = [C.c_int]
            L.svlo_set_norm_order.argtypes = [C.c_int]
            L.svlo_get_norm_order.restype = C.c_int
            L.svlo_get_threads.restype = C.c_int
            L.svlo_get_fma.restype = C.c_int
            L.svlo_dot.argtypes = [vp, vp, sz]
            L.svlo_dot.restype = C.c_float
            for name in ["svlo_exp", "svlo_silu", "svlo_gelu_tanh", "svlo_gelu_erf"]:
                getattr(L, name).argtypes = [C.c_float]
                getattr(L, name).restype = C.c_float
            L.svlo_silu_n.argtypes = [vp, sz]
            L.svlo_gelu_tanh_n.argtypes = [vp, sz]
            L.svlo_matvec.argtypes = [vp, vp, vp, vp, sz, sz]
            L.svlo_attention.argtypes = [vp, vp, vp, vp] + [sz] * 9
            L.svlo_attention.restype = C.c_int
            L.svlo_rms_norm.argtypes = [vp, vp, vp, sz, sz, C.c_float]
            L.svlo_layer_norm.argtypes = [vp, vp, vp, vp, sz, sz, C.c_float]
            L.svlo_rope_i.argtypes = [vp, vp, vp, sz, sz, sz]
            L.svlo_rope_tables.argtypes = [sz, sz, sz, C.c_double, vp, vp]
            L.svlo_argmax.argtypes = [vp, sz]
            L.svlo_argmax.restype = C.c_uint32
            L.svlo_model_create.argtypes = [C.POINTER(Config), C.POINTER(Tensor), sz, C.POINTER(vp)]
            L.svlo_model_create.restype = C.c_int
            L.svlo_model_destroy.argtypes = [vp]
            L.svlo_last_error.restype = C.c_char_p
            L.svlo_model_linear_weight.argtypes = [vp, C.c_char_p, vp, sz]
            L.svlo_model_linear_weight.restype = C.c_int
            L.svlo_state_create.argtypes = [vp, C.c_int32]
            L.svlo_state_create.restype = vp
            L.svlo_state_duplicate.argtypes = [vp]
            L.svlo_state_duplicate.restype = vp
            L.svlo_state_destroy.argtypes = [vp]
            L.svlo_state_position.argtypes = [vp]
            L.svlo_state_position.restype = C.c_int64
            L.svlo_state_cache_info.argtypes = [vp, C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
            L.svlo_state_cache_copy.argtypes = [vp, C.c_int, vp, vp]
            L.svlo_state_from_layer_caches.argtypes = [vp, C.c_int32, C.c_int64, C.POINTER(vp), C.POINTER(vp)]
            L.svlo_state_from_layer_caches.restype = vp
            L.svlo_transformer_forward.argtypes = [vp, vp, vp, C.c_int64, vp]
            L.svlo_transformer_forward.restype = C.c_int
            L.svlo_stt_step.argtypes = [vp, vp, C.c_uint32, vp, C.POINTER(C.c_uint32), vp, vp]
            L.svlo_stt_step.restype = C.c_int
            L.svlo_stt_greedy.argtypes = [vp, vp, C.c_int64, vp, vp, vp, vp]
            L.svlo_tts_step.argtypes = [vp, vp, vp, vp, C.c_int, vp, vp]
            L.svlo_rvq_create.argtypes = [C.c_int, C.c_int, vp, vp, vp, vp]
            L.svlo_rvq_create.restype = vp
            L.svlo_rvq_destroy.argtypes = [vp]
            L.svlo_rvq_codebook.argtypes = [vp, C.c_int, vp, vp]
            L.svlo_rvq_encode.argtypes = [vp, sz, sz, vp, vp]
            L.svlo_turn_init.argtypes = [vp, C.c_float, C.c_int, C.c_int]
            L.svlo_turn_init.restype = None
            L.svlo_turn_word.argtypes = [vp]
            L.svlo_turn_activity.argtypes = [vp, vp, C.c_int]
            L.svlo_turn_step.argtypes = [vp, C.c_uint32, vp, C.c_int]
            L.svlo_tts_step.restype = C.c_int
            L.svlo_model_flow.argtypes = [vp]
            L.svlo_model_flow.restype = vp
            L.svlo_flow_time_embed.argtypes = [vp, C.c_int, C.c_float, vp]
            L.svlo_flow_time_embed.restype = None
            L.svlo_flow_time_mean.argtypes = [vp, vp, vp]
            L.svlo_flow_time_mean.restype = None
            L.svlo_flow_forward.argtypes = [vp, vp, vp, vp, vp, vp]
            L.svlo_flow_forward.restype = None
            L.svlo_flow_decode.argtypes = [vp, vp, vp, C.c_int, vp]
            L.svlo_flow_decode.restype = None
            L.svlo_flow_eos_logit.argtypes = [vp, vp]
            L.svlo_flow_eos_logit.restype = C.c_float
            L.svlo_softmax_first.argtypes = [vp, sz]
            L.svlo_softmax_first.restype = C.c_float
            L.svlo_stt_greedy.restype = C.c_int
            L.svlo_tts_backbone_step.argtypes = [vp, vp, vp, vp]
            L.svlo_tts_backbone_step.restype = C.c_int
            _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def set_fma(on: bool) -> None:
    lib().svlo_set_fma(1 if on else 0)


def set_threads(n: int) -> None:
    lib().svlo_set_threads(int(n))


def get_threads() -> int:
    return lib().svlo_get_threads()


NORM_ORDERS = {"element": 0, "blocked": 1}


def set_norm_order(order: str) -> None:
    """Summation order of the RMSNorm / LayerNorm statistics: "element" (candle's CPU ops, the
    default) or "blocked" (the order of the GPU kernels)."""
    lib().svlo_set_norm_order(NORM_ORDERS[order])


def get_norm_order() -> str:
    return {v: k for k, v in NORM_ORDERS.items()}[lib().svlo_get_norm_order()]


# ---- formats --------------------------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().svlo_f32_to_f16_n(_p(x), _p(y), x.size)
    return y


def f16_bits_to_f32(h: int) -> float:
    return lib().svlo_f16_to_f32(int(h))


def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().svlo_f32_to_bf16_n(_p(x), _p(y), x.size)
    return y


def bf16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().svlo_bf16_to_f32_n(_p(h), _p(y), h.size)
    return y


def quantize_q8_0(x) -> np.ndarray:
    """[rows, k] f32 -> [rows, k/32 * 34] uint8 candle Q8_0 blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    assert k % 32 == 0
    out = np.empty(x.shape[:-1] + (k // 32 * Q8_0_BLOCK_BYTES,), dtype=np.uint8)
    lib().svlo_quantize_q8_0(_p(x), _p(out), x.size)
    return out


def dequantize_q8_0(blocks, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows = blocks.size // (k // 32 * Q8_0_BLOCK_BYTES)
    out = np.empty(blocks.shape[:-1] + (k,), dtype=np.float32)
    lib().svlo_dequantize_q8_0(_p(blocks), _p(out), rows * k)
    return out


def vec_dot_q8_0(w_blocks, x_blocks, n: int) -> float:
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x_blocks, dtype=np.uint8)
    return lib().svlo_vec_dot_q8_0(n, _p(w), _p(x))


def quantize_q4_0(x) -> np.ndarray:
    """[rows, k] f32 -> [rows, k/32 * 18] uint8 candle Q4_0 blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    assert k % 32 == 0
    out = np.empty(x.shape[:-1] + (k // 32 * Q4_0_BLOCK_BYTES,), dtype=np.uint8)
    lib().svlo_quantize_q4_0(_p(x), _p(out), x.size)
    return out


def dequantize_q4_0(blocks, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows = blocks.size // (k // 32 * Q4_0_BLOCK_BYTES)
    out = np.empty(blocks.shape[:-1] + (k,), dtype=np.float32)
    lib().svlo_dequantize_q4_0(_p(blocks), _p(out), rows * k)
    return out


def vec_dot_q4_0_q8_0(w_blocks, x_blocks, n: int) -> float:
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x_blocks, dtype=np.uint8)
    return lib().svlo_vec_dot_q4_0_q8_0(n, _p(w), _p(x))


def quantize_q4k(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    assert k % 256 == 0
    out = np.empty(x.shape[:-1] + (k // 256 * Q4K_BLOCK_BYTES,), dtype=np.uint8)
    lib().svlo_quantize_q4k(_p(x), _p(out), x.size)
    return out


def dequantize_q4k(blocks, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows = blocks.size // (k // 256 * Q4K_BLOCK_BYTES)
    out = np.empty(blocks.shape[:-1] + (k,), dtype=np.float32)
    lib().svlo_dequantize_q4k(_p(blocks), _p(out), rows * k)
    return out


def quantize_q8k(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    out = np.empty(x.shape[:-1] + (k // 256 * Q8K_BLOCK_BYTES,), dtype=np.uint8)
    lib().svlo_quantize_q8k(_p(x), _p(out), x.size)
    return out


def vec_dot_q4k_q8k(w_blocks, x_blocks, n: int) -> float:
    w = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x_blocks, dtype=np.uint8)
    return lib().svlo_vec_dot_q4k_q8k(n, _p(w), _p(x))


# ---- kernels ---------------------------------------------------------------------------------

def dot(a, b) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().svlo_dot(_p(a), _p(b), a.size)


def exp(x: float) -> float:
    return lib().svlo_exp(float(x))


def silu_n(x) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True).ravel()
    lib().svlo_silu_n(_p(y), y.size)
    return y.reshape(np.shape(x))


def gelu_erf(x: float) -> float:
    return lib().svlo_gelu_erf(float(x))


def gelu_tanh_n(x) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True).ravel()
    lib().svlo_gelu_tanh_n(_p(y), y.size)
    return y.reshape(np.shape(x))


def matvec(x, w, bias=None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    assert x.size == k
    y = np.empty(n, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().svlo_matvec(_p(x), _p(w), None if b is None else _p(b), _p(y), n, k)
    return y


def attention(q, k, v, position: int, first_key: int, context: int | None) -> np.ndarray:
    """q [b,h,t,d]; k, v [b,kvh,n,d] -> [b,t,h,d]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    b, h, t, d = q.shape
    _, kvh, n, _ = k.shape
    out = np.empty((b, t, h, d), dtype=np.float32)
    rc = lib().svlo_attention(_p(q), _p(k), _p(v), _p(out), b, h, t, d, kvh, n, position, first_key,
                              context or 0)
    if rc:
        raise ValueError("attention: shapes")
    return out


def rms_norm(x, alpha, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    a = np.ascontiguousarray(alpha, dtype=np.float32)
    y = np.empty_like(x)
    dim = x.shape[-1]
    lib().svlo_rms_norm(_p(x), _p(a), _p(y), x.size // dim, dim, eps)
    return y


def layer_norm(x, w, b, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    y = np.empty_like(x)
    dim = x.shape[-1]
    lib().svlo_layer_norm(_p(x), _p(w), _p(b), _p(y), x.size // dim, dim, eps)
    return y


def rope_tables(position: int, t: int, head_dim: int, max_period: float):
    cs = np.empty((t, head_dim // 2), dtype=np.float32)
    sn = np.empty((t, head_dim // 2), dtype=np.float32)
    lib().svlo_rope_tables(position, t, head_dim, max_period, _p(cs), _p(sn))
    return cs, sn


def rope_i(x, cos_t, sin_t) -> np.ndarray:
    """x [b,h,t,d] -> rotated copy."""
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    b, h, t, d = y.shape
    cs = np.ascontiguousarray(cos_t, dtype=np.float32)
    sn = np.ascontiguousarray(sin_t, dtype=np.float32)
    lib().svlo_rope_i(_p(y), _p(cs), _p(sn), b * h, t, d)
    return y


def softmax_first(x) -> float:
    """Element 0 of softmax(x) (the oracle's restatement of candle's softmax_last_dim)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(lib().svlo_softmax_first(_p(x), x.size))


def argmax(x) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().svlo_argmax(_p(x), x.size))


# ---- turns (the recognizer's word events and TurnDetector, SVL/stt/mod.rs:283-351, 564-590) ------

class _Turn(C.Structure):
    _fields_ = [("threshold", C.c_float), ("frames", C.c_int32), ("head", C.c_int32),
                ("above", C.c_int64), ("in_turn", C.c_int32), ("pending", C.c_int32)]


class TurnDetector:
    """TurnDetector (threshold 0.5, frames 1, HEAD 2 by default) with the recognizer's pending
    word tokens."""

    def __init__(self, threshold: float = 0.5, frames: int = 1, head: int = 2):
        self.t = _Turn()
        lib().svlo_turn_init(C.byref(self.t), threshold, frames, head)

    def word(self) -> bool:
        return bool(lib().svlo_turn_word(C.byref(self.t)))

    def activity(self, probs) -> bool:
        p = np.ascontiguousarray(probs, dtype=np.float32)
        return bool(lib().svlo_turn_activity(C.byref(self.t), _p(p), p.size))

    def step(self, token: int, probs) -> bool:
        p = np.ascontiguousarray(probs, dtype=np.float32)
        return bool(lib().svlo_turn_step(C.byref(self.t), token, _p(p) if p.size else None, p.size))


# ---- Mimi's split residual vector quantizer (rvq.c) ---------------------------------------------

RVQ_IN, RVQ_DIM = 512, 256


class Rvq:
    """Quantizer::encode (SVL/stt/model.rs:84-174).  w_first / w_rest: input_proj weights
    [256, 512] (or [256, 512, 1]); sums [n_q, bins, 256], usage [n_q, bins]: embedding_sum and
    cluster_usage of the first quantizer's codebook, then the rest's."""

    def __init__(self, w_first, w_rest, sums, usage):
        self._w = [np.ascontiguousarray(np.reshape(w, (RVQ_DIM, RVQ_IN)), dtype=np.float32) for w in (w_first, w_rest)]
        s = np.ascontiguousarray(sums, dtype=np.float32)
        u = np.ascontiguousarray(usage, dtype=np.float32)
        self.n_q, self.bins = s.shape[0], s.shape[1]
        assert s.shape == (self.n_q, self.bins, RVQ_DIM) and u.shape == (self.n_q, self.bins)
        self.h = lib().svlo_rvq_create(self.n_q, self.bins, _p(self._w[0]), _p(self._w[1]), _p(s), _p(u))
        if not self.h:
            raise RuntimeError("svlo_rvq_create failed")

    def __del__(self):
        if getattr(self, "h", None):
            lib().svlo_rvq_destroy(self.h)
            self.h = None

    def codebook(self, stage: int):
        emb = np.empty((self.bins, RVQ_DIM), np.float32)
        hn = np.empty(self.bins, np.float32)
        lib().svlo_rvq_codebook(self.h, stage, _p(emb), _p(hn))
        return emb, hn

    def encode(self, latents) -> np.ndarray:
        """latents [batch, 512, frames] -> codes [batch, frames, n_q] (uint32)."""
        x = np.ascontiguousarray(latents, dtype=np.float32)
        b, c, t = x.shape
        assert c == RVQ_IN
        codes = np.empty((b, t, self.n_q), np.uint32)
        lib().svlo_rvq_encode(self.h, b, t, _p(x), _p(codes))
        return codes


# ---- model -------------------------------------------------------------------------------------

def make_config(**kw) -> Config:
    cfg = Config()
    for k, v in kw.items():
        setattr(cfg, k, v)
    return cfg


class Model:
    """Oracle model.  ``tensors`` maps name -> (dtype, shape, ndarray)."""

    def __init__(self, cfg: dict, tensors: dict):
        L = lib()
        self.cfg = dict(cfg)
        self._keep = []
        arr = (Tensor * len(tensors))()
        for i, (name, (dtype, shape, data)) in enumerate(tensors.items()):
            data = np.ascontiguousarray(data)
            self._keep.append(data)
            nm = name.encode()
            self._keep.append(nm)
            arr[i].name = nm
            arr[i].dtype = dtype
            arr[i].ndim = len(shape)
            for j, s in enumerate(shape):
                arr[i].shape[j] = s
            arr[i].data = data.ctypes.data
        c = make_config(**cfg)
        h = C.c_void_p()
        rc = L.svlo_model_create(C.byref(c), arr, len(tensors), C.byref(h))
        self._keep = []
        if rc:
            raise ValueError(L.svlo_last_error().decode())
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib().svlo_model_destroy(self.h)
            self.h = None

    def linear_weight(self, name: str, out: int, inp: int) -> np.ndarray:
        w = np.empty((out, inp), dtype=np.float32)
        if lib().svlo_model_linear_weight(self.h, name.encode(), _p(w), w.size):
            raise ValueError(lib().svlo_last_error().decode())
        return w

    # -- flow head (FlowHead / TimestepEmbedder / out_eos, SVL/tts/flow_lm.rs:181-387) --------
    def _flow(self):
        f = lib().svlo_model_flow(self.h)
        if not f:
            raise ValueError("the model has no flow head")
        return f

    def flow_time_embed(self, i: int, t: float) -> np.ndarray:
        out = np.empty(self.cfg["flow_dim"], dtype=np.float32)
        lib().svlo_flow_time_embed(self._flow(), i, t, _p(out))
        return out

    def flow_time_mean(self, times) -> np.ndarray:
        t = np.ascontiguousarray(times, dtype=np.float32)
        out = np.empty(self.cfg["flow_dim"], dtype=np.float32)
        lib().svlo_flow_time_mean(self._flow(), _p(t), _p(out))
        return out

    def flow_forward(self, cond, times, xs) -> np.ndarray:
        cond = np.ascontiguousarray(cond, dtype=np.float32)
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        t = None if times is None else np.ascontiguousarray(times, dtype=np.float32)
        out = np.empty(self.cfg["latent_dim"], dtype=np.float32)
        lib().svlo_flow_forward(self._flow(), _p(cond), None if t is None else _p(t), None, _p(xs), _p(out))
        return out

    def flow_decode(self, cond, noise, steps: int) -> np.ndarray:
        cond = np.ascontiguousarray(cond, dtype=np.float32)
        noise = np.ascontiguousarray(noise, dtype=np.float32)
        out = np.empty(self.cfg["latent_dim"], dtype=np.float32)
        lib().svlo_flow_decode(self._flow(), _p(cond), _p(noise), steps, _p(out))
        return out

    def eos_logit(self, z) -> float:
        z = np.ascontiguousarray(z, dtype=np.float32)
        return float(lib().svlo_flow_eos_logit(self._flow(), _p(z)))

    def new_state(self, batch: int = 1) -> "State":
        return State(self, lib().svlo_state_create(self.h, batch))

    def state_from_layer_caches(self, ks, vs, batch: int = 1) -> "State":
        n = ks[0].shape[2] if ks else 0
        ks = [np.ascontiguousarray(k, dtype=np.float32) for k in ks]
        vs = [np.ascontiguousarray(v, dtype=np.float32) for v in vs]
        kp = (C.c_void_p * len(ks))(*[k.ctypes.data for k in ks])
        vp = (C.c_void_p * len(vs))(*[v.ctypes.data for v in vs])
        return State(self, lib().svlo_state_from_layer_caches(self.h, batch, n, kp, vp))


class State:
    def __init__(self, model: Model, h):
        self.model = model
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib().svlo_state_destroy(self.h)
            self.h = None

    @property
    def position(self) -> int:
        return lib().svlo_state_position(self.h)

    def duplicate(self) -> "State":
        return State(self.model, lib().svlo_state_duplicate(self.h))

    def cache(self, layer: int):
        ln, st = C.c_int64(), C.c_int64()
        lib().svlo_state_cache_info(self.h, layer, C.byref(ln), C.byref(st))
        cfg = self.model.cfg
        b = 1
        k = np.empty((b, cfg["num_kv_heads"], ln.value, cfg["head_dim"]), dtype=np.float32)
        v = np.empty_like(k)
        lib().svlo_state_cache_copy(self.h, layer, _p(k), _p(v))
        return k, v, st.value

    def forward(self, xs) -> np.ndarray:
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        ys = np.empty_like(xs)
        if lib().svlo_transformer_forward(self.model.h, self.h, _p(xs), xs.shape[1], _p(ys)):
            raise ValueError(lib().svlo_last_error().decode())
        return ys

    def stt_step(self, text_token: int, audio, want_logits: bool = False, want_probs: bool = False):
        audio = np.ascontiguousarray(audio, dtype=np.uint32)
        tok = C.c_uint32()
        logits = np.empty(self.model.cfg["text_card"], dtype=np.float32) if want_logits else None
        probs = (np.empty(self.model.cfg.get("extra_heads_num", 0), dtype=np.float32)
                 if want_probs else None)
        rc = lib().svlo_stt_step(self.model.h, self.h, text_token, _p(audio), C.byref(tok),
                                 None if logits is None else _p(logits),
                                 None if probs is None else _p(probs))
        if rc:
            raise ValueError(lib().svlo_last_error().decode())
        res = (tok.value,) + ((logits,) if want_logits else ()) + ((probs,) if want_probs else ())
        return res if len(res) > 1 else tok.value

    def stt_greedy(self, audio, n: int | None = None, want_logits: bool = False,
                   want_probs: bool = False):
        audio = np.ascontiguousarray(audio, dtype=np.uint32)
        nq = self.model.cfg["n_q"]
        n = audio.size // nq if n is None else n
        out = np.empty(n, dtype=np.uint32)
        logits = np.empty(self.model.cfg["text_card"], dtype=np.float32) if want_logits else None
        probs = (np.empty((n, self.model.cfg.get("extra_heads_num", 0)), dtype=np.float32)
                 if want_probs else None)
        rc = lib().svlo_stt_greedy(self.model.h, self.h, n, _p(audio), _p(out),
                                   None if logits is None else _p(logits),
                                   None if probs is None else _p(probs))
        if rc:
            raise ValueError(lib().svlo_last_error().decode())
        res = (out,) + ((logits,) if want_logits else ()) + ((probs,) if want_probs else ())
        return res if len(res) > 1 else out

    def tts_step(self, latent=None) -> np.ndarray:
        cfg = self.model.cfg
        zd = cfg.get("z_dim", 0) or cfg["d_model"]
        z = np.empty(zd, dtype=np.float32)
        lat = None if latent is None else np.ascontiguousarray(latent, dtype=np.float32)
        if lib().svlo_tts_backbone_step(self.model.h, self.h, None if lat is None else _p(lat), _p(z)):
            raise ValueError(lib().svlo_last_error().decode())
        return z

    def tts_full_step(self, latent, noise, decode_steps: int = 1):
        """FlowLm::step with the sampler's noise -> (next latent [latent_dim], eos logit)."""
        cfg = self.model.cfg
        out = np.empty(cfg["latent_dim"], dtype=np.float32)
        eos = C.c_float()
        lat = None if latent is None else np.ascontiguousarray(latent, dtype=np.float32)
        nz = np.ascontiguousarray(noise, dtype=np.float32)
        if lib().svlo_tts_step(self.model.h, self.h, None if lat is None else _p(lat), _p(nz), decode_steps,
                               _p(out), C.byref(eos)):
            raise ValueError(lib().svlo_last_error().decode())
        return out, eos.value
