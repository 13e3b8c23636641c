"""Synthetic workloads of the streaming-transformer step: model shapes and seeded weights.

Shapes follow the reference's derivations:
  * STT language model (crates/semantic-voice-local/src/stt/model.rs:196-233): RMSNorm eps 1e-8,
    gated SiLU with hidden = 2 * (hidden_scale * dim) / 3, head_dim = dim / num_heads,
    kv_heads = num_heads, window = `context`, text vocabulary text_card (+1 embedding row),
    n_q audio codebooks of card (+1) entries.
  * Pocket-TTS flow-LM backbone (src/tts/flow_lm.rs:45-126, configs/tts/english.yaml):
    LayerNorm eps 1e-5, plain tanh-GELU MLP, no window, latent 32 -> input_linear -> d_model.

Weights are drawn per tensor from numpy's PCG64 seeded with (seed, crc32(name)), so every tensor
is reproducible on its own.  Linear weights, embeddings and LayerNorm biases are N(0, 0.02);
norm scales are 1 + N(0, 0.02) (unit-gain norms, so activations keep their scale through the
layers).  Dtypes: "f32" keeps f32; "bf16" rounds to bfloat16 (round to nearest even, as candle's
`half` crate); "q8_0"/"q4k" hand f32 linear weights to the model with `quantize` set, which
quantizes them when the model is created (SVL/nn/mod.rs:76-87).
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass, field

import numpy as np

F32, BF16, F16, Q8_0, Q4K, Q4_0 = 0, 1, 2, 3, 4, 5
NORM_LAYER, NORM_RMS = 0, 1
FF_PLAIN, FF_GATED, FF_PLAIN_ERF = 0, 1, 2
MODEL_TRANSFORMER, MODEL_STT, MODEL_TTS = 0, 1, 2
FLOW_LSD, FLOW_MATCHING, FLOW_DRIFTING, FLOW_POINTWISE = 0, 1, 2, 3


@dataclass
class Shape:
    name: str
    kind: int
    d_model: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    ff_kind: int
    ff_hidden: int
    norm_kind: int
    norm_eps: float
    context: int  # 0 = unlimited
    max_period: float = 10000.0
    layer_scale: int = 0
    card: int = 0
    n_q: int = 0
    text_card: int = 0
    latent_dim: int = 0
    z_dim: int = 0
    extra_heads_num: int = 0   # STT VAD heads (SVL/stt/model.rs:217-222)
    extra_heads_dim: int = 0
    flow_dim: int = 0          # TTS flow head (FlowHeadConfig, SVL/tts/config.rs:197-204); 0 = none
    flow_depth: int = 0
    flow_kind: int = 0         # FLOW_LSD, FLOW_MATCHING, FLOW_DRIFTING, FLOW_POINTWISE

    def config(self, quantize: int = 0) -> dict:
        return dict(kind=self.kind, d_model=self.d_model, num_layers=self.num_layers,
                    num_heads=self.num_heads, num_kv_heads=self.num_kv_heads,
                    head_dim=self.head_dim, ff_kind=self.ff_kind, ff_hidden=self.ff_hidden,
                    norm_kind=self.norm_kind, norm_eps=self.norm_eps,
                    layer_scale=self.layer_scale, context=self.context,
                    max_period=self.max_period, quantize=quantize, card=self.card,
                    n_q=self.n_q, text_card=self.text_card, latent_dim=self.latent_dim,
                    z_dim=self.z_dim, extra_heads_num=self.extra_heads_num,
                    extra_heads_dim=self.extra_heads_dim, flow_dim=self.flow_dim,
                    flow_depth=self.flow_depth, flow_kind=self.flow_kind)


def stt_shape(name, dim, layers, heads, hidden_scale, context, card=2048, n_q=32, text_card=8000):
    """SVL/stt/model.rs:201-216."""
    ff = int(hidden_scale * dim)
    return Shape(name, MODEL_STT, dim, layers, heads, heads, dim // heads, FF_GATED, 2 * ff // 3,
                 NORM_RMS, 1e-8, context, card=card, n_q=n_q, text_card=text_card)


def tts_shape(name, dim, layers, heads, hidden, latent=32, z_dim=0, flow_dim=0, flow_depth=0,
              flow_kind=FLOW_LSD):
    """SVL/tts/flow_lm.rs:52-71; the flow head of configs/tts/english.yaml:16-19 (dim 512,
    depth 6, LSD)."""
    return Shape(name, MODEL_TTS, dim, layers, heads, heads, dim // heads, FF_PLAIN, hidden,
                 NORM_LAYER, 1e-5, 0, latent_dim=latent, z_dim=z_dim, flow_dim=flow_dim,
                 flow_depth=flow_depth, flow_kind=flow_kind)


# The five benchmark shapes.
S1 = stt_shape("stt-1b", 2048, 16, 16, 4.125, 750)          # hidden 5632
S2 = stt_shape("stt-2.6b", 2560, 24, 20, 4.05, 3000)         # hidden 6912
T1 = tts_shape("pocket-tts", 1024, 6, 16, 4096, flow_dim=512, flow_depth=6)
# Reduced shapes with the same structure, for parity tests the oracle finishes in seconds.
S1_SMALL = stt_shape("stt-small", 256, 3, 4, 4.125, 24, card=64, n_q=4, text_card=100)  # hidden 704
S2_SMALL = stt_shape("stt-small-q4k", 512, 2, 4, 4.5, 40, card=64, n_q=4, text_card=96)  # hidden 1536
T1_SMALL = tts_shape("tts-small", 256, 2, 4, 1024, flow_dim=64, flow_depth=2)

assert S1.ff_hidden == 5632 and S2.ff_hidden == 6912

# The Kyutai STT Mimi's encoder transformer (SVL/stt/model.rs:60-70, SVL/nn/mimi.rs:87-103): d 512,
# 8 layers of 8 heads, erf-GELU feed-forward 2048, LayerNorm 1e-5, layer scale, context 250; it
# runs at the SEANet frame rate (25 Hz), between the SEANet encoder and the downsampling.
MIMI_ENC = Shape("mimi-encoder-transformer", MODEL_TRANSFORMER, 512, 8, 8, 8, 64, FF_PLAIN_ERF, 2048, NORM_LAYER,
                 1e-5, 250, layer_scale=1)


def _rng(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def normal(seed: int, name: str, shape, std: float = 0.02, mean: float = 0.0) -> np.ndarray:
    x = _rng(seed, name).standard_normal(int(np.prod(shape)), dtype=np.float32)
    x *= np.float32(std)
    if mean:
        x += np.float32(mean)
    return x.reshape(shape)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """f32 -> nearest bfloat16 (ties to even), returned as f32 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    rounded = np.where(nan, (u | 0x00400000) & 0xFFFF0000, rounded).astype(np.uint32)
    return rounded.view(np.float32)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def tensor_names(s: Shape):
    """(name, shape, role) of every tensor the model reads; role in {linear, emb, norm_w,
    norm_b, vec}."""
    d, hd = s.d_model, s.head_dim
    qkv = (s.num_heads + 2 * s.num_kv_heads) * hd
    pre = "" if s.kind == MODEL_TRANSFORMER else "transformer."
    out = []
    for i in range(s.num_layers):
        p = f"{pre}layers.{i}."
        if s.norm_kind == NORM_RMS:
            out += [(p + "norm1.alpha", (1, 1, d), "norm_w"), (p + "norm2.alpha", (1, 1, d), "norm_w")]
        else:
            out += [(p + "norm1.weight", (d,), "norm_w"), (p + "norm1.bias", (d,), "norm_b"),
                    (p + "norm2.weight", (d,), "norm_w"), (p + "norm2.bias", (d,), "norm_b")]
        if s.layer_scale:
            out += [(p + "layer_scale_1.scale", (d,), "vec"), (p + "layer_scale_2.scale", (d,), "vec")]
        if s.kind == MODEL_STT:
            out.append((p + "self_attn.in_proj_weight", (qkv, d), "linear"))
        else:
            out.append((p + "self_attn.in_proj.weight", (qkv, d), "linear"))
        out.append((p + "self_attn.out_proj.weight", (d, s.num_heads * hd), "linear"))
        if s.ff_kind == FF_GATED:
            out += [(p + "gating.linear_in.weight", (2 * s.ff_hidden, d), "linear"),
                    (p + "gating.linear_out.weight", (d, s.ff_hidden), "linear")]
        else:
            out += [(p + "linear1.weight", (s.ff_hidden, d), "linear"),
                    (p + "linear2.weight", (d, s.ff_hidden), "linear")]
    if s.kind == MODEL_STT:
        out.append(("text_emb.weight", (s.text_card + 1, d), "emb"))
        out += [(f"emb.{i}.weight", (s.card + 1, d), "emb") for i in range(s.n_q)]
        out.append(("out_norm.alpha", (1, 1, d), "norm_w"))
        out.append(("text_linear.weight", (s.text_card, d), "linear"))
        # dense, never quantized (Linear::load(.., false), SVL/stt/model.rs:219)
        out += [(f"extra_heads.{i}.weight", (s.extra_heads_dim, d), "dense_linear")
                for i in range(s.extra_heads_num)]
    elif s.kind == MODEL_TTS:
        out.append(("input_linear.weight", (d, s.latent_dim), "dense_linear"))
        out += [("out_norm.weight", (d,), "norm_w"), ("out_norm.bias", (d,), "norm_b")]
        if s.z_dim:
            out.append(("z_proj.weight", (s.z_dim, d), "dense_linear"))
        out.append(("bos_emb", (s.latent_dim,), "vec"))
        out += flow_tensor_names(s)
    return out


def flow_tensor_names(s: Shape):
    """The flow head and end-of-speech head (SVL/tts/flow_lm.rs:107-113, 232-251, 322-331,
    359-368): (name, shape, role); roles "flow_linear" (weights) and "vec" (biases),
    "norm_w" / "norm_b", "freqs" (the timestep embedders' frequencies)."""
    if not s.flow_dim:
        return []
    D, L = s.flow_dim, s.latent_dim
    cond = s.z_dim or s.d_model
    n_time = {FLOW_LSD: 2, FLOW_MATCHING: 1}.get(s.flow_kind, 0)
    p = "flow_net."
    out = []
    for i in range(n_time):
        t = f"{p}time_embed.{i}."
        out += [(t + "freqs", (128,), "freqs"),
                (t + "mlp.0.weight", (D, 256), "flow_linear"), (t + "mlp.0.bias", (D,), "vec"),
                (t + "mlp.2.weight", (D, D), "flow_linear"), (t + "mlp.2.bias", (D,), "vec"),
                (t + "mlp.3.alpha", (D,), "norm_w")]
    out += [(p + "cond_embed.weight", (D, cond), "flow_linear"), (p + "cond_embed.bias", (D,), "vec"),
            (p + "input_proj.weight", (D, L), "flow_linear"), (p + "input_proj.bias", (D,), "vec")]
    for j in range(s.flow_depth):
        r = f"{p}res_blocks.{j}."
        out += [(r + "in_ln.weight", (D,), "norm_w"), (r + "in_ln.bias", (D,), "norm_b"),
                (r + "mlp.0.weight", (D, D), "flow_linear"), (r + "mlp.0.bias", (D,), "vec"),
                (r + "mlp.2.weight", (D, D), "flow_linear"), (r + "mlp.2.bias", (D,), "vec"),
                (r + "adaLN_modulation.1.weight", (3 * D, D), "flow_linear"),
                (r + "adaLN_modulation.1.bias", (3 * D,), "vec")]
    f = p + "final_layer."
    out += [(f + "adaLN_modulation.1.weight", (2 * D, D), "flow_linear"),
            (f + "adaLN_modulation.1.bias", (2 * D,), "vec"),
            (f + "linear.weight", (L, D), "flow_linear"), (f + "linear.bias", (L,), "vec"),
            ("out_eos.weight", (1, cond), "flow_linear"), ("out_eos.bias", (1,), "vec")]
    return out


def make_weights(s: Shape, dtype: str, seed: int = 0, threads: int | None = None) -> dict:
    """name -> (dtype code, shape, ndarray) for the oracle and for libsvl.

    dtype "f32": everything f32.  "bf16": everything bf16 (stored as bf16 bits).
    "q8_0"/"q4_0"/"q4k": linear weights f32 (quantized by the model), the rest bf16.
    Tensors are drawn in parallel threads (each has its own generator, so the result does not
    depend on the thread count)."""
    from concurrent.futures import ThreadPoolExecutor
    import os

    def one(item):
        name, shape, role = item
        if role == "freqs":
            # the timestep embedders' frequencies, exp(-ln(10000) k / 128) as the checkpoints
            # hold them
            x = np.exp(-np.log(10000.0) * np.arange(128) / 128).astype(np.float32)
            return name, (F32, shape, x)
        if role == "norm_w":
            x = normal(seed, name, shape, 0.02, 1.0)
        elif role == "vec":
            x = normal(seed, name, shape, 0.02, 1.0 if "layer_scale" in name else 0.0)
        else:
            x = normal(seed, name, shape, 0.02)
        if dtype == "f32" or role == "flow_linear" or (dtype in ("q8_0", "q4_0", "q4k") and role in ("linear", "dense_linear")):
            return name, (F32, shape, x)
        return name, (BF16, shape, to_bf16_bits(x))

    items = tensor_names(s)
    n = threads or min(16, os.cpu_count() or 4)
    with ThreadPoolExecutor(n) as ex:
        return dict(ex.map(one, items))


def quantize_code(dtype: str) -> int:
    return {"f32": 0, "bf16": 0, "q8_0": Q8_0, "q4_0": Q4_0, "q4k": Q4K}[dtype]


def audio_tokens(s: Shape, steps: int, seed: int = 1, batch: int = 1) -> np.ndarray:
    """[batch, steps, n_q] uniform ids in [0, card] (the embedding tables have card + 1 rows)."""
    rng = np.random.default_rng([seed, 0xA0D10])
    return rng.integers(0, s.card + 1, size=(batch, steps, s.n_q), dtype=np.uint32)


def latents(s: Shape, steps: int, seed: int = 2) -> np.ndarray:
    """[steps, latent_dim] N(0, 1) latents fed to the TTS backbone step."""
    rng = np.random.default_rng([seed, 0x1A7E])
    return rng.standard_normal((steps, s.latent_dim), dtype=np.float32)


def prefill_caches(s: Shape, length: int, seed: int = 3):
    """Per-layer seeded K/V caches [1, kvh, length, hd] (as after a voice + text prompt)."""
    ks, vs = [], []
    for i in range(s.num_layers):
        ks.append(normal(seed, f"prefill.k.{i}", (1, s.num_kv_heads, length, s.head_dim), 1.0))
        vs.append(normal(seed, f"prefill.v.{i}", (1, s.num_kv_heads, length, s.head_dim), 1.0))
    return ks, vs


def linear_bytes(s: Shape, dtype: str) -> int:
    """Bytes of the linear weights one step reads, in the format held on the device."""
    total = 0
    for name, shape, role in tensor_names(s):
        if role not in ("linear", "dense_linear"):
            continue
        n = shape[0] * shape[1]
        if role == "dense_linear":
            total += n * (2 if dtype == "bf16" else 4)
        elif dtype == "q8_0" and shape[1] % 32 == 0:
            total += n // 32 * 34
        elif dtype == "q4_0" and shape[1] % 32 == 0:
            total += n // 32 * 18
        elif dtype == "q4k" and shape[1] % 256 == 0:
            total += n // 256 * 144
        elif dtype == "bf16":
            total += n * 2
        else:
            total += n * 4
    return total


def voice_tensors(keys, values, pad_to: int = 0) -> dict:
    """Per-layer caches [1, kvh, len, hd] in the layout Voice::save writes (SVL/tts/voice.rs:76-99):
    "transformer.layers.{i}.self_attn/cache" [2, 1, time, kvh, hd] f32, "/offset" [len] i64 and
    "/pad" [0] i64; `pad_to` > len leaves seeded junk in the time rows past the offset."""
    out = {}
    for i, (k, v) in enumerate(zip(keys, values)):
        k = np.asarray(k, np.float32).reshape(k.shape[-3:])  # [kvh, len, hd]
        v = np.asarray(v, np.float32).reshape(v.shape[-3:])
        n = k.shape[1]
        t = max(pad_to, n)
        cache = _rng(7, f"voice.junk.{i}").standard_normal((2, 1, t, k.shape[0], k.shape[2]), dtype=np.float32)
        cache[0, 0, :n] = k.transpose(1, 0, 2)
        cache[1, 0, :n] = v.transpose(1, 0, 2)
        m = f"transformer.layers.{i}.self_attn"
        out[m + "/cache"] = (F32, cache.shape, cache)
        out[m + "/offset"] = (6, (1,), np.array([n], np.int64))
        out[m + "/pad"] = (6, (1,), np.array([0], np.int64))
    return out



# ---- the STT quantizer (SVL/stt/model.rs:84-174; Kyutai STT: 32 codebooks of 2048 entries) -------

RVQ_NQ, RVQ_BINS = 32, 2048


def rvq_weights(n_q: int = RVQ_NQ, bins: int = RVQ_BINS, seed: int = 0):
    """Seeded quantizer weights: input projections [256, 512] for the first and the rest quantizer,
    embedding sums [n_q, bins, 256] ~ N(0, 1) and cluster usages [n_q, bins] in [0.5, 4) (a few
    below the 1e-5 floor), stage order (the first quantizer's codebook, then the rest's)."""
    w_first = normal(seed, "rvq.w_first", (256, 512), 0.05)
    w_rest = normal(seed, "rvq.w_rest", (256, 512), 0.05)
    sums = normal(seed, "rvq.sums", (n_q, bins, 256), 1.0)
    usage = _rng(seed, "rvq.usage").uniform(0.5, 4.0, (n_q, bins)).astype(np.float32)
    usage[:, ::97] = np.float32(1e-7)
    return w_first, w_rest, sums, usage


def rvq_tensors(w_first, w_rest, sums, usage) -> dict:
    """The quantizer's tensors under the names svl_rvq_create reads (the checkpoint's, after its
    `quantizer.` prefix), input projections as [256, 512, 1] convolution weights."""
    out = {"rvq_first.input_proj.weight": (F32, (256, 512, 1), np.asarray(w_first, np.float32).reshape(256, 512, 1)),
           "rvq_rest.input_proj.weight": (F32, (256, 512, 1), np.asarray(w_rest, np.float32).reshape(256, 512, 1))}
    n_q, bins = sums.shape[0], sums.shape[1]
    for s in range(n_q):
        pre = "rvq_first.vq.layers.0._codebook." if s == 0 else f"rvq_rest.vq.layers.{s - 1}._codebook."
        out[pre + "embedding_sum"] = (F32, (bins, 256), np.ascontiguousarray(sums[s]))
        out[pre + "cluster_usage"] = (F32, (bins,), np.ascontiguousarray(usage[s]))
    return out


def rvq_latents(batch: int, frames: int, seed: int = 0) -> np.ndarray:
    """Seeded encoder latents [batch, 512, frames] ~ N(0, 1)."""
    return normal(seed, f"rvq.latents.{batch}.{frames}", (batch, 512, frames), 1.0)
