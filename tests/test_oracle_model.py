"""Pins the oracle's transformer, KV cache and backbone steps.

  * transformer.rs:598-628  streaming == full sequence within 1e-4, chunks [1,3,1,7,1,1,9],
                            context None and Some(5) (d 16, 2 layers, 4/2 heads, hd 4,
                            LayerNorm, layer scale, tanh-GELU hidden 32, weights N(0, 0.3))
  * brute force             every output of a tiny model against a float64 textbook
                            transformer written here in numpy (pre-norm residual blocks,
                            q/k/v split in that order, interleaved RoPE, causal window, gated
                            SiLU with the gate first), for STT-, TTS- and bare configurations
  * state API               duplicate / from_layer_caches / layer caches continue identically
"""
import numpy as np
import pytest

import oracle
from svl import workloads as W


def tiny_shape(context, gated=False, rms=False, kvh=2, layer_scale=1):
    return W.Shape("tiny", W.MODEL_TRANSFORMER, 16, 2, 4, kvh, 4, W.FF_GATED if gated else W.FF_PLAIN,
                   32, W.NORM_RMS if rms else W.NORM_LAYER, 1e-8 if rms else 1e-5, context or 0,
                   layer_scale=layer_scale)


def random_tensors(shape, std=0.3, seed=0):
    """The reference test's VarMap weights: every tensor N(0, std)."""
    out = {}
    for name, shp, _ in W.tensor_names(shape):
        out[name] = (W.F32, shp, W.normal(seed, name, shp, std))
    return out


def np_transformer(shape, tensors, xs, pos0=0):
    """Float64 textbook forward of xs [T, d] at positions pos0.. (full causal sequence)."""
    c = shape
    T, d = xs.shape
    H, KVH, hd = c.num_heads, c.num_kv_heads, c.head_dim
    pre = "" if c.kind == W.MODEL_TRANSFORMER else "transformer."
    g = lambda n: tensors[pre + n][2].astype(np.float64).reshape(tensors[pre + n][1])
    x = xs.astype(np.float64)
    pos = pos0 + np.arange(T)
    inv = np.exp(-np.log(c.max_period) * 2 * np.arange(hd // 2) / hd)
    ang = pos[:, None] * inv[None, :]

    def norm(v, p):
        if c.norm_kind == W.NORM_RMS:
            a = g(p + ".alpha").reshape(-1)
            return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + c.norm_eps) * a
        mu = v.mean(-1, keepdims=True)
        return (v - mu) / np.sqrt(((v - mu) ** 2).mean(-1, keepdims=True) + c.norm_eps) * g(p + ".weight") + g(p + ".bias")

    def rope(v):  # v [heads, T, hd]
        z = (v[..., 0::2] + 1j * v[..., 1::2]) * np.exp(1j * ang)[None]
        out = np.empty_like(v)
        out[..., 0::2], out[..., 1::2] = z.real, z.imag
        return out

    for i in range(c.num_layers):
        p = f"layers.{i}."
        h = norm(x, p + "norm1")
        win = p + ("self_attn.in_proj_weight" if pre + p + "self_attn.in_proj_weight" in tensors else "self_attn.in_proj.weight")
        qkv = h @ g(win).T
        q = qkv[:, :H * hd].reshape(T, H, hd).transpose(1, 0, 2)
        k = qkv[:, H * hd:(H + KVH) * hd].reshape(T, KVH, hd).transpose(1, 0, 2)
        v = qkv[:, (H + KVH) * hd:].reshape(T, KVH, hd).transpose(1, 0, 2)
        q, k = rope(q), rope(k)
        k = np.repeat(k, H // KVH, axis=0)
        v = np.repeat(v, H // KVH, axis=0)
        s = q @ k.transpose(0, 2, 1) / np.sqrt(hd)
        qi, kj = np.meshgrid(np.arange(T), np.arange(T), indexing="ij")
        vis = (kj <= qi) & ((c.context == 0) | (qi - kj < (c.context or 1)))
        s = np.where(vis[None], s, -np.inf)
        w = np.exp(s - s.max(-1, keepdims=True))
        w /= w.sum(-1, keepdims=True)
        att = (w @ v).transpose(1, 0, 2).reshape(T, H * hd)
        upd = att @ g(p + "self_attn.out_proj.weight").T
        if c.layer_scale:
            upd = upd * g(p + "layer_scale_1.scale")
        x = x + upd
        h = norm(x, p + "norm2")
        if c.ff_kind == W.FF_GATED:
            hid = h @ g(p + "gating.linear_in.weight").T
            F = c.ff_hidden
            gate = hid[:, :F]
            upd = (gate / (1 + np.exp(-gate)) * hid[:, F:]) @ g(p + "gating.linear_out.weight").T
        else:
            hid = h @ g(p + "linear1.weight").T
            y = np.sqrt(2 / np.pi) * (hid + 0.044715 * hid ** 3)
            upd = (hid / (1 + np.exp(-2 * y))) @ g(p + "linear2.weight").T
        if c.layer_scale:
            upd = upd * g(p + "layer_scale_2.scale")
        x = x + upd
    return x


@pytest.mark.parametrize("context", [None, 5])
def test_streaming_matches_full_sequence(context):
    """transformer.rs:598-628."""
    shape = tiny_shape(context)
    m = oracle.Model(shape.config(0), random_tensors(shape))
    xs = np.random.default_rng(7).standard_normal((1, 23, 16)).astype(np.float32)
    full = m.new_state().forward(xs)
    st = m.new_state()
    chunks, start = [], 0
    for n in [1, 3, 1, 7, 1, 1, 9]:
        chunks.append(st.forward(xs[:, start:start + n]))
        start += n
    streamed = np.concatenate(chunks, axis=1)
    assert np.max(np.abs(full - streamed)) < 1e-4
    assert st.position == 23


@pytest.mark.parametrize("context,gated,rms,kvh", [(None, False, False, 2), (5, False, False, 4),
                                                   (6, True, True, 4), (0, True, True, 1)])
def test_brute_force_against_float64(context, gated, rms, kvh):
    shape = tiny_shape(context, gated, rms, kvh, layer_scale=0 if gated else 1)
    tensors = random_tensors(shape, 0.3, seed=11)
    m = oracle.Model(shape.config(0), tensors)
    xs = np.random.default_rng(8).standard_normal((1, 19, 16)).astype(np.float32)
    st = m.new_state()
    got = np.concatenate([st.forward(xs[:, i:i + 1]) for i in range(19)], axis=1)[0]
    expected = np_transformer(shape, tensors, xs[0])
    assert np.max(np.abs(got - expected)) < 2e-4 * max(1.0, np.abs(expected).max())


def test_window_cache_compaction_is_a_ring():
    """The compacting cache (transformer.rs:508-550) exposes the last `context` keys: after
    wrapping several times the state's caches equal a fresh state rebuilt from those keys."""
    shape = tiny_shape(5)
    m = oracle.Model(shape.config(0), random_tensors(shape))
    xs = np.random.default_rng(9).standard_normal((1, 40, 16)).astype(np.float32)
    st = m.new_state()
    for i in range(40):
        st.forward(xs[:, i:i + 1])
    k, v, start = st.cache(0)
    assert start + k.shape[2] == 40 and k.shape[2] >= 5
    # Rebuild from the last 5 keys only: next outputs are identical, since only they are visible.
    ks, vs = [], []
    for layer in range(shape.num_layers):
        kk, vv, s0 = st.cache(layer)
        ks.append(kk)
        vs.append(vv)
    a = st.duplicate()
    b = m.state_from_layer_caches(ks, vs)
    assert b.position == k.shape[2]  # from_layer_caches restarts positions at the cache length
    ya = a.forward(xs[:, :1])
    assert np.array_equal(ya, st.forward(xs[:, :1]))


def test_duplicate_and_from_layer_caches_continue_identically():
    shape = tiny_shape(None)
    m = oracle.Model(shape.config(0), random_tensors(shape))
    xs = np.random.default_rng(10).standard_normal((1, 12, 16)).astype(np.float32)
    st = m.new_state()
    st.forward(xs[:, :6])
    dup = st.duplicate()
    ks, vs = zip(*[(c[0], c[1]) for c in (st.cache(i) for i in range(2))])
    reb = m.state_from_layer_caches(list(ks), list(vs))
    y1 = st.forward(xs[:, 6:])
    assert np.array_equal(y1, dup.forward(xs[:, 6:]))
    assert np.array_equal(y1, reb.forward(xs[:, 6:]))


def test_stt_step_brute_force():
    """LanguageModel::step: text + audio embeddings summed, transformer, RMS out_norm 1e-8,
    text_linear, argmax (SVL/stt/model.rs:239-258) against float64."""
    s = W.stt_shape("stt-tiny", 64, 2, 2, 4.125, 6, card=10, n_q=3, text_card=20)
    tensors = W.make_weights(s, "f32", seed=3)
    m = oracle.Model(s.config(0), tensors)
    st = m.new_state()
    audio = W.audio_tokens(s, 9)[0]
    get = lambda n: tensors[n][2].astype(np.float64).reshape(tensors[n][1])
    xs, toks, logits_all = [], [], []
    text = s.text_card
    for i in range(9):
        tok, logits = st.stt_step(text, audio[i], want_logits=True)
        x = get("text_emb.weight")[text] + sum(get(f"emb.{c}.weight")[audio[i][c]] for c in range(s.n_q))
        xs.append(x)
        y = np_transformer(s, tensors, np.array(xs))[-1]
        y = y / np.sqrt((y ** 2).mean() + 1e-8) * get("out_norm.alpha").reshape(-1)
        ref = y @ get("text_linear.weight").T
        assert np.max(np.abs(logits - ref)) < 1e-4
        assert tok == int(np.argmax(logits))
        text = tok


def test_stt_extra_heads_brute_force():
    """LanguageModel::step's extra heads (SVL/stt/model.rs:217-222, 259-271): per head, the dense
    [dim, d] linear over the out_norm'ed output, softmax, probability of class 0 -- against float64.
    The heads leave the text tokens and logits unchanged."""
    base = W.stt_shape("stt-tiny", 64, 2, 2, 4.125, 6, card=10, n_q=3, text_card=20)
    s = W.Shape(**{**base.__dict__, "extra_heads_num": 4, "extra_heads_dim": 6})
    tensors = W.make_weights(s, "f32", seed=13)
    assert tensors["extra_heads.3.weight"][1] == (6, 64)
    m = oracle.Model(s.config(0), tensors)
    plain = oracle.Model(base.config(0), {k: v for k, v in tensors.items() if not k.startswith("extra_heads")})
    st, sp = m.new_state(), plain.new_state()
    audio = W.audio_tokens(s, 8, seed=2)[0]
    get = lambda n: tensors[n][2].astype(np.float64).reshape(tensors[n][1])
    xs, text = [], s.text_card
    for i in range(8):
        tok, logits, probs = st.stt_step(text, audio[i], want_logits=True, want_probs=True)
        tok_p, logits_p = sp.stt_step(text, audio[i], want_logits=True)
        assert tok == tok_p and np.array_equal(logits, logits_p)
        xs.append(get("text_emb.weight")[text] + sum(get(f"emb.{c}.weight")[audio[i][c]] for c in range(s.n_q)))
        y = np_transformer(s, tensors, np.array(xs))[-1]
        y = y / np.sqrt((y ** 2).mean() + 1e-8) * get("out_norm.alpha").reshape(-1)
        for h in range(4):
            lg = get(f"extra_heads.{h}.weight") @ y
            e = np.exp(lg - lg.max())
            assert abs(probs[h] - e[0] / e.sum()) < 1e-5, (i, h)
        text = tok
    # the greedy loop returns every step's probabilities, equal to the single steps'
    toks, pr = m.new_state().stt_greedy(audio, want_probs=True)
    st2, text = m.new_state(), s.text_card
    for i in range(8):
        a = np.full(s.n_q, s.card, np.uint32) if i == 0 else audio[i]
        t, p1 = st2.stt_step(text, a, want_probs=True)
        assert t == toks[i] and np.array_equal(p1, pr[i])
        text = t


def test_stt_greedy_initial_tokens_and_feedback():
    """Recognizer::step: step 0 sees `card` audio tokens and text_card; then the previous argmax."""
    s = W.S1_SMALL
    m = oracle.Model(s.config(W.Q8_0), W.make_weights(s, "q8_0", seed=5))
    audio = W.audio_tokens(s, 12)[0]
    toks = m.new_state().stt_greedy(audio)
    st = m.new_state()
    text = s.text_card
    for i in range(12):
        a = np.full(s.n_q, s.card, np.uint32) if i == 0 else audio[i]
        t = st.stt_step(text, a)
        assert t == toks[i]
        text = t


def test_tts_backbone_brute_force():
    """FlowLm::step backbone: latent or bos -> input_linear -> transformer -> LayerNorm 1e-5."""
    s = W.tts_shape("tts-tiny", 64, 2, 2, 128, latent=8)
    tensors = W.make_weights(s, "f32", seed=4)
    m = oracle.Model(s.config(0), tensors)
    st = m.new_state()
    lat = W.latents(s, 5)
    get = lambda n: tensors[n][2].astype(np.float64).reshape(tensors[n][1])
    ins = []
    for i in range(5):
        inp = get("bos_emb") if i == 0 else lat[i].astype(np.float64)
        z = st.tts_step(None if i == 0 else lat[i])
        ins.append(inp @ get("input_linear.weight").T)
        y = np_transformer(s, tensors, np.array(ins))[-1]
        mu = y.mean()
        ref = (y - mu) / np.sqrt(((y - mu) ** 2).mean() + 1e-5) * get("out_norm.weight") + get("out_norm.bias")
        assert np.max(np.abs(z - ref)) < 2e-4


def test_q8_0_linear_is_candle_matmul():
    """A Q8_0 model's linear = per-row activation quantization + vec_dot per output."""
    s = W.S1_SMALL
    t = W.make_weights(s, "q8_0", seed=6)
    m = oracle.Model(s.config(W.Q8_0), t)
    w = t["text_linear.weight"][2]
    blocks = oracle.quantize_q8_0(w)
    assert np.array_equal(m.linear_weight("text_linear", *w.shape), oracle.dequantize_q8_0(blocks, w.shape[1]))


def test_model_errors():
    s = W.S1_SMALL
    t = W.make_weights(s, "f32")
    bad = dict(t)
    del bad["emb.2.weight"]
    with pytest.raises(ValueError, match="emb.2.weight"):
        oracle.Model(s.config(0), bad)
    m = oracle.Model(s.config(0), t)
    with pytest.raises(ValueError, match="out of range"):
        m.new_state().stt_step(s.text_card + 1, np.zeros(s.n_q, np.uint32))


def test_norm_statistics_are_element_order_sums():
    """candle-nn's CPU rms_norm / layer_norm sum each row with one f32 accumulator in index
    order.  Row: 1.0 followed by 4096 copies of 2^-13.  In index order every square 2^-26 is
    absorbed (1 + 2^-26 rounds back to 1, half an ulp of 1 being 2^-24), so sum(x^2) = 1 and
    sum(x) = 1 + 4096 * 2^-13 = 1.5 (each 2^-13 is a multiple of ulp(1)); any order that adds the
    small squares before the 1.0 absorbs them (the 64-way blocked order, a tree, float64) gets a
    larger sum."""
    K = 1 + 4096
    x = np.full(K, 2.0 ** -13, dtype=np.float32)
    x[0] = 1.0
    alpha = np.ones(K, np.float32)
    sum2, sum1 = np.float32(1.0), np.float32(1.5)
    # RMSNorm: y = x / m, m = sqrt(sum2 / K + eps)
    m = np.sqrt(np.float32(sum2 / np.float32(K)) + np.float32(1e-8), dtype=np.float32)
    assert np.array_equal(oracle.rms_norm(x[None], alpha, 1e-8)[0].view(np.uint32), (x / m).view(np.uint32))
    oracle.set_norm_order("blocked")
    try:
        other = oracle.rms_norm(x[None], alpha, 1e-8)[0]
    finally:
        oracle.set_norm_order("element")
    assert np.all(other < x / m)  # a larger sum of squares, a smaller normalized row
    # LayerNorm: mean = sum1 / K, var = sum2 / K - mean^2, y = (x - mean) * (1 / sqrt(var + eps))
    w, b = np.ones(K, np.float32), np.zeros(K, np.float32)
    mean = np.float32(sum1 / np.float32(K))
    var = np.float32(np.float32(sum2 / np.float32(K)) - np.float32(mean * mean))
    inv = np.float32(np.float32(1.0) / np.sqrt(np.float32(var + np.float32(1e-5)), dtype=np.float32))
    expected = ((x - mean) * inv).astype(np.float32)
    assert np.array_equal(oracle.layer_norm(x[None], w, b, 1e-5)[0].view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("dtype,steps", [("q8_0", 200), ("q4k", 100)])
def test_norm_order_decides_quantized_greedy_tokens(dtype, steps):
    """With quantized activations the step is sensitive to the last bit of the norm statistic:
    summing the same squares in another order (the 64-way blocked order) changes the greedy
    tokens within these runs, while f32 weights keep them.  This is why the GPU kernels sum the
    statistics in candle's element order."""
    shape = W.S1_SMALL if dtype == "q8_0" else W.S2_SMALL
    m = oracle.Model(shape.config(W.quantize_code(dtype)), W.make_weights(shape, dtype, seed=0))
    audio = W.audio_tokens(shape, steps, seed=1)[0]
    try:
        oracle.set_norm_order("blocked")
        blocked = m.new_state().stt_greedy(audio)
    finally:
        oracle.set_norm_order("element")
    element = m.new_state().stt_greedy(audio)
    assert not np.array_equal(blocked, element)
