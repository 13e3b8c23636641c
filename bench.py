"""Decode-step benchmark of the streaming-transformer step on one MI355X.

The metric is decode steps/s at B = 1 and B = 64 on the STT-1B shape with Q8_0 linears (16 layers,
d_model 2048, 16 heads x 128, gated SiLU 5632, RMSNorm, window 750, text vocabulary 8000, 32 audio
codebooks; bf16 embeddings, f32 KV cache), as a fraction of the HBM roofline.  A step is one
decode step: embedding gather-sum, 16 layers, output norm, text_linear, argmax, the argmax fed
back as the next text token on the device.  Weights and token ids are synthetic and seeded;
inputs are resident in HBM before timing.

Default run (--workload stt1b-q8): ONE JSON line whose `value` is the B = 1 rate, with
  * the timed window placed so that its mean position is that of a 256-step greedy run from
    position 0 (the window starts at max(0, 128 - steps / 2); with --steps 256 it starts at 0):
    the visible keys per step, hence the bytes per step, are those of the 256-step config;
  * `steady_state`: the same step with the ring full (750 visible keys), a long-running stream;
  * `b64`: 64 lockstep streams, each ring pre-filled to a seeded fill in [1, 750] (MFMA GEMMs),
    with its own roofline and CPU baseline;
  * `roofline`: the dominant kernel of the B = 1 step -- the Q8_0 GEMV kernel instance
    gemv_phase_kernel<1u,4> (the step's GEMVs over rows of 2048) -- priced by the algorithmic
    bytes of its launches over their durations, each phase of the step replayed back to back
    on the state's stream and timed with HIP events (svl_bench_phase; the time includes the gap
    between consecutive launches); `step_roofline` prices the whole step (every launch, gaps
    included) the same way;
  * `cpu_baseline`: the oracle (this repository's C restatement of the reference's CPU path) on
    4 host threads (the reference's default) over a bounded sample, with its tokens compared
    to the GPU's, the CPU model and an all-cores figure;
  * `copy_ceiling`: libsvl's copy kernel over 1 GiB (read and written), the achievable HBM rate
    beside the vendor peak; each roofline also gives `frac_of_copy_ceiling`;
  * `read_floor` in each roofline that states its bytes per launch: the same bytes moved by a bare
    streaming read kernel launched back to back over cold buffers (the floor of any one launch of
    that size), and `frac_of_read_floor` = that floor's time / the kernel's time per launch.
Other workloads (--workload): stt1b-bf16-b1, stt2.6b-q4k-b1, tts-f32-b1 (one line each).

`--calibrate-copy BYTES` runs libsvl's plain copy kernel over BYTES three times (the known-size
reference that scales the traffic counters) and prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "semantic-ai_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
WORKLOADS = ["stt1b-q8", "stt1b-bf16-b1", "stt2.6b-q4k-b1", "tts-f32-b1"]
METRIC = "decode steps/s at B=1 and B=64 (STT-1B-shape, Q8_0); % of HBM roofline"
PH_EMBED, PH_GEMV, PH_ATTN, PH_ARGMAX, PH_QUANT, PH_QGEMM = 0, 1, 2, 4, 8, 9


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def traffic_file(name):
    return os.path.join(ROOT, "profiles", f"{name}.traffic.txt")


def read_traffic(name):
    """The committed counter summary of a workload (rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by the
    copy-kernel calibration): {"hbm_bytes_per_step", "steps", "per_kernel": {kernel group: HBM bytes
    per launch}} (lines `hbm_bytes_per_launch[<kernel group>]: N`), or {}."""
    path = traffic_file(name)
    if not os.path.exists(path):
        return {}
    kv = {}
    for line in open(path):
        if ":" in line and not line.lstrip().startswith("#"):
            k, v = line.split(":", 1)
            kv[k.strip()] = v.strip()
    out = {"per_kernel": {}}
    for k in ("hbm_bytes_per_step", "steps"):
        try:
            out[k] = int(float(kv[k]))
        except (KeyError, ValueError):
            pass
    for k, v in kv.items():
        if k.startswith("hbm_bytes_per_launch[") and k.endswith("]"):
            try:
                out["per_kernel"][k[len("hbm_bytes_per_launch["):-1]] = int(float(v))
            except ValueError:
                pass
    return out


def step_bytes(shape, dtype, kv_bytes, visible):
    """Algorithmic HBM bytes of one decode step: linear weights once, and for every stream the
    visible K/V it reads (`visible` = keys per stream), its written K/V row, its gathered
    embedding rows and the norm weights."""
    from svl import workloads as W

    d, L = shape.d_model, shape.num_layers
    kvw = shape.num_kv_heads * shape.head_dim
    w = W.linear_bytes(shape, dtype)
    emb = (1 + shape.n_q) * d * (4 if dtype == "f32" else 2) if shape.kind == W.MODEL_STT else 0
    norms = (2 * L + 1) * d * 4 * (2 if shape.norm_kind == W.NORM_LAYER else 1)
    per_stream = [L * (2 * v * kvw * kv_bytes + 2 * kvw * kv_bytes) + emb + norms for v in visible]
    return w + float(sum(per_stream))


def phase_bytes(info, shape, B, visible, kv_bytes=4):
    """Algorithmic HBM bytes of one launch of a step phase (svl_bench_phase's info): a GEMV's
    weights (in the format held on the device) and input rows; an attention launch's visible K/V;
    the embedding rows; the logits the argmax reads."""
    kind, fmt, rows, k = info[0], info[1], info[2], info[3]
    if kind in (PH_GEMV, PH_QGEMM):
        wb = {3: k // 32 * 34, 4: k // 256 * 144, 0: 4 * k, 5: 4 * k, 1: 2 * k, 6: 2 * k}[fmt]
        return rows * wb + B * k * 4
    if kind == PH_QUANT:
        return B * k * 5
    if kind == PH_ATTN:
        kvw = shape.num_kv_heads * shape.head_dim
        return sum(2 * v * kvw * kv_bytes for v in visible)
    if kind == PH_EMBED:
        return B * (1 + shape.n_q) * shape.d_model * 2
    if kind == PH_ARGMAX:
        return B * shape.text_card * 4
    return 0


def cpu_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count()


def calibrate_copy(nbytes):
    import svl
    from svl import hip

    L = svl.load_library()
    src, dst = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
    e0, e1 = hip.Event(), hip.Event()
    times = []
    for _ in range(3):
        e0.record(None)
        svl._check(L.svl_bench_copy(0, src.address, dst.address, nbytes, None))
        e1.record(None)
        hip.synchronize()
        times.append(e0.elapsed_ms(e1))
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "dispatches": 3,
                      "ms": [round(t, 4) for t in times],
                      "GBps_read_plus_write": round(2 * nbytes / (min(times) / 1e3) / 1e9, 1)}), flush=True)


def copy_ceiling(nbytes=1 << 30):
    """The achievable HBM rate of a plain kernel: libsvl's copy kernel over `nbytes` (read and
    written), best of three after one warm-up, HIP events."""
    import svl
    from svl import hip

    L = svl.load_library()
    src, dst = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
    e0, e1 = hip.Event(), hip.Event()
    best = None
    for i in range(4):
        e0.record(None)
        svl._check(L.svl_bench_copy(0, src.address, dst.address, nbytes, None))
        e1.record(None)
        hip.synchronize()
        if i:
            t = e0.elapsed_ms(e1)
            best = t if best is None else min(best, t)
    del src, dst
    gbs = 2 * nbytes / (best / 1e3) / 1e9
    return {"GBps": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes_read": nbytes,
            "bytes_written": nbytes, "kernel": "libsvl copy kernel (16-byte loads and stores)"}


READ_SHAPES = [(256, 1024), (512, 512), (512, 1024), (1024, 512), (2048, 256)]


def read_floor(bytes_per_launch, total=1 << 30):
    """The per-launch floor of moving `bytes_per_launch` bytes: libsvl's bare streaming read kernel
    launched back to back over distinct buffers of that size (together at least `total` bytes,
    more than every cache, so each launch reads cold bytes as the step's kernels do), for several
    grid shapes; HIP events over three passes after one warm-up pass.  Returns the best shape."""
    import svl
    from svl import hip

    L = svl.load_library()
    b = -(-int(bytes_per_launch) // 256) * 256
    nb = max(2, -(-total // b))
    buf, out = hip.DeviceBuffer(b * nb), hip.DeviceBuffer(4 * max(bl * th for bl, th in READ_SHAPES))
    e0, e1 = hip.Event(), hip.Event()
    best = None
    for blocks, threads in READ_SHAPES:
        def one_pass():
            for i in range(nb):
                svl._check(L.svl_bench_read(0, buf.address + i * b, b, blocks, threads, out.address, None))
        one_pass()
        e0.record(None)
        for _ in range(3):
            one_pass()
        e1.record(None)
        hip.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / (3 * nb)
        if best is None or us < best[0]:
            best = (us, blocks, threads)
    del buf, out
    us, blocks, threads = best
    gbs = b / (us / 1e6) / 1e9
    return {"us_per_launch": round(us, 3), "GBps": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_launch": b, "buffers": nb, "grid": [blocks, threads],
            "kernel": "libsvl bare read kernel (non-temporal 16-byte loads), back to back over cold buffers"}


def timed_launch(model, st, n, d_audio, d_out, warmup):
    """Warm-up launches of the same size from the same start (on copies of `st`), then one
    timed launch of n steps on another copy; returns (gpu_ms, wall_s)."""
    from svl import hip

    for _ in range(max(1, -(-warmup // n)) if warmup > 0 else 0):
        w = st.duplicate()
        model.recognize_async(n, d_audio.address, d_out.address, w)
        w.synchronize()
    run = st.duplicate()
    run.synchronize()
    hip.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    t0 = time.perf_counter()
    e0.record(run.stream)
    model.recognize_async(n, d_audio.address, d_out.address, run)
    e1.record(run.stream)
    run.synchronize()
    return e0.elapsed_ms(e1), time.perf_counter() - t0


def roofline_obj(achieved_gbs, traffic=None, **extra):
    r = {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(achieved_gbs / HBM_PEAK_GBS, 4), "traffic": traffic}
    r.update(extra)
    return r


def phase_table(model, st, shape, B, visible, program=0, reps=40):
    """Every phase of the state's step program replayed `reps` times back to back (on a copy of
    the state): [(index, info, us_per_launch, algorithmic bytes)]."""
    import ctypes as C

    import svl

    L = svl.load_library()
    dup = st.duplicate()
    out = []
    i = 0
    while True:
        us = C.c_float()
        info = (C.c_int * 6)()
        rc = L.svl_bench_phase(model.h, dup.h, program, i, reps, C.byref(us), info)
        if rc == svl.ERR_INVALID_INPUT and i > 0:
            break
        svl._check(rc)
        inf = list(info)
        out.append((i, inf, us.value, phase_bytes(inf, shape, B, visible)))
        i += 1
    dup.close()
    return out


def kernel_roofline(table, pick, name):
    """The roofline of one kernel instance: the algorithmic bytes of its launches in a step over
    their replayed durations."""
    sel = [(us, b) for _, inf, us, b in table if pick(inf)]
    if not sel:
        return None
    t = sum(us for us, _ in sel)
    b = sum(b for _, b in sel)
    return {"kernel": name, "launches_per_step": len(sel), "algorithmic_bytes_per_launch": int(b / len(sel)),
            "avg_launch_us": round(t / len(sel), 3), "achieved_gbs": b / (t * 1e-6) / 1e9,
            "share_of_replayed_step": None}


# The kernel groups a step's replayed phases are sorted into (svl_bench_phase's info: kind, weight
# format, rows, input width); the names key the committed traffic files' per-kernel entries.
KERNEL_GROUPS = {
    "gemv_phase_kernel<1u,4> (Q8_0 GEMV, input rows <= 2048)": lambda i: i[0] == PH_GEMV and i[1] == 3 and i[3] <= 2048,
    "gemv_phase_kernel<1u,16> (Q8_0 GEMV, input rows > 4096)": lambda i: i[0] == PH_GEMV and i[1] == 3 and i[3] > 4096,
    "gemv_phase_kernel<2u,*> (Q4K GEMV)": lambda i: i[0] == PH_GEMV and i[1] == 4,
    "gemv_phase_kernel<4u,*> (dense GEMV)": lambda i: i[0] == PH_GEMV and i[1] in (0, 1, 5, 6),
    "attn_phase_kernel (attention)": lambda i: i[0] == PH_ATTN,
    "batch_phase_kernel (MFMA int8 GEMM)": lambda i: i[0] == PH_QGEMM,
    "batch_phase_kernel (activation quantization)": lambda i: i[0] == PH_QUANT,
    "phase_kernel (embedding, argmax, other)": lambda i: i[0] not in (PH_GEMV, PH_ATTN, PH_QGEMM, PH_QUANT),
}


def dominant_roofline(table, B):
    """Roofline of the kernel group with the largest share of the replayed step (the Q8_0 GEMV
    over rows of 2048, gemv_phase_kernel<1u,4>, at B = 1; the attention or the MFMA GEMM at
    B = 64, within a percent of each other).  Also the shares of every group."""
    total = sum(us for _, _, us, _ in table)
    shares = {}
    best = None
    for name, pick in KERNEL_GROUPS.items():
        r = kernel_roofline(table, pick, name)
        if r is None:
            continue
        t = r["avg_launch_us"] * r["launches_per_step"]
        r["share_of_replayed_step"] = round(t / total, 3)
        shares[name] = r
        if best is None or t > best[0]:
            best = (t, r)
    return best[1], shares


def stt_model(shape, dtype):
    import svl
    from svl import workloads as W

    t0 = time.perf_counter()
    tensors = W.make_weights(shape, dtype, seed=0)
    log(f"weights generated in {time.perf_counter() - t0:.1f} s")
    model = svl.Model(shape.config(W.quantize_code(dtype)), tensors, kv_dtype=svl.F32)
    return tensors, model


def bench_b1(args, shape, dtype, tensors, model, steps, warmup, with_steady=True):
    """B = 1 greedy decode: the timed window of `steps` steps starts at position p0, reached by
    untimed greedy steps of the same stream."""
    import svl
    from svl import hip
    from svl import workloads as W

    p0 = max(0, int(round(127.5 - (steps - 1) / 2)))
    audio = W.audio_tokens(shape, max(p0 + steps, args.cpu_steps), seed=1)[0]  # [>= p0 + steps, n_q]
    st = model.init_state()
    pre = model.recognize(audio[:p0, None, :], st) if p0 else np.zeros((0, 1), np.uint32)
    d_audio = hip.DeviceBuffer.from_array(np.ascontiguousarray(audio[p0:p0 + steps, None, :]))
    d_out = hip.DeviceBuffer(steps * 4)
    gpu_ms, wall = timed_launch(model, st, steps, d_audio, d_out, warmup)
    toks = np.concatenate([pre[:, 0], d_out.to_array(np.uint32, steps)])
    log(f"B=1: {steps} steps from position {p0}: {gpu_ms:.2f} ms")
    visible = [[min(p + 1, shape.context)] for p in range(p0, p0 + steps)]
    sb = sum(step_bytes(shape, dtype, 4, v) for v in visible)
    res = {"steps_per_s": steps / (gpu_ms / 1e3), "ms_per_step": gpu_ms / steps, "gpu_ms": gpu_ms, "wall": wall,
           "p0": p0, "tokens": toks, "audio": audio, "bytes": sb}
    # per-phase replay at the window's middle position
    mid = model.init_state()
    if p0 + steps // 2:
        model.recognize(audio[: p0 + steps // 2, None, :], mid)
    vis_mid = [min(p0 + steps // 2 + 1, shape.context)]
    res["table"] = phase_table(model, mid, shape, 1, vis_mid)
    mid.close()
    if with_steady:
        # the ring full: 750 seeded keys, then `steps` timed steps
        ks, vs = W.prefill_caches(shape, shape.context, seed=3)
        full = model.init_state()
        full.load_stream(0, ks, vs)
        del ks, vs
        gms, _ = timed_launch(model, full, steps, d_audio, d_out, warmup)
        vb = step_bytes(shape, dtype, 4, [shape.context])
        res["steady"] = {"steps_per_s": round(steps / (gms / 1e3), 2), "ms_per_step": round(gms / steps, 4),
                         "visible_keys": shape.context,
                         "roofline_frac": round(vb * steps / (gms / 1e3) / 1e9 / HBM_PEAK_GBS, 4)}
        full.close()
    st.close()
    return res


def cpu_b1(args, shape, dtype, tensors, res):
    """The oracle from position 0 through the GPU's timed window (at least 64 steps): steps/s on
    4 threads and on all cores, tokens compared with the GPU's."""
    import oracle
    from svl import workloads as W

    audio = res["audio"]
    n = min(len(res["tokens"]), args.cpu_steps)  # through the GPU's timed window, bounded
    m = oracle.Model(shape.config(W.quantize_code(dtype)), tensors)
    model_name, nproc = cpu_info()
    out = {}
    for threads in (args.cpu_threads, min(16, nproc or 1)):
        oracle.set_threads(threads)
        m.new_state().stt_greedy(audio[:2])  # warm-up
        t0 = time.perf_counter()
        toks = m.new_state().stt_greedy(audio[:n])
        out[threads] = (n / (time.perf_counter() - t0), toks)
    value, toks = out[args.cpu_threads]
    k = min(len(toks), len(res["tokens"]))
    return {"value": round(value, 3), "unit": "steps/s", "cores": args.cpu_threads, "kind": "port",
            "sample": f"{n} greedy steps of the same stream from position 0 (the GPU's timed window is steps "
                      f"{res['p0']} .. {len(res['tokens']) - 1}; oracle, {args.cpu_threads} threads, the reference's "
                      f"default)",
            "tokens_match": bool(np.array_equal(toks[:k], res["tokens"][:k])), "tokens_compared": int(k),
            "cpu_model": model_name, "nproc": nproc,
            "all_cores": {"threads": min(16, nproc or 1), "value": round(out[min(16, nproc or 1)][0], 3)}}


def bench_b64(args, shape, dtype, tensors, model, steps, warmup):
    """64 lockstep streams, rings pre-filled to seeded fills in [1, window]."""
    from svl import hip
    from svl import workloads as W

    B = 64
    fills = [int(f) for f in np.random.default_rng(7).integers(1, shape.context + 1, size=B)]
    ks, vs = W.prefill_caches(shape, shape.context, seed=8)
    st = model.init_state(batch=B)
    for b in range(B):
        st.load_stream(b, [k[:, :, :fills[b]] for k in ks], [v[:, :, :fills[b]] for v in vs])
    st.synchronize()
    audio = W.audio_tokens(shape, steps, seed=1, batch=B)  # [B, n, n_q]
    d_audio = hip.DeviceBuffer.from_array(np.ascontiguousarray(audio.transpose(1, 0, 2)))
    d_out = hip.DeviceBuffer(steps * B * 4)
    gpu_ms, wall = timed_launch(model, st, steps, d_audio, d_out, warmup)
    log(f"B=64: {steps} steps: {gpu_ms:.2f} ms")
    toks = d_out.to_array(np.uint32, steps * B).reshape(steps, B)
    sb = sum(step_bytes(shape, dtype, 4, [min(f + s + 1, shape.context) for f in fills]) for s in range(steps))
    mid = [min(f + steps // 2 + 1, shape.context) for f in fills]
    table = phase_table(model, st, shape, B, mid, reps=10)
    st.close()
    dom, shares = dominant_roofline(table, B)
    achieved = sb / (gpu_ms / 1e3) / 1e9
    out = {"value": round(steps / (gpu_ms / 1e3), 2), "unit": "lockstep steps/s",
           "tokens_per_s": round(steps * B / (gpu_ms / 1e3), 1), "ms_per_step": round(gpu_ms / steps, 4),
           "steps": steps, "warmup": warmup, "batch": B, "mean_fill": round(float(np.mean(fills)), 1),
           "roofline": roofline_obj(dom["achieved_gbs"], kernel=dom["kernel"],
                                    launches_per_step=dom["launches_per_step"],
                                    algorithmic_bytes_per_launch=dom["algorithmic_bytes_per_launch"],
                                    avg_launch_us=dom["avg_launch_us"]),
           "step_roofline": roofline_obj(achieved, algorithmic_bytes_per_step=int(sb / steps)),
           "kernel_shares": {k: {"share": v["share_of_replayed_step"], "avg_launch_us": v["avg_launch_us"],
                                 "GBps": round(v["achieved_gbs"], 1)} for k, v in shares.items()}}
    tr = read_traffic("stt1b_q8_b64")
    out["roofline"]["traffic"] = tr.get("per_kernel", {}).get(dom["kernel"])
    out["step_roofline"]["traffic"] = tr.get("hbm_bytes_per_step")
    out["step_roofline"]["traffic_counter_steps"] = tr.get("steps")
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_b64(args, shape, dtype, tensors, fills, ks, vs, audio, toks)
    return out


def cpu_b64(args, shape, dtype, tensors, fills, ks, vs, audio, gpu_toks):
    import oracle
    from svl import workloads as W

    oracle.set_threads(args.cpu_threads)
    m = oracle.Model(shape.config(W.quantize_code(dtype)), tensors)
    ns, n = 8, min(4, gpu_toks.shape[0])
    t_total, match = 0.0, True
    for b in range(ns):
        st = m.state_from_layer_caches([k[:, :, :fills[b]] for k in ks], [v[:, :, :fills[b]] for v in vs])
        t0 = time.perf_counter()
        toks = st.stt_greedy(audio[b, :n])
        t_total += time.perf_counter() - t0
        match &= bool(np.array_equal(toks, gpu_toks[:n, b]))
    return {"value": round(ns * n / t_total / 64, 4), "unit": "lockstep steps/s", "cores": args.cpu_threads,
            "kind": "port", "tokens_match": match, "streams_compared": ns,
            "sample": f"{ns} of the 64 streams x {n} steps each from their fills (oracle, {args.cpu_threads} "
                      f"threads); stream-steps/s divided by 64"}


def counter_run(args, steps):
    """One launch of `steps` steps at B = 1 from position 0 and (unless --no-b64) one at B = 64 from
    the seeded fills, nothing else: every step-kernel dispatch of a counter run belongs to them."""
    from svl import hip
    from svl import workloads as W

    shape = W.S1
    _, model = stt_model(shape, "q8_0")
    out = {"counter_run": True, "steps": steps}
    if not args.no_b1:
        audio = W.audio_tokens(shape, steps, seed=1)[0]
        d_audio = hip.DeviceBuffer.from_array(np.ascontiguousarray(audio[:, None, :]))
        d_out = hip.DeviceBuffer(steps * 4)
        st = model.init_state()
        model.recognize_async(steps, d_audio.address, d_out.address, st)
        st.synchronize()
        out["b1_algorithmic_bytes_per_step"] = sum(step_bytes(shape, "q8_0", 4, [min(p + 1, shape.context)])
                                                   for p in range(steps)) / steps
        st.close()
    if not args.no_b64:
        B = 64
        fills = [int(f) for f in np.random.default_rng(7).integers(1, shape.context + 1, size=B)]
        ks, vs = W.prefill_caches(shape, shape.context, seed=8)
        st = model.init_state(batch=B)
        for b in range(B):
            st.load_stream(b, [k[:, :, :fills[b]] for k in ks], [v[:, :, :fills[b]] for v in vs])
        st.synchronize()
        audio = W.audio_tokens(shape, steps, seed=1, batch=B)
        d_audio = hip.DeviceBuffer.from_array(np.ascontiguousarray(audio.transpose(1, 0, 2)))
        d_out = hip.DeviceBuffer(steps * B * 4)
        model.recognize_async(steps, d_audio.address, d_out.address, st)
        st.synchronize()
        out["b64_algorithmic_bytes_per_step"] = sum(
            step_bytes(shape, "q8_0", 4, [min(f + s + 1, shape.context) for f in fills]) for s in range(steps)) / steps
    print(json.dumps(out), flush=True)


def base_line(value, steps, warmup, ms_per_step, dtype, data, config):
    return {"metric": METRIC, "value": round(value, 2), "unit": "steps/s", "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": data, "config": config}


DTYPES = {"q8_0": "q8_0 (int8 x int8 -> int32 block dots, f32 scales and sums)",
          "q4k": "q4k x q8k (4-bit x int8 -> int32 sub-block dots, f32 scales and lane sums)",
          "bf16": "bf16 weights, f32 arithmetic (16-lane FMA dot)"}
DATA = "synthetic (seeded N(0, 0.02) weights, uniform audio ids, greedy text feedback)"


def stt_config(shape, name, B, p0, steps):
    return {"workload": name, "layers": shape.num_layers, "d_model": shape.d_model, "heads": shape.num_heads,
            "head_dim": shape.head_dim, "ff_hidden": shape.ff_hidden, "window": shape.context,
            "text_vocab": shape.text_card, "codebooks": shape.n_q, "batch": B, "kv_dtype": "f32",
            "start_position": p0, "mean_visible_keys": round(
                float(np.mean([min(p + 1, shape.context) for p in range(p0, p0 + steps)])), 1)}


def b1_line(args, shape, dtype, tensors, model, steps, warmup, name, traffic_name):
    res = bench_b1(args, shape, dtype, tensors, model, steps, warmup, with_steady=dtype == "q8_0")
    cfg = stt_config(shape, name, 1, res["p0"], steps)
    cfg["wall_s"] = round(res["wall"], 4)
    line = base_line(res["steps_per_s"], steps, warmup, res["ms_per_step"], DTYPES[dtype], DATA, cfg)
    dom, shares = dominant_roofline(res["table"], 1)
    tr = read_traffic(traffic_name)
    traffic, tsteps = tr.get("hbm_bytes_per_step"), tr.get("steps")
    line["roofline"] = roofline_obj(dom["achieved_gbs"], traffic=tr.get("per_kernel", {}).get(dom["kernel"]),
                                    traffic_counter_steps=tsteps, kernel=dom["kernel"],
                                    launches_per_step=dom["launches_per_step"],
                                    algorithmic_bytes_per_launch=dom["algorithmic_bytes_per_launch"],
                                    avg_launch_us=dom["avg_launch_us"],
                                    timing="each phase replayed back to back on the state's stream, HIP events "
                                           "(includes the gap between launches)")
    achieved = res["bytes"] / (res["gpu_ms"] / 1e3) / 1e9
    line["step_roofline"] = roofline_obj(achieved, traffic=traffic, traffic_counter_steps=tsteps,
                                         algorithmic_bytes_per_step=int(res["bytes"] / steps),
                                         launches_per_step=len(res["table"]),
                                         timing="the timed launch's HIP events: every phase launch of the steps, "
                                                "gaps included")
    line["kernel_shares"] = {k: {"share": v["share_of_replayed_step"], "avg_launch_us": v["avg_launch_us"],
                                 "GBps": round(v["achieved_gbs"], 1)} for k, v in shares.items()}
    if "steady" in res:
        line["steady_state"] = res["steady"]
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_b1(args, shape, dtype, tensors, res)
    return line


def bench_tts(args, steps, warmup):
    import svl
    from svl import hip
    from svl import workloads as W

    shape = W.T1
    tensors = W.make_weights(shape, "f32", seed=0)
    model = svl.Model(shape.config(0), tensors, kv_dtype=svl.F32)
    ks, vs = W.prefill_caches(shape, 256, seed=3)
    lat = W.latents(shape, max(steps, 2), seed=4)
    cap = 256 + steps + 8
    w = model.state_from_layer_caches(ks, vs, capacity=cap)
    for i in range(min(warmup, steps)):
        model.backbone_step(lat[i][None], w)
    st = model.state_from_layer_caches(ks, vs, capacity=cap)
    st.synchronize()
    hip.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        model.backbone_step(lat[i][None], st)
    wall = time.perf_counter() - t0
    log(f"timed {steps} steps: {wall * 1e3:.2f} ms (host loop)")
    bytes_total = sum(step_bytes(shape, "f32", 4, [257 + s]) for s in range(steps))
    achieved = bytes_total / wall / 1e9
    config = {"workload": "pocket-tts backbone f32, batch 1, 256 prefilled positions, one call per step",
              "layers": shape.num_layers, "d_model": shape.d_model, "heads": shape.num_heads,
              "head_dim": shape.head_dim, "ff_hidden": shape.ff_hidden, "batch": 1, "kv_dtype": "f32",
              "timing": f"host wall clock over the {steps} synchronous calls"}
    line = base_line(steps / wall, steps, warmup, wall * 1e3 / steps, "f32",
                     "synthetic (seeded N(0, 0.02) weights, N(0, 1) latents, seeded prefilled K/V)", config)
    line["roofline"] = roofline_obj(achieved, kernel="the step's phase kernels, one call per step (host loop)",
                                    algorithmic_bytes_per_step=int(bytes_total / steps))
    # the whole FlowLm step on the device (backbone, out_eos, one flow-head decode step): frames
    # enqueued with device pointers, each fed the previous frame's latent and the sampler's
    # pre-drawn noise, no host round trip; HIP events on the state's stream
    ld = shape.latent_dim
    d_noise = hip.DeviceBuffer.from_array(np.ascontiguousarray(W.latents(shape, steps, seed=5)))
    d_lat = [hip.DeviceBuffer(ld * 4), hip.DeviceBuffer(ld * 4)]
    d_eos = hip.DeviceBuffer(steps * 4)

    def frames(stv, n):
        for f in range(n):
            model.tts_step_async(0 if f == 0 else d_lat[(f - 1) % 2].address, d_noise.address + f * ld * 4, 1,
                                 d_lat[f % 2].address, d_eos.address + f * 4, stv)

    wst = model.state_from_layer_caches(ks, vs, capacity=cap)
    frames(wst, max(1, min(warmup, steps)))
    wst.synchronize()
    sd = model.state_from_layer_caches(ks, vs, capacity=cap)
    sd.synchronize()
    hip.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(sd.stream)
    frames(sd, steps)
    e1.record(sd.stream)
    sd.synchronize()
    dms = e0.elapsed_ms(e1)
    flow_bytes = sum(int(np.prod(sh)) * 4 for name, sh, _ in W.tensor_names(shape) if name.startswith("flow_net."))
    dev_bytes = bytes_total + steps * flow_bytes
    line["device_loop"] = {
        "value": round(steps / (dms / 1e3), 2), "unit": "frames/s", "ms_per_frame": round(dms / steps, 4),
        "workload": "FlowLm::step whole (backbone, out_eos, one flow-head decode step) with svl_tts_step_async, "
                    "latents fed back on the device",
        "roofline": roofline_obj(dev_bytes / (dms / 1e3) / 1e9, kernel="every launch of the frames (HIP events)",
                                 algorithmic_bytes_per_step=int(dev_bytes / steps))}
    log(f"device loop: {steps} frames: {dms:.2f} ms")
    if not args.no_cpu_baseline:
        import oracle

        oracle.set_threads(args.cpu_threads)
        m = oracle.Model(shape.config(0), tensors)
        o = m.state_from_layer_caches(ks, vs)
        n = min(32, steps)
        t0 = time.perf_counter()
        for i in range(n):
            o.tts_step(lat[i])
        dt = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(n / dt, 3), "unit": "steps/s", "cores": args.cpu_threads,
                                "kind": "port",
                                "sample": f"{n} backbone steps after the same 256 prefilled positions "
                                          f"(oracle, {args.cpu_threads} threads)"}
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=WORKLOADS, default=WORKLOADS[0])
    ap.add_argument("--steps", type=int, default=0, help="timed steps (default 256; 128 for B=64 and tts)")
    ap.add_argument("--warmup", type=int, default=-1, help="warm-up steps (default: as many as timed)")
    ap.add_argument("--cpu-steps", type=int, default=0,
                    help="oracle steps at B=1 (default 256 for q8_0, 128 for bf16, 32 for q4k)")
    ap.add_argument("--cpu-threads", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-b64", action="store_true", help="skip the B=64 part of the default workload")
    ap.add_argument("--no-b1", action="store_true", help="counter runs: skip the B=1 launch")
    ap.add_argument("--counter-run", action="store_true",
                    help="one launch per batch size and nothing else (for rocprofv3 counter runs)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode step has no multi-GPU path "
              "(independent streams shard across GPUs with no communication).", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    if args.counter_run:
        counter_run(args, args.steps or 16)
        return
    from svl import workloads as W

    wl = args.workload
    if wl == "tts-f32-b1":
        steps = args.steps or 128
        line = bench_tts(args, steps, steps if args.warmup < 0 else args.warmup)
    elif wl == "stt1b-q8":
        args.cpu_steps = args.cpu_steps or 256
        steps = args.steps or 256
        warmup = steps if args.warmup < 0 else args.warmup
        tensors, model = stt_model(W.S1, "q8_0")
        line = b1_line(args, W.S1, "q8_0", tensors, model, steps, warmup,
                       "stt-1b q8_0 greedy decode, batch 1", "stt1b_q8_b1")
        if not args.no_b64:
            s64 = args.steps or 128
            line["b64"] = bench_b64(args, W.S1, "q8_0", tensors, model, s64, s64 if args.warmup < 0 else args.warmup)
    else:
        shape = W.S2 if wl == "stt2.6b-q4k-b1" else W.S1
        dtype = "q4k" if wl == "stt2.6b-q4k-b1" else "bf16"
        steps = args.steps or 256
        warmup = steps if args.warmup < 0 else args.warmup
        args.cpu_steps = args.cpu_steps or (32 if dtype == "q4k" else 128)
        tensors, model = stt_model(shape, dtype)
        name = f"{shape.name} {dtype} greedy decode, batch 1"
        line = b1_line(args, shape, dtype, tensors, model, steps, warmup, name, wl.replace("-", "_"))
    # the achievable ceiling beside the vendor peak: the dominant kernel's rate as a fraction of it
    line["copy_ceiling"] = copy_ceiling()
    for r in [line.get("roofline")] + ([line["b64"].get("roofline")] if "b64" in line else []):
        if r:
            r["frac_of_copy_ceiling"] = round(r["achieved"] / line["copy_ceiling"]["GBps"], 4)
        # the same bytes per launch moved by a bare read kernel, launch after launch: the floor of
        # any one launch of this size, gap included like the kernel's own figure
        if r and r.get("algorithmic_bytes_per_launch") and r.get("avg_launch_us"):
            r["read_floor"] = read_floor(r["algorithmic_bytes_per_launch"])
            r["frac_of_read_floor"] = round(r["read_floor"]["us_per_launch"] / r["avg_launch_us"], 4)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
