"""Decode-step benchmark of the streaming-transformer step on one MI355X.

Default workload (--workload stt1b-q8-b1): STT-1B shape (16 layers, d_model 2048, 16 heads x 128,
gated SiLU 5632, RMSNorm, window 750, text vocabulary 8000, 32 audio codebooks) with every
linear in candle Q8_0, bf16 embeddings, f32 KV cache, batch 1, greedy decoding from an empty
state.  A step is one decode step: embedding gather-sum, 16 layers, output norm, text_linear,
argmax, with the argmax fed back as the next text token on the device.  Inputs (weights, audio
tokens) are resident in HBM before timing.

Other workloads (one JSON line each, same fields):
  stt1b-q8-b64   64 lockstep streams, each ring pre-filled to a seeded fill in [1, 750], 128
                 steps; linears run as int8 MFMA GEMMs; a step advances all 64 streams.
  stt1b-bf16-b1  the default workload with bf16 linears (dense 16-lane-dot GEMV), 256 steps.
  stt2.6b-q4k-b1 STT-2.6B shape (24 layers, d_model 2560, 20 heads x 128, gated SiLU 6912, window
                 3000) with every linear in candle Q4K (activations quantized to Q8K), 256 steps.
  tts-f32-b1     Pocket-TTS backbone (6 layers, d 1024, 16 x 64, GELU 4096, LayerNorm), f32,
                 256 prefilled positions, 128 steps of seeded N(0, 1) latents; one call per step
                 (the reference returns to the host every frame).

Prints ONE JSON line (rank 0).  `value` is decode steps/s; `roofline` prices the dominant
kernel -- the step's phase kernels (phase_kernel; gemv_phase_kernel for the weight-streaming GEMVs;
attn_phase_kernel for attention; batch_phase_kernel for the batched MFMA path), launched once per phase of every step (83 launches per STT-1B step, 148
at B=64) -- against MI355X HBM bandwidth: `achieved` = algorithmic bytes per launch / average
launch time, i.e. the algorithmic bytes of the timed steps over their HIP-event time (which
also counts the gaps between launches); `traffic` is the HBM bytes per launch measured by
rocprofv3 counters on a run of the same workload (profiles/; `traffic_counter_steps` says how
many steps that run had); `cpu_baseline` is the oracle (this repository's C restatement of the
reference's CPU path) on the host cores.

`--calibrate-copy BYTES` instead runs the plain copy kernel of libsvl three times over BYTES
(the known-size reference that scales the traffic counters) and prints one JSON line.
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
WORKLOADS = ["stt1b-q8-b1", "stt1b-q8-b64", "stt1b-bf16-b1", "stt2.6b-q4k-b1", "tts-f32-b1"]


def traffic_file(workload):
    return os.path.join(ROOT, "profiles", f"phase_kernel.{workload.replace('-', '_')}.traffic.txt")


def read_traffic(workload):
    """(HBM bytes per phase_kernel launch, steps of the counter run) from the committed counter
    summary of this workload (FETCH_SIZE + WRITE_SIZE summed over the run's dispatches, scaled
    by the copy-kernel calibration, divided by the dispatches), or (None, None)."""
    path = traffic_file(workload)
    if not os.path.exists(path):
        return None, None
    kv = {}
    for line in open(path):
        if ":" in line and not line.lstrip().startswith("#"):
            k, v = line.split(":", 1)
            kv[k.strip()] = v.strip()
    try:
        return int(float(kv["hbm_bytes_per_launch"])), int(kv["steps"])
    except (KeyError, ValueError):
        return None, None


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


def stt_phases_per_step(shape, B, dtype):
    """Launches per STT step: embedding; per layer QKV, attention, out, FF-in, FF-out (each
    Q8_0 linear of a batch of 16 or more streams is an activation-quantization launch and a GEMM
    launch); text_linear (+ quantization) and argmax."""
    batched = dtype == "q8_0" and B >= 16
    per_layer = 5 + (4 if batched else 0)
    return 1 + shape.num_layers * per_layer + (2 if batched else 1) + 1


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


def base_line(value, steps, warmup, ms_per_step, dtype, data, config):
    return {"metric": "decode steps/s at B=1 and B=64 (STT-1B-shape, Q8_0); % of HBM roofline",
            "value": round(value, 2), "unit": "steps/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": data, "config": config}


def bench_stt(args, wl, steps, warmup):
    import svl
    from svl import hip
    from svl import workloads as W

    shape = W.S2 if wl == "stt2.6b-q4k-b1" else W.S1
    dtype = {"stt1b-bf16-b1": "bf16", "stt2.6b-q4k-b1": "q4k"}.get(wl, "q8_0")
    B = 64 if wl == "stt1b-q8-b64" else 1
    t0 = time.perf_counter()
    tensors = W.make_weights(shape, dtype, seed=0)
    print(f"weights generated in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    model = svl.Model(shape.config(W.quantize_code(dtype)), tensors, kv_dtype=svl.F32)
    audio = W.audio_tokens(shape, max(steps, args.cpu_steps), seed=1, batch=B)  # [B, n, n_q]
    d_audio = hip.DeviceBuffer.from_array(np.ascontiguousarray(audio[:, :steps].transpose(1, 0, 2)))
    d_out = hip.DeviceBuffer(steps * B * 4)
    st = model.init_state(batch=B)
    fills = [0] * B
    if B > 1:
        # each stream's ring pre-filled to a seeded fill in [1, window]; one seeded cache of the
        # full window is shared, each stream taking its first `fill` positions
        fills = [int(f) for f in np.random.default_rng(7).integers(1, shape.context + 1, size=B)]
        ks, vs = W.prefill_caches(shape, shape.context, seed=8)
        for b in range(B):
            st.load_stream(b, [k[:, :, :fills[b]] for k in ks], [v[:, :, :fills[b]] for v in vs])
        del ks, vs
        st.synchronize()
    gpu_ms, wall = timed_launch(model, st, steps, d_audio, d_out, warmup)
    print(f"timed {steps} steps: {gpu_ms:.2f} ms", file=sys.stderr, flush=True)
    bytes_launch = sum(step_bytes(shape, dtype, 4, [min(f + s + 1, shape.context) for f in fills])
                       for s in range(steps))
    achieved = bytes_launch / (gpu_ms / 1e3) / 1e9
    name = {"stt1b-q8-b1": "stt-1b q8_0 greedy decode, batch 1, from position 0",
            "stt1b-bf16-b1": "stt-1b bf16 greedy decode, batch 1, from position 0",
            "stt2.6b-q4k-b1": "stt-2.6b q4k greedy decode, batch 1, from position 0",
            "stt1b-q8-b64": "stt-1b q8_0 greedy decode, 64 lockstep streams, rings pre-filled to U[1, 750]"}[wl]
    config = {"workload": name, "layers": shape.num_layers, "d_model": shape.d_model, "heads": shape.num_heads,
              "head_dim": shape.head_dim, "ff_hidden": shape.ff_hidden, "window": shape.context,
              "text_vocab": shape.text_card, "codebooks": shape.n_q, "batch": B, "kv_dtype": "f32",
              "wall_s": round(wall, 4)}
    if B > 1:
        config["tokens_per_s"] = round(steps * B / (gpu_ms / 1e3), 1)
        config["mean_fill"] = round(float(np.mean(fills)), 1)
    dt = {"q8_0": "q8_0 (int8 x int8 -> int32 block dots, f32 scales and sums)",
          "q4k": "q4k x q8k (4-bit x int8 -> int32 sub-block dots, f32 scales and lane sums)",
          "bf16": "bf16 weights, f32 arithmetic (16-lane FMA dot)"}[dtype]
    line = base_line(steps / (gpu_ms / 1e3), steps, warmup, gpu_ms / steps, dt,
                     "synthetic (seeded N(0, 0.02) weights, uniform audio ids, greedy text feedback)", config)
    launches = steps * stt_phases_per_step(shape, B, dtype)
    traffic, traffic_steps = read_traffic(wl)
    line["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                        "traffic_counter_steps": traffic_steps,
                        "kernel": "step phase kernels (phase_kernel, gemv_phase_kernel, attn_phase_kernel, batch_phase_kernel; one launch per phase of each step)",
                        "launches": launches,
                        "algorithmic_bytes_per_launch": int(bytes_launch / launches),
                        "avg_launch_us": round(gpu_ms * 1e3 / launches, 3), "timed_ms": round(gpu_ms, 4)}
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_stt(args, shape, dtype, tensors, audio, fills, d_out, steps, B)
    return line


def cpu_stt(args, shape, dtype, tensors, audio, fills, d_out, steps, B):
    import oracle
    from svl import workloads as W

    oracle.set_threads(args.cpu_threads)
    m = oracle.Model(shape.config(W.quantize_code(dtype)), tensors)
    if B == 1:
        n = args.cpu_steps
        m.new_state().stt_greedy(audio[0, :2])  # warm-up
        st = m.new_state()
        t0 = time.perf_counter()
        toks = st.stt_greedy(audio[0, :n])
        dt = time.perf_counter() - t0
        gpu_toks = d_out.to_array(np.uint32, steps)[: min(n, steps)]
        return {"value": round(n / dt, 3), "unit": "steps/s", "cores": args.cpu_threads, "kind": "port",
                "sample": f"{n} greedy steps of the same workload from position 0 "
                          f"(oracle, {args.cpu_threads} threads)",
                "tokens_match": bool(np.array_equal(gpu_toks, toks[: gpu_toks.size]))}
    # batched: a sample of streams, two steps each at their fills, scaled to lockstep steps of B
    ns, n = 4, 2
    ks, vs = W.prefill_caches(shape, shape.context, seed=8)
    t_total = 0.0
    for b in range(ns):
        st = m.state_from_layer_caches([k[:, :, :fills[b]] for k in ks], [v[:, :, :fills[b]] for v in vs])
        t0 = time.perf_counter()
        st.stt_greedy(audio[b, :n])
        t_total += time.perf_counter() - t0
    return {"value": round(ns * n / t_total / B, 4), "unit": "steps/s", "cores": args.cpu_threads, "kind": "port",
            "sample": f"{ns} of the {B} streams x {n} steps each at their fills (oracle, {args.cpu_threads} "
                      f"threads), stream-steps/s divided by {B}"}


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
    print(f"timed {steps} steps: {wall * 1e3:.2f} ms (host loop)", file=sys.stderr, flush=True)
    bytes_total = sum(step_bytes(shape, "f32", 4, [257 + s]) for s in range(steps))
    achieved = bytes_total / wall / 1e9
    config = {"workload": "pocket-tts backbone f32, batch 1, 256 prefilled positions, one call per step",
              "layers": shape.num_layers, "d_model": shape.d_model, "heads": shape.num_heads,
              "head_dim": shape.head_dim, "ff_hidden": shape.ff_hidden, "batch": 1, "kv_dtype": "f32",
              "timing": f"host wall clock over the {steps} synchronous calls"}
    line = base_line(steps / wall, steps, warmup, wall * 1e3 / steps, "f32",
                     "synthetic (seeded N(0, 0.02) weights, N(0, 1) latents, seeded prefilled K/V)", config)
    line["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                        "kernel": "step phase kernels (phase_kernel, gemv_phase_kernel, attn_phase_kernel, batch_phase_kernel; one launch per phase; one call = one step)",
                        "algorithmic_bytes_per_step": int(bytes_total / steps)}
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
    ap.add_argument("--steps", type=int, default=0, help="timed steps (default 256; 128 for b64 and tts)")
    ap.add_argument("--warmup", type=int, default=-1, help="warm-up steps (default: as many as timed)")
    ap.add_argument("--cpu-steps", type=int, default=0, help="oracle steps (default 64; 16 for q4k)")
    ap.add_argument("--cpu-threads", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode step has no multi-GPU path "
              "(independent streams shard across GPUs with no communication).", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    wl = args.workload
    args.cpu_steps = args.cpu_steps or (16 if wl == "stt2.6b-q4k-b1" else 64)
    steps = args.steps or (128 if wl in ("stt1b-q8-b64", "tts-f32-b1") else 256)
    warmup = steps if args.warmup < 0 else args.warmup
    line = bench_tts(args, steps, warmup) if wl == "tts-f32-b1" else bench_stt(args, wl, steps, warmup)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
