"""Decode-step benchmark of the streaming-transformer step on one MI355X.

Default workload: STT-1B shape (16 layers, d_model 2048, 16 heads x 128, gated SiLU 5632,
RMSNorm, window 750, text vocabulary 8000, 32 audio codebooks) with every linear in candle
Q8_0, batch 1, greedy decoding from an empty state.  A step is one decode step: embedding
gather-sum, 16 layers, output norm, text_linear, argmax, with the argmax fed back as the next
text token on the device.  Inputs (weights, audio tokens) are resident in HBM before timing.

Prints ONE JSON line (rank 0).  `value` is decode steps/s; `roofline` prices the dominant
kernel -- the persistent step-program kernel, one launch of which runs all the timed steps --
against MI355X HBM bandwidth with the algorithmic bytes of the steps it ran; its `traffic` is the
HBM bytes of that launch as measured by rocprofv3 counters (profiles/), when the profiled launch
had the same number of steps; `cpu_baseline` is the oracle (this repository's C restatement of
the reference's CPU path) on the host cores.

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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "step_program_kernel.stt1b_q8_0_b1.traffic.txt")


def read_traffic(steps):
    """HBM bytes of one step-program launch of `steps` steps, from the committed counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy-kernel calibration), or
    None when no summary for that launch size exists."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    kv = {}
    for line in open(TRAFFIC_FILE):
        if ":" in line and not line.lstrip().startswith("#"):
            k, v = line.split(":", 1)
            kv[k.strip()] = v.strip()
    try:
        if int(kv["steps_per_dispatch"]) != steps:
            return None
        return int(float(kv["hbm_bytes_per_dispatch"]))
    except (KeyError, ValueError):
        return None


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


def step_bytes(shape, dtype, kv_bytes, positions, window):
    """Algorithmic HBM bytes of one decode step per stream at each position in `positions`:
    linear weights + visible K/V reads + K/V write + gathered embedding rows + norm weights."""
    from svl import workloads as W

    d, L = shape.d_model, shape.num_layers
    kvw = shape.num_kv_heads * shape.head_dim
    w = W.linear_bytes(shape, dtype)
    emb = (1 + shape.n_q) * d * (4 if dtype == "f32" else 2) if shape.kind == W.MODEL_STT else 0
    norms = (2 * L + 1) * d * 4 * (2 if shape.norm_kind == W.NORM_LAYER else 1)
    out = []
    for p in positions:
        vis = min(p + 1, window) if window else p + 1
        out.append(w + L * (2 * vis * kvw * kv_bytes + 2 * kvw * kv_bytes) + emb + norms)
    return np.array(out, dtype=np.float64)


def cpu_baseline(shape, dtype, tensors, audio, steps, threads):
    import oracle

    oracle.set_threads(threads)
    m = oracle.Model(shape.config(__import__("svl").workloads.quantize_code(dtype)), tensors)
    st = m.new_state()
    st.stt_greedy(audio[:2])  # warm-up
    st = m.new_state()
    t0 = time.perf_counter()
    toks = st.stt_greedy(audio[:steps])
    dt = time.perf_counter() - t0
    return steps / dt, toks


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--cpu-steps", type=int, default=64)
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

    import svl
    from svl import hip
    from svl import workloads as W

    shape, dtype = W.S1, "q8_0"
    t0 = time.perf_counter()
    tensors = W.make_weights(shape, dtype, seed=0)
    print(f"weights generated in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    model = svl.Model(shape.config(W.quantize_code(dtype)), tensors, kv_dtype=svl.F32)
    audio = W.audio_tokens(shape, max(args.steps, args.cpu_steps), seed=1)[0]
    d_audio = hip.DeviceBuffer.from_array(audio)
    d_out = hip.DeviceBuffer(args.steps * 4)

    st = model.init_state()
    e0, e1 = hip.Event(), hip.Event()
    # warm-up: launches of the same size as the timed one, each from position 0
    for _ in range(max(1, -(-args.warmup // args.steps)) if args.warmup > 0 else 0):
        model.recognize_async(args.steps, d_audio.address, d_out.address, st)
        st.synchronize()
        st.reset()
    hip.synchronize()
    t0 = time.perf_counter()
    e0.record(st.stream)
    model.recognize_async(args.steps, d_audio.address, d_out.address, st)
    e1.record(st.stream)
    st.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_ms(e1)
    print(f"timed {args.steps} steps: {gpu_ms:.2f} ms", file=sys.stderr, flush=True)
    steps_per_s = args.steps / (gpu_ms / 1e3)

    bytes_per_step = step_bytes(shape, dtype, 4, range(args.steps), shape.context)
    launch_bytes = float(bytes_per_step.sum())
    achieved = launch_bytes / (gpu_ms / 1e3) / 1e9

    line = {
        "metric": "decode steps/s at B=1 (STT-1B-shape, Q8_0); % of HBM roofline",
        "value": round(steps_per_s, 2),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 (int8 x int8 -> int32 block dots, f32 scales and sums)",
        "data": "synthetic (seeded N(0, 0.02) weights, uniform audio ids, greedy text feedback)",
        "config": {"workload": "stt-1b q8_0 greedy decode, batch 1, from position 0",
                   "layers": shape.num_layers, "d_model": shape.d_model, "heads": shape.num_heads,
                   "head_dim": shape.head_dim, "ff_hidden": shape.ff_hidden, "window": shape.context,
                   "text_vocab": shape.text_card, "codebooks": shape.n_q, "batch": 1,
                   "kv_dtype": "f32", "wall_s": round(wall, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(args.steps),
                     "kernel": "step_program_kernel (one launch = all timed steps)",
                     "algorithmic_bytes_per_launch": int(launch_bytes),
                     "launch_ms": round(gpu_ms, 4)},
    }
    if not args.no_cpu_baseline:
        cps, toks = cpu_baseline(shape, dtype, tensors, audio, args.cpu_steps, args.cpu_threads)
        line["cpu_baseline"] = {"value": round(cps, 3), "unit": "steps/s", "cores": args.cpu_threads,
                                "kind": "port",
                                "sample": f"{args.cpu_steps} greedy steps of the same workload from position 0 "
                                          f"(oracle, {args.cpu_threads} threads)"}
        gpu_toks = d_out.to_array(np.uint32, args.steps)[: min(args.cpu_steps, args.steps)]
        line["cpu_baseline"]["tokens_match"] = bool(np.array_equal(gpu_toks, toks[: gpu_toks.size]))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
