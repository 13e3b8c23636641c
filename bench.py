"""Decode-step benchmark of the streaming-transformer step on one MI355X.

Default workload: STT-1B shape (16 layers, d_model 2048, 16 heads x 128, gated SiLU 5632,
RMSNorm, window 750, text vocabulary 8000, 32 audio codebooks) with every linear in candle
Q8_0, batch 1, greedy decoding from an empty state.  A step is one decode step: embedding
gather-sum, 16 layers, output norm, text_linear, argmax, with the argmax fed back as the next
text token on the device.  Inputs (weights, audio tokens) are resident in HBM before timing.

Prints ONE JSON line (rank 0).  `value` is decode steps/s; `roofline` prices the step against
MI355X HBM bandwidth with the algorithmic bytes of the steps actually timed; `cpu_baseline` is
the oracle (this repository's C restatement of the reference's CPU path) on the host cores.
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
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--cpu-steps", type=int, default=64)
    ap.add_argument("--cpu-threads", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the decode step has no multi-GPU path "
              "(independent streams shard across GPUs with no communication).", file=sys.stderr)
        sys.exit(2)

    import svl
    from svl import hip
    from svl import workloads as W

    shape, dtype = W.S1, "q8_0"
    t0 = time.perf_counter()
    tensors = W.make_weights(shape, dtype, seed=0)
    print(f"weights generated in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    model = svl.Model(shape.config(W.quantize_code(dtype)), tensors, kv_dtype=svl.F32)
    n_total = args.warmup + args.steps
    audio = W.audio_tokens(shape, max(n_total, args.cpu_steps), seed=1)[0]
    d_audio = hip.DeviceBuffer.from_array(audio)
    d_out = hip.DeviceBuffer(n_total * 4)

    st = model.init_state()
    e0, e1 = hip.Event(), hip.Event()
    # warm-up, then restart the stream from position 0
    model.recognize_async(args.warmup, d_audio.address, d_out.address, st)
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
    achieved = float(bytes_per_step.mean()) / (gpu_ms / 1e3 / args.steps) / 1e9

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
        "roofline": {"bound": "hbm", "kernel": "decode step (all kernels of one step)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "bytes_per_step": int(bytes_per_step.mean()), "traffic": None},
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
