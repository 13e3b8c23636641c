"""bench.py's host-side accounting (no GPU): the one-GPU contract, the per-kernel traffic entries of
the committed counter summaries, and the algorithmic bytes of a phase."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


@pytest.mark.parametrize("name", ["stt1b_q8_b1", "stt1b_q8_b64"])
def test_traffic_entries_name_bench_kernel_groups(name):
    tr = bench.read_traffic(name)
    assert tr["steps"] > 0 and tr["hbm_bytes_per_step"] > 0
    assert tr["per_kernel"], "no per-kernel entry"
    for k, v in tr["per_kernel"].items():
        assert k in bench.KERNEL_GROUPS, k
        assert 0 < v < tr["hbm_bytes_per_step"]


def test_read_traffic_parses_entries(tmp_path, monkeypatch):
    p = tmp_path / "profiles"
    p.mkdir()
    (p / "x.traffic.txt").write_text("# comment: ignored\nsteps: 16\nhbm_bytes_per_step: 1000\n"
                                     "hbm_bytes_per_launch[attn_phase_kernel (attention)]: 250\n")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    assert bench.read_traffic("x") == {"steps": 16, "hbm_bytes_per_step": 1000,
                                       "per_kernel": {"attn_phase_kernel (attention)": 250}}
    assert bench.read_traffic("missing") == {}


def test_phase_bytes_of_a_q8_0_gemv_and_attention():
    from svl import workloads as W

    shape = W.S1
    # Q8_0 (format 3): 34 bytes per 32 weights, plus the f32 input rows
    assert bench.phase_bytes([bench.PH_GEMV, 3, 6144, 2048], shape, 1, [1]) == 6144 * 2048 // 32 * 34 + 2048 * 4
    kvw = shape.num_kv_heads * shape.head_dim
    assert bench.phase_bytes([bench.PH_ATTN, 0, 0, 0], shape, 2, [10, 750]) == 2 * (10 + 750) * kvw * 4
    # every group classifies a GEMV of its own format
    kinds = {name: [pick(i) for i in ([1, 3, 1, 2048], [1, 3, 1, 5632], [1, 4, 1, 2048], [1, 6, 1, 2048])]
             for name, pick in bench.KERNEL_GROUPS.items()}
    assert sum(sum(v) for v in kinds.values()) == 4


def test_read_floor_shapes_are_grids_the_read_kernel_accepts():
    """svl_bench_read takes 1 .. 65536 workgroups of 64 .. 1024 threads (a multiple of 64); every
    shape the read floor tries must be one, and each writes blocks x threads words."""
    assert bench.READ_SHAPES
    for blocks, threads in bench.READ_SHAPES:
        assert 1 <= blocks <= 65536 and 64 <= threads <= 1024 and threads % 64 == 0
