"""The bench's workloads are the reference's benchmark configurations (CPU).

Parameter and tensor counts of each synthetic configuration, the rank-0
share of the tensor-sharded Llama set, the byte model's per-parameter figures,
and the one-GPU guard of the command line.
"""

import math
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _count(shapes):
    return len(shapes), sum(math.prod(s) for _, s in shapes)


def test_workload_sizes():
    assert _count(bench.gpt2_block_shapes()) == (12, 7_087_872)
    assert _count(bench.gpt2_124m_shapes()) == (148, 124_439_808)
    assert _count(bench.llama3_8b_shapes()) == (291, 8_030_261_248)
    assert _count(bench.WORKLOADS["c1"][0]()) == (1, 1 << 28)
    ragged = bench.ragged_shapes()
    assert len(ragged) == 1000 and all(1 <= math.prod(s) <= 1 << 20 for _, s in ragged)
    assert sum(math.prod(s) % 128 != 0 for _, s in ragged) > 900  # tail blocks almost everywhere


def test_rank0_of8_is_a_balanced_eighth():
    full = dict(bench.llama3_8b_shapes())
    part = bench.llama3_8b_rank0_of8_shapes()
    names = [n for n, _ in part]
    assert len(set(names)) == len(names) and all(full[n] == s for n, s in part)
    _, total = _count(part)
    assert abs(total - 8_030_261_248 / 8) / (8_030_261_248 / 8) < 0.01
    assert "embed" in names


def test_byte_model():
    # CoState bf16: 2P + 2G + 2 + 3/8 + 37/128 over the step; pass 0 alone 2P + G + 2 + 8/128 + 1/8 + 7/128
    k1, total = bench.bytes_per_param(2, True)
    assert math.isclose(total, 2 * 2 + 2 * 2 + 2 + 3 / 8 + 37 / 128)
    assert math.isclose(k1, 2 * 2 + 2 + 2 + 8 / 128 + 1 / 8 + 7 / 128)
    k1e, total_e = bench.bytes_per_param(2, True, ef=True)
    assert math.isclose(k1e - k1, 4.0) and math.isclose(total_e - total, 14.0 + 2)
    # fp32 m (no CoState): exp_avg read and written in pass 0, which is the whole step
    k1, total = bench.bytes_per_param(4, False)
    assert math.isclose(k1, total) and math.isclose(total, 2 * 4 + 4 + 2 + 8 / 128 + 8)


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=300, cwd=ROOT)
    assert res.returncode == 2
    assert "one GPU" in res.stderr


def test_ragged_sweep_workloads():
    # the ragged set's sweep: every v_bits x (null_pct, amp_pct) pair on the same 1000 tensors
    names = sorted(n for n in bench.WORKLOADS if n.startswith("c4-b"))
    assert len(names) == 8
    pairs = {(bench.WORKLOADS[n][2]["v_bits"], bench.WORKLOADS[n][2]["null_pct"], bench.WORKLOADS[n][2]["amp_pct"])
             for n in names}
    assert pairs == {(b, nl, am) for b in (2, 3, 6, 8) for nl, am in ((0.10, 0.90), (0.05, 0.95))}
    assert all(bench.WORKLOADS[n][0] is bench.ragged_shapes for n in names)


def test_cpu_baseline_sample():
    # workloads up to 300M parameters run whole; the 8B-shaped set is timed one
    # tensor per distinct shape, each counted as often as the set holds it
    for name in ("c0", "c1", "c2", "c4"):
        shapes = bench.WORKLOADS[name][0]()
        assert bench.cpu_sample(shapes) == ([(list(shapes), 1)], False)
    shapes = bench.llama3_8b_shapes()
    parts, sampled = bench.cpu_sample(shapes)
    assert sampled
    names = {tensors[0][0]: count for tensors, count in parts}
    assert names == {"embed": 2, "l0.q": 64, "l0.k": 64, "l0.gate": 64, "l0.down": 32, "l0.norm1": 65}
    assert all(len(tensors) == 1 for tensors, _ in parts)
    # the counts rebuild the whole set
    assert sum(math.prod(t[0][1]) * c for t, c in parts) == _count(shapes)[1] == 8_030_261_248
    assert len(shapes) == sum(c for _, c in parts)


def test_kernel_source_sha_gates_the_traffic_figure():
    # a profile summary names the kernel sources it measured; another build reads null
    for name in ("c1", "c2", "c3", "c4"):
        path = os.path.join(ROOT, "profiles", f"tam_k1_main_{name}_fetch_write.md")
        if not os.path.exists(path):
            continue
        sha = [ln.split("`")[1] for ln in open(path) if ln.startswith("Kernel sources")][0]
        t = bench.measured_traffic(name)
        assert (t is not None) == (sha == bench.kernel_source_sha())
    assert bench.measured_traffic("c0") is None
