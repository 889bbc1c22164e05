"""Benchmark of the fused TurboAdam step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3]

A step is one TurboAdam.step() over the whole synthetic parameter set with
its gradients already resident in HBM.  Default workload (the headline
configuration): the Llama-3-8B-shaped parameter set (291 tensors,
8,030,261,248 parameters) in bf16, m+v compression, v_bits=4.  Prints one
JSON line with throughput (parameters updated per second), the roofline of
the dominant pass (pass 0) timed live with HIP events on the launch stream,
and a CPU baseline: the reference's CPU step (restated op for op in torch,
oracle/torch_mirror.py) timed on a bounded sample on this host.
"""

import argparse
import gc
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "params updated/sec per step + % HBM roofline, 8B-shaped m+v 4-bit"
HBM_PEAK_GBPS = 8000.0


# ---------------------------------------------------------------- workloads
def llama3_8b_shapes():
    h, kv, inter, vocab, layers = 4096, 1024, 14336, 128256, 32
    shapes = [("embed", (vocab, h))]
    for i in range(layers):
        shapes += [
            (f"l{i}.q", (h, h)), (f"l{i}.k", (kv, h)), (f"l{i}.v", (kv, h)), (f"l{i}.o", (h, h)),
            (f"l{i}.gate", (inter, h)), (f"l{i}.up", (inter, h)), (f"l{i}.down", (h, inter)),
            (f"l{i}.norm1", (h,)), (f"l{i}.norm2", (h,)),
        ]
    shapes += [("norm", (h,)), ("lm_head", (vocab, h))]
    return shapes


def gpt2_block_shapes(prefix=""):
    return [(prefix + "ln_1.w", (768,)), (prefix + "ln_1.b", (768,)), (prefix + "attn.c_attn.w", (768, 2304)),
            (prefix + "attn.c_attn.b", (2304,)), (prefix + "attn.c_proj.w", (768, 768)),
            (prefix + "attn.c_proj.b", (768,)), (prefix + "ln_2.w", (768,)), (prefix + "ln_2.b", (768,)),
            (prefix + "mlp.c_fc.w", (768, 3072)), (prefix + "mlp.c_fc.b", (3072,)),
            (prefix + "mlp.c_proj.w", (3072, 768)), (prefix + "mlp.c_proj.b", (768,))]


def gpt2_124m_shapes():
    s = [("wte", (50257, 768)), ("wpe", (1024, 768))]
    for i in range(12):
        s += gpt2_block_shapes(f"h{i}.")
    s += [("ln_f.w", (768,)), ("ln_f.b", (768,))]
    return s


def llama3_8b_rank0_of8_shapes():
    """Rank 0's share of the Llama-3-8B-shaped set when whole tensors are dealt
    to 8 ranks by greedy bin packing on size (largest first, to the lightest
    rank): the per-GPU shape of tensor-granular data-parallel sharding."""
    shapes = llama3_8b_shapes()
    load, bins = [0] * 8, [[] for _ in range(8)]
    for name, shp in sorted(shapes, key=lambda x: -math.prod(x[1])):
        r = min(range(8), key=lambda i: load[i])
        bins[r].append((name, shp))
        load[r] += math.prod(shp)
    order = {name: i for i, (name, _) in enumerate(shapes)}
    return sorted(bins[0], key=lambda x: order[x[0]])


def ragged_shapes(seed=0, count=1000):
    rng = np.random.default_rng(seed)
    sizes = np.maximum(1, np.round(2.0 ** (20 * rng.random(count)))).astype(np.int64)
    return [(f"t{i}", (int(n),)) for i, n in enumerate(sizes)]


WORKLOADS = {
    # name: (shapes fn, dtype, optimizer kwargs, log-sigma center, description)
    "c3": (llama3_8b_shapes, torch.bfloat16, dict(lr=3e-4, weight_decay=0.1, v_bits=4), math.log(1e-4),
           "llama3-8b-shaped bf16 m+v v_bits=4"),
    "c1": (lambda: [("p", (1 << 28,))], torch.float32, dict(lr=1e-3, compress_m=False, v_bits=4), math.log(1e-3),
           "v-only 2^28 fp32 v_bits=4"),
    "c2": (gpt2_124m_shapes, torch.float32, dict(lr=6e-4, weight_decay=0.01, v_bits=4), math.log(1e-3),
           "gpt2-124m fp32 m+v v_bits=4"),
    "c0": (gpt2_block_shapes, torch.float32, dict(lr=6e-4, weight_decay=0.01, v_bits=4), math.log(1e-3),
           "gpt2-block fp32 m+v v_bits=4"),
    "c4": (ragged_shapes, torch.float32, dict(lr=1e-3, v_bits=4), math.log(1e-3),
           "ragged 1000 tensors fp32 m+v v_bits=4"),
    "c3-ef": (llama3_8b_shapes, torch.bfloat16, dict(lr=3e-4, weight_decay=0.1, v_bits=4, error_feedback=True),
              math.log(1e-4), "llama3-8b-shaped bf16 m+v v_bits=4, error feedback"),
    "c3-rank0of8": (llama3_8b_rank0_of8_shapes, torch.bfloat16, dict(lr=3e-4, weight_decay=0.1, v_bits=4),
                    math.log(1e-4), "llama3-8b-shaped bf16 m+v v_bits=4, rank 0 of 8 (tensor sharding)"),
}
# the ragged set's sweep: v_bits in {2, 3, 6, 8} x (null_pct, amp_pct) in {(0.10, 0.90), (0.05, 0.95)}
for _bits in (2, 3, 6, 8):
    for _null, _amp in ((0.10, 0.90), (0.05, 0.95)):
        WORKLOADS[f"c4-b{_bits}-n{round(_null * 100):02d}"] = (
            ragged_shapes, torch.float32, dict(lr=1e-3, v_bits=_bits, null_pct=_null, amp_pct=_amp), math.log(1e-3),
            f"ragged 1000 tensors fp32 m+v v_bits={_bits} null/amp pct {_null:.2f}/{_amp:.2f}")


def bytes_per_param(dtype_bytes: int, costate: bool, compress_v: bool = True, ef: bool = False):
    """Algorithmic HBM bytes per parameter per step (whole step and pass 0 alone).

    pass 0 reads p, g, the 1Q indices and scales and (CoState) the previous
    signs/labels/norms/amplitudes and writes p, indices and scales; an fp32-m
    tensor reads and writes exp_avg instead.  CoState adds pass 2 (g, the
    previous encoding, new encoding, ratios) and the selection (ratios, labels).
    Error feedback adds the fp32 residual to pass 0's reads, and a fifth pass
    that reads g, the residual and both encodings and writes the residual and
    the committed encoding (14 + G bytes in all).
    """
    P = G = dtype_bytes
    v = (2.0 + 8.0 / 128) if compress_v else 8.0
    if costate:
        k1 = 2 * P + G + v + (1.0 / 8 + 7.0 / 128) + (4.0 if ef else 0.0)
        total = 2 * P + 2 * G + 2.0 + 3.0 / 8 + 37.0 / 128 + ((14.0 + G) if ef else 0.0)
    else:
        k1 = 2 * P + G + v + 8.0
        total = k1
    return k1, total


# ---------------------------------------------------------------- CPU baseline
FULL_SAMPLE_MAX = 300_000_000  # workloads up to this many parameters run whole on the CPU
ONE_THREAD_PARAMS = 16_000_000


def cpu_info():
    """CPU model, logical CPUs online, and the CPUs this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return model, os.cpu_count() or 1, usable


def cpu_sample(shapes):
    """The parts of a workload the CPU baseline steps, as (tensors, count)
    pairs: the whole workload once when it has at most FULL_SAMPLE_MAX
    parameters; otherwise one tensor of each distinct shape, counted as many
    times as the workload holds that shape.  On the 8B-shaped set that is the
    first decoder layer's five shapes, the RMSNorm, and the 525M-parameter
    embedding standing for itself and the output head (the reference's largest
    sorts, costate.py:114-118); every tensor of one shape costs the same.
    Returns (parts, sampled)."""
    total = sum(math.prod(shp) for _, shp in shapes)
    if total <= FULL_SAMPLE_MAX:
        return [(list(shapes), 1)], False
    first, count = {}, {}
    for name, shp in shapes:
        first.setdefault(shp, name)
        count[shp] = count.get(shp, 0) + 1
    return [([(first[shp], shp)], count[shp]) for shp in first], True


def host_ram_gib() -> float:
    """Total host memory in GiB (/proc/meminfo), 0 when unknown."""
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemTotal:"):
                    return int(line.split()[1]) / 2**20
    except (OSError, ValueError, IndexError):
        pass
    return 0.0


def _time_mirror(TM, shapes, dtype, kw, log_sigma, threads, min_steps, budget_s, gen):
    """Median seconds of the steady-state steps (second and later) of the
    reference's CPU step over the given shapes; gradients are drawn outside
    the timed region."""
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        params = [(torch.randn(shp, generator=gen) * 0.02).to(dtype) for _, shp in shapes]
        sig = [math.exp(log_sigma + float(torch.randn((), generator=gen))) for _ in shapes]
        opt = TM.MirrorTurboAdam(params, ops=TM.FaithfulOps, seed=1, **kw)
        times = []
        t_end = time.perf_counter() + budget_s
        while len(times) < min_steps or (time.perf_counter() < t_end and len(times) < 6):
            grads = [(torch.randn(p.shape, generator=gen) * s).to(dtype) for p, s in zip(params, sig)]
            t0 = time.perf_counter()
            opt.step(grads)
            times.append(time.perf_counter() - t0)
            del grads
        return float(np.median(times[1:])), len(times)
    finally:
        torch.set_num_threads(prev)


def cpu_baseline(shapes, dtype, kw, log_sigma, budget_s=20.0):
    """The reference's CPU step timed on this host, as the reported baseline.

    Runs oracle/torch_mirror.py in faithful mode -- the reference CPU path
    restated op for op in torch (it reproduces the reference's outputs bit for
    bit, tests/test_golden.py) -- with every CPU this process may use (at most
    OMP_NUM_THREADS when that is set), median of the steady-state steps.  A
    workload above FULL_SAMPLE_MAX parameters is timed part by part
    (cpu_sample: one tensor of each distinct shape) and its whole step is the
    sum of each part's time times its count; two whole steps of the 8B-shaped
    set would take several minutes of CPU time (the figure is reported), more
    than this run may hold the GPU.  A 1-thread figure is taken on the first
    tensors up to ONE_THREAD_PARAMS parameters (a leading 1-D slice of the
    first tensor when that alone is larger).
    """
    from oracle import torch_mirror as TM

    model, online, usable = cpu_info()
    threads = usable
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = max(1, min(threads, int(os.environ["OMP_NUM_THREADS"])))
    gen = torch.Generator().manual_seed(7)
    parts, sampled = cpu_sample(shapes)
    n_all = sum(math.prod(shp) for _, shp in shapes)
    n_part = [sum(math.prod(shp) for _, shp in tensors) for tensors, _ in parts]
    n_sample = sum(n_part)
    t_step, t_sample, steps = 0.0, 0.0, []
    for (tensors, count), n in zip(parts, n_part):
        # each part's share of the time budget follows its size
        t, k = _time_mirror(TM, tensors, dtype, kw, log_sigma, threads, 2, max(2.0, budget_s * n / n_sample), gen)
        t_step += count * t
        t_sample += t
        steps.append(k)

    one, n_one = [], 0
    for name, shp in (tensors[0] for tensors, _ in parts) if sampled else parts[0][0]:
        n = math.prod(shp)
        if n_one + n > 2 * ONE_THREAD_PARAMS:
            if not one:
                one, n_one = [(name + "[:%d]" % ONE_THREAD_PARAMS, (ONE_THREAD_PARAMS,))], ONE_THREAD_PARAMS
            break
        one.append((name, shp))
        n_one += n
        if n_one >= ONE_THREAD_PARAMS:
            break
    t1, steps1 = _time_mirror(TM, one, dtype, kw, log_sigma, 1, 2, budget_s / 2, gen)

    if sampled:
        listing = "; ".join(f"{tensors[0][0]} {list(tensors[0][1])} x{count}" for tensors, count in parts)
        how = (f"one tensor of each distinct shape ({listing}; {n_sample} of {n_all} params), each timed on its "
               f"own; whole step = sum of count x time ({min(steps)}-{max(steps)} steps per part)")
    else:
        how = f"the whole workload ({len(parts[0][0])} tensors, {n_sample} params; {steps[0]} steps)"
    return {"value": n_all / t_step, "unit": "params/s", "cores": threads, "kind": "port",
            "sample": f"{how}, {str(dtype)[6:]}; median of steps 2+; reference CPU step restated in torch ops "
                      f"(faithful mirror, bit-identical to the reference), {threads} threads",
            "ms_per_step_workload": t_step * 1e3,
            "sample_params_per_s": n_sample / t_sample,
            "one_thread": {"value": n_one / t1, "unit": "params/s", "steps": steps1,
                           "sample": ", ".join(n for n, _ in one) + f" ({n_one} params)"},
            "cpu_model": model, "cpus_online": online, "cpus_usable": usable,
            "host_ram_gib": round(host_ram_gib(), 1)}


# ---------------------------------------------------------------- HBM traffic
KERNEL_SOURCES = ("tam_step.hip", "tam_math.h", "tam_tables.h")


def kernel_source_sha() -> str:
    """First 16 hex digits of the sha256 over the kernel sources, in order."""
    import hashlib

    h = hashlib.sha256()
    for name in KERNEL_SOURCES:
        with open(os.path.join(ROOT, "turboadam_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(workload: str):
    """HBM bytes per pass-0 launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary of this workload (counters scaled by their plain-copy
    calibration), or None when no summary covers the workload or the summary
    was taken on other kernel sources than the ones built here."""
    path = os.path.join(ROOT, "profiles", f"tam_k1_main_{workload}_fetch_write.md")
    if not os.path.exists(path):
        return None
    sha, traffic = None, None
    for line in open(path):
        if line.startswith("Kernel sources") and "`" in line:
            sha = line.split("`")[1]
        elif line.startswith("traffic_bytes_per_launch"):
            traffic = float(line.split("=")[1])
    return traffic if sha == kernel_source_sha() else None


# ---------------------------------------------------------------- copy reference
def copy_reference(args):
    """Plain device-to-device copy of 2^30 fp32 (4 GiB read + 4 GiB written).

    Calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE (known bytes per dispatch)
    and measures the bandwidth a streaming kernel actually reaches.
    """
    dev = torch.device("cuda:0")
    x = torch.ones(1 << 30, dtype=torch.float32, device=dev)
    y = torch.empty_like(x)
    for _ in range(args.warmup):
        y.copy_(x)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        y.copy_(x)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    nbytes = 2 * x.numel() * 4
    print(json.dumps({"workload": "copy 2^30 fp32", "ms_per_copy": ms, "bytes_per_copy": nbytes,
                      "GBps": nbytes / (ms * 1e-3) / 1e9}), flush=True)


# ---------------------------------------------------------------- streaming ceiling
STREAM_KINDS = {"read": (0, 1), "write": (1, 1), "copy": (2, 2), "2r1w": (3, 3), "inplace": (4, 3)}
STREAM_LAYOUTS = {0: "grid-stride", 1: "wave-contiguous", 2: "lane-contiguous"}


def _stream_lib():
    import ctypes

    from turboadam_amd.build import STREAM_LIB_PATH

    lib = ctypes.CDLL(STREAM_LIB_PATH)
    lib.tam_stream_run.restype = ctypes.c_long
    lib.tam_stream_run.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int,
                                   ctypes.c_void_p]
    lib.tam_stream_pass0.restype = ctypes.c_long
    lib.tam_stream_pass0.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint64, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_uint32, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.tam_stream_pass0_sizes.restype = None
    lib.tam_stream_pass0_sizes.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]
    return lib


def _time_launches(launch, warmup: int, steps: int, stream) -> float:
    """Milliseconds per launch (HIP events on the launch stream)."""
    for _ in range(max(1, warmup)):
        launch()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(steps):
        launch()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def stream_reference(args):
    """Bandwidth of plain streaming kernels (turboadam_amd/csrc/tam_stream.hip)
    over 4 GiB per array: read, write, copy, two reads + one write to a third
    array, and an in-place read-modify-write of one array with a read of a
    second (the access shape of the step's parameter update).  Sweeps words in
    flight per lane (4, 8, 16), workgroup size (256, 512, 1024), grid rounds
    (1-16), nontemporal loads and stores off and on, and three access layouts
    (STREAM_LAYOUTS).  Prints one JSON line per variant, then the best variant
    of each kind."""
    lib = _stream_lib()
    dev = torch.device("cuda:0")
    n16 = 1 << 28  # 16-byte words per array: 4 GiB
    bufs = [torch.ones(n16 * 4, dtype=torch.int32, device=dev) for _ in range(3)]
    stream = torch.cuda.current_stream(dev)
    best = {}
    for name, (kind, arrays) in STREAM_KINDS.items():
        for nt in (0, 1):
            for words in (4, 8, 16):
                for wg in (256, 512, 1024):
                    for layout in STREAM_LAYOUTS:
                        for rounds in (1, 2, 4, 8, 16):
                            grid = [0]

                            def launch():
                                grid[0] = lib.tam_stream_run(kind, nt, words, wg, layout, bufs[0].data_ptr(),
                                                             bufs[1].data_ptr(), bufs[2].data_ptr(), n16, rounds,
                                                             stream.cuda_stream)
                                if grid[0] < 0:
                                    raise ValueError(grid[0])

                            try:
                                ms = _time_launches(launch, 1, args.steps, stream)
                            except ValueError:
                                continue  # a combination the library refuses (register budget)
                            nbytes = arrays * n16 * 16
                            gbps = nbytes / (ms * 1e-3) / 1e9
                            rec = {"workload": "stream", "kernel": name, "nontemporal": bool(nt), "words": words,
                                   "wg": wg, "layout": STREAM_LAYOUTS[layout], "rounds": rounds, "grid": grid[0],
                                   "ms_per_launch": ms, "bytes_per_launch": nbytes, "GBps": gbps,
                                   "frac_of_8TBps": gbps / HBM_PEAK_GBPS}
                            print(json.dumps(rec), flush=True)
                            if gbps > best.get(name, {}).get("GBps", 0.0):
                                best[name] = rec
    print(json.dumps({"workload": "stream", "best": best}), flush=True)


def stream_pass0_reference(args):
    """Bandwidth of a stream with the step's first pass's arrays and access
    widths (tam_stream_pass0: 16-bit parameter and gradient, u8 1Q indices,
    per-block scales and CoState bytes, partial sums), 2^30 elements, across
    workgroup sizes, workgroups per CU, grid rounds, and with or without an
    LDS allocation that caps a CU at 4 waves per SIMD (the main pass-0 kernels'
    register budget), for two element-to-lane layouts with and without
    nontemporal access.  One JSON line per variant, then the best."""
    import ctypes

    lib = _stream_lib()
    dev = torch.device("cuda:0")
    units = 1 << 20
    sizes = (ctypes.c_uint64 * 9)()
    lib.tam_stream_pass0_sizes(units, sizes)
    bufs = [torch.ones((int(s) + 255) // 4, dtype=torch.int32, device=dev) for s in sizes]
    ptrs = (ctypes.c_void_p * 9)(*[b.data_ptr() for b in bufs])
    stream = torch.cuda.current_stream(dev)
    # bytes per launch: the parameter and indices and scales are read and written
    nbytes = int(sum(sizes)) + int(sizes[0]) + int(sizes[2]) + int(sizes[3])
    best = None
    variants = [(layout, nt, wg, per_cu, rounds, cap) for layout, nt in ((0, 0), (0, 1), (1, 0), (1, 1))
                for wg in (128, 256) for per_cu in (4, 8, 16) for rounds in (1, 4, 16) for cap in (False, True)]
    # larger grids, up to one unit per wave (lane layout, capped)
    variants += [(0, nt, wg, per_cu, rounds, True) for nt in (0, 1) for wg in (128, 256)
                 for per_cu in (32, 64) for rounds in (16, 64)]
    for layout, nt, wg, per_cu, rounds, cap in variants:
        lds = (163840 // (16 * 64 // wg)) if cap else 0  # 16 waves per CU when capped

        def launch():
            g = lib.tam_stream_pass0(ptrs, units, wg, per_cu, rounds, lds, layout, nt,
                                     stream.cuda_stream)
            if g < 0:
                raise RuntimeError(f"tam_stream_pass0 failed ({g})")

        ms = _time_launches(launch, 1, args.steps, stream)
        gbps = nbytes / (ms * 1e-3) / 1e9
        rec = {"workload": "stream-pass0", "layout": ["lane 16 elements", "wave-contiguous 2x8"][layout],
               "nontemporal": bool(nt), "wg": wg, "wgs_per_cu": per_cu, "rounds": rounds,
               "cap_4_waves_per_simd": cap, "elements": units * 1024, "ms_per_launch": ms,
               "bytes_per_launch": nbytes, "GBps": gbps, "frac_of_8TBps": gbps / HBM_PEAK_GBPS}
        print(json.dumps(rec), flush=True)
        if best is None or gbps > best["GBps"]:
            best = rec
    print(json.dumps({"workload": "stream-pass0", "best": best}), flush=True)


# ---------------------------------------------------------------- fallback rates
def fallback_stats(args, opt, params, set_grads, desc):
    """Step the workload with the counting build and print, for each requested
    step, how many lanes and elements of pass 0's full units fell back from
    the certified fast paths to the exact sequence (the re-quantisation of v,
    per half unit, and the 16-bit update, per half unit), with their rates."""
    import ctypes

    from turboadam_amd import _lib

    lib = _lib.load()
    lib.tam_stats_read.restype = ctypes.c_int
    lib.tam_stats_read.argtypes = [ctypes.POINTER(ctypes.c_uint64), ctypes.c_int]
    out = (ctypes.c_uint64 * 4)()
    want = sorted({int(x) for x in args.fallback_stats.split(",") if x.strip()})
    units = sum(p.numel() // 1024 for p in params)  # full units (every tensor here is aligned)
    _lib.check(lib.tam_stats_read(out, 1), "tam_stats_read")
    for s in range(1, want[-1] + 1):
        set_grads(s - 1)
        opt.step()
        _lib.check(lib.tam_stats_read(out, 1), "tam_stats_read")
        if s in want:
            vq_l, vq_e, up_l, up_p = (int(x) for x in out)
            print(json.dumps({"workload": desc, "step": s, "full_units": units,
                              "vq_lanes": vq_l, "vq_lane_frac": vq_l / (128 * units),
                              "vq_elems": vq_e, "vq_elem_frac": vq_e / (1024 * units),
                              "update_lanes": up_l, "update_lane_frac": up_l / (128 * units),
                              "update_pairs": up_p, "update_pair_frac": up_p / (512 * units)}), flush=True)


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c3", choices=sorted(WORKLOADS) + ["copy", "stream", "stream-pass0"])
    ap.add_argument("--grad-sets", type=int, default=2)
    ap.add_argument("--pass-steps", type=int, default=5,
                    help="extra steps after the timed region, issued pass by pass, that time pass 0")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-baseline-only", action="store_true",
                    help="time only the CPU baseline of the workload (no GPU work)")
    ap.add_argument("--fallback-stats", default="",
                    help="comma-separated step numbers: instead of timing, step the workload with the counting "
                         "build (python -m turboadam_amd.build --stats) and print how often pass 0's certified "
                         "fast paths fell back to the exact sequence at those steps")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the optimizer step is single-device); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from turboadam_amd import TurboAdam, _lib

    if args.fallback_stats:
        from turboadam_amd.build import STATS_LIB_PATH

        _lib.load(STATS_LIB_PATH)  # the counting build serves every call of this process
    _lib.load()
    if args.workload == "copy":
        copy_reference(args)
        return
    if args.workload == "stream":
        stream_reference(args)
        return
    if args.workload == "stream-pass0":
        stream_pass0_reference(args)
        return
    shapes_fn, dtype, kw, log_sigma, desc = WORKLOADS[args.workload]
    shapes = shapes_fn()
    if args.cpu_baseline_only:
        print(json.dumps({"workload": desc, "cpu_baseline": cpu_baseline(
            shapes, dtype, kw, log_sigma)}), flush=True)
        return
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    params, grad_sets = [], [[] for _ in range(args.grad_sets)]
    sig_rng = np.random.default_rng(1)
    for name, shp in shapes:
        p = torch.empty(shp, dtype=dtype, device=dev)
        if "norm" in name or name.startswith("ln") or ".ln_" in name:
            p.fill_(1.0)
        else:
            p.normal_(0.0, 0.02, generator=gen)
        params.append(torch.nn.Parameter(p))
        sigma = math.exp(log_sigma + sig_rng.standard_normal())
        drift = torch.randn(shp, device=dev, generator=gen, dtype=torch.float32)
        for k in range(args.grad_sets):
            z = torch.randn(shp, device=dev, generator=gen, dtype=torch.float32)
            grad_sets[k].append((sigma * (z + 0.3 * drift)).to(dtype))
        del drift, z
    nparams = sum(p.numel() for p in params)
    opt = TurboAdam(params, **kw)

    def set_grads(k):
        for p, g in zip(params, grad_sets[k % args.grad_sets]):
            p.grad = g

    if args.fallback_stats:
        fallback_stats(args, opt, params, set_grads, desc)
        return
    for s in range(args.warmup):
        set_grads(s)
        opt.step()
    torch.cuda.synchronize()

    # timed region: K steps of the production call (one tam_multi_tensor_step per step)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # a full collection of the warmup's garbage (tens of ms) would otherwise
    # fire inside the first timed steps, while the GPU waits on an empty queue
    gc.collect()
    torch.cuda.synchronize()
    start.record()
    for s in range(args.steps):
        set_grads(args.warmup + s)
        opt.step()
    stop.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    ms_step = total_ms / args.steps

    # pass 0 alone: further steps issued pass by pass, pass 0 bracketed by HIP
    # events recorded on the launch stream (outside the timed region above)
    ev = []

    def hook(k, when):
        if k == 0:
            e = torch.cuda.Event(enable_timing=True)
            e.record(torch.cuda.current_stream(dev))
            ev.append(e)

    opt._pass_hook = hook
    for s in range(max(1, args.pass_steps)):
        set_grads(args.warmup + args.steps + s)
        opt.step()
    torch.cuda.synchronize()
    opt._pass_hook = None
    k1_ms = [ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(len(ev) // 2)]
    k1_avg = float(np.mean(k1_ms))

    dbytes = torch.tensor([], dtype=dtype).element_size()
    k1_bytes = 0.0
    step_bytes = 0.0
    for p in params:
        st = opt.state[p]
        ef = st["_compress_m"] and st["m_mgr"]._error_feedback
        k1, tot = bytes_per_param(dbytes, st["_compress_m"], "compressed_v" in st, ef)
        k1_bytes += k1 * p.numel()
        step_bytes += tot * p.numel()
    k1_gbps = k1_bytes / (k1_avg * 1e-3) / 1e9
    step_gbps = step_bytes / (ms_step * 1e-3) / 1e9

    out = {
        "metric": METRIC,
        "value": nparams / (ms_step * 1e-3),
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": desc,
            "params": nparams,
            "tensors": len(params),
            "param_dtype": str(dtype).replace("torch.", ""),
            "grad_dtype": str(dtype).replace("torch.", ""),
            "optimizer": {k: v for k, v in kw.items()},
            "step_bytes_alg": step_bytes,
            "step_hbm_frac": step_gbps / HBM_PEAK_GBPS,
        },
        "roofline": {
            "kernel": ("pass 0 (tam_k1_ef + tam_k1_tail)" if kw.get("error_feedback")
                       else "pass 0 (tam_k1_main_<dtype> + tam_k1_tail)"),
            "bound": "hbm",
            "achieved": k1_gbps,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": k1_gbps / HBM_PEAK_GBPS,
            "traffic": measured_traffic(args.workload),
            "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0, "
                            "from the profile of these kernel sources; null if none)",
            "ms_per_launch": k1_avg,
            "launches_timed": len(k1_ms),
            "bytes_alg_per_launch": k1_bytes,
        },
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(shapes, dtype, kw, log_sigma)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
