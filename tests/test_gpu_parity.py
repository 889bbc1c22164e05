"""GPU parity: the gfx950 kernels (through the C ABI) against the CPU oracle.

Bar: bit-exact for every packed-state byte (1Q indices, fp16 scales, sign
bits, labels, fp16 amplitudes), for block norms, alpha and parameters, on
identical inputs and Philox draws.  Sizes are small enough for the CPU
oracle to finish in seconds; the benchmark configurations at full size are in
test_gpu_fullsize.py.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import compare_states, from_torch, gpu_state, log, make_grads, run_side_by_side, to_bits, \
    to_torch

pytestmark = pytest.mark.gpu

F32, BF16, F16 = O.DT_F32, O.DT_BF16, O.DT_F16


def _lib():
    from turboadam_amd import _lib

    return _lib, _lib.load()


def _eval(fn, x):
    _l, lib = _lib()
    dev = torch.device("cuda:0")
    xi = torch.from_numpy(x).to(dev)
    out = torch.empty_like(xi)
    _l.check(lib.tam_math_eval(fn, xi.data_ptr(), out.data_ptr(), x.size, _l.stream_of(dev)), "tam_math_eval")
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _edge_floats(rng, n):
    bits = rng.integers(0, 0x7F800000, size=n, dtype=np.uint32)
    specials = np.array([0x00000001, 0x007FFFFF, 0x00800000, 0x3F800000, 0x3F7FFFFF, 0x3F800001,
                         0x7F7FFFFF, 0x00000000, 0x7F800000, 0x0036F9F6], dtype=np.uint32)
    return np.concatenate([bits, specials]).view(np.float32)


def test_device_log_is_correctly_rounded():
    log("tam_math_eval log: 4M random positive fp32 + edges")
    rng = np.random.default_rng(1)
    x = _edge_floats(rng, 1 << 22)
    got = _eval(0, x)
    L = O.lib()
    idx = rng.choice(x.size, 200000, replace=False)
    want = np.array([L.or_logf(float(v)) for v in x[idx]], dtype=np.float32)
    assert np.array_equal(got[idx].view(np.uint32), want.view(np.uint32))
    # device == host build of the same function over all samples
    host = np.log(x.astype(np.longdouble)).astype(np.float32)
    ok = np.isfinite(x) & (x > 0)
    assert np.array_equal(got[ok].view(np.uint32), host[ok].view(np.uint32))


def test_device_exp_is_correctly_rounded():
    log("tam_math_eval exp: [-104, 89]")
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.uniform(-104, 89, 1 << 22), rng.uniform(-90, -60, 1 << 20),
                        np.array([-87.5, -69.0625, 0.0, 88.72, -103.9])]).astype(np.float32)
    got = _eval(1, x)
    want = np.exp(x.astype(np.longdouble)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_device_half_and_bf16_rounding():
    log("tam_math_eval f16/bf16 round trips")
    rng = np.random.default_rng(3)
    x = np.concatenate([_edge_floats(rng, 1 << 20), -_edge_floats(rng, 1 << 18)]).astype(np.float32)
    x = x[np.isfinite(x)]
    got16 = _eval(2, x)
    want16 = x.astype(np.float16).astype(np.float32)
    assert np.array_equal(got16.view(np.uint32), want16.view(np.uint32))
    gotbf = _eval(3, x)
    wantbf = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(gotbf.view(np.uint32), wantbf.view(np.uint32))


def test_device_hardware_bf16_rounding_equals_software():
    # the certified bf16 update path uses v_cvt_pk_bf16_f32; it must agree with
    # round-to-nearest-even on every non-NaN input (subnormals, ties, overflow)
    rng = np.random.default_rng(5)
    x = np.concatenate([_edge_floats(rng, 1 << 21), -_edge_floats(rng, 1 << 19),
                        (np.arange(0, 1 << 16, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
                        (np.arange(0, 1 << 16, dtype=np.uint32) << 16 | 0x7FFF).view(np.float32)])
    x = x[~np.isnan(x)]
    hw = _eval(5, x)
    sw = _eval(3, x)
    assert np.array_equal(hw.view(np.uint32), sw.view(np.uint32))


def test_device_sqrt_is_correctly_rounded():
    rng = np.random.default_rng(4)
    x = _edge_floats(rng, 1 << 20)
    got = _eval(4, x)
    assert np.array_equal(got.view(np.uint32), np.sqrt(x).view(np.uint32))


def test_hardware_sqrt_rcp_log2_error_bounds_on_every_normal_input():
    """The certified fast paths rest on three hardware instructions' error
    bounds: v_sqrt_f32 and v_rcp_f32 (bf16/fp16 update) within 2^-23 relative,
    v_log_f32 (1Q index) within 2^-21 relative of log2.  Checked on every
    positive normal fp32 input (v_rcp_f32 where 1/x is normal too; log2 exact
    at 1), against fp64 references on the device, 2^27 inputs at a time."""
    _l, lib = _lib()
    dev = torch.device("cuda:0")
    lo, hi, chunk = 0x00800000, 0x7F800000, 1 << 27
    worst = {6: 0.0, 7: 0.0, 8: 0.0}
    out = torch.empty(chunk, dtype=torch.float32, device=dev)
    for start in range(lo, hi, chunk):
        n = min(chunk, hi - start)
        bits = torch.arange(start, start + n, dtype=torch.int64, device=dev).to(torch.int32)
        x = bits.view(torch.float32)
        xd = x.double()
        for fn in (6, 7, 8):
            _l.check(lib.tam_math_eval(fn, x.data_ptr(), out.data_ptr(), n, _l.stream_of(dev)), "tam_math_eval")
            y = out[:n].double()
            if fn == 6:
                ref = torch.sqrt(xd)
                rel = ((y - ref) / ref).abs()
            elif fn == 7:
                ref = 1.0 / xd
                rel = ((y - ref) * xd).abs()
                rel = torch.where(x < 2.0 ** 126, rel, torch.zeros_like(rel))
            else:
                ref = torch.log2(xd)
                exact_one = x == 1.0
                assert bool((y[exact_one] == 0.0).all())
                rel = torch.where(exact_one, torch.zeros_like(ref), ((y - ref) / ref).abs())
            worst[fn] = max(worst[fn], float(rel.max()))
        del bits, x, xd, y, ref, rel
    log(f"max relative error over every normal input: v_sqrt_f32 2^{np.log2(worst[6]):.3f}, "
        f"v_rcp_f32 2^{np.log2(worst[7]):.3f}, v_log_f32 2^{np.log2(worst[8]):.3f}")
    assert worst[6] <= 2.0 ** -23
    assert worst[7] <= 2.0 ** -23
    assert worst[8] <= 2.0 ** -21


def test_philox_uniforms_match_oracle():
    _l, lib = _lib()
    dev = torch.device("cuda:0")
    for tid, step, seed, count in [(0, 1, 0, 1000), (7, 123, 0x7A3D5EED0BADC0DE, 4099), (291, 20, 42, 1 << 16)]:
        log(f"philox tid={tid} step={step} count={count}")
        out = torch.empty(count, dtype=torch.float32, device=dev)
        _l.check(lib.tam_philox_uniforms(tid, step, seed, count, out.data_ptr(), _l.stream_of(dev)), "philox")
        torch.cuda.synchronize()
        want = O.philox_uniforms(tid, step, seed, count)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _check(bad):
    assert not bad, "\n".join(bad[:20])


def test_v_only_fp32_ragged():
    log("v-only fp32, sizes with tails, 8 steps")
    _check(run_side_by_side([70000, 300, 1, 4096 + 77], [F32] * 4, steps=8, compress_m=False, lr=1e-3))


def test_m_and_v_fp32_mixed_sizes():
    log("m+v fp32 (CoState + fp32-m), 10 steps, wd")
    sizes = [4096, 5000, 128 * 40 + 3, 300, 1, 2304 * 8]
    _check(run_side_by_side(sizes, [F32] * len(sizes), steps=10, lr=6e-4, weight_decay=0.01))


def test_m_and_v_bf16():
    log("m+v bf16, 8 steps")
    sizes = [4096 * 3, 8192 + 128, 777]
    _check(run_side_by_side(sizes, [BF16] * len(sizes), steps=8, lr=1e-3, weight_decay=0.1))


def test_m_and_v_fp16():
    log("m+v fp16, 6 steps")
    sizes = [4096 * 2, 1000]
    _check(run_side_by_side(sizes, [F16] * len(sizes), steps=6, lr=1e-3))


def test_m_and_v_mixed_dtypes_split_pass_2():
    # 16-bit and fp32 CoState tensors in one step: pass 2's 16-bit kernel takes
    # the 16-bit units and every tail quarter, its fp32 kernel the full fp32
    # units; then the same with unaligned views (every unit to the quarter path)
    log("m+v mixed bf16 / fp32 / fp16 with tails, aligned and unaligned, 4 steps")
    sizes = [8192 * 9 + 300, 4096 * 5 + 17, 8192 * 3, 5000, 1024 * 7 + 129]
    dts = [F32, BF16, F32, F16, F32]
    _check(run_side_by_side(sizes, dts, steps=4, lr=1e-3, weight_decay=0.01))
    _check(run_side_by_side(sizes, dts, steps=3, offset=1, lr=1e-3, weight_decay=0.01))


@pytest.mark.parametrize("bits", [2, 3, 6, 8])
def test_v_bits(bits):
    log(f"m+v fp32 v_bits={bits}")
    sizes = [4096 + 1000, 513]
    _check(run_side_by_side(sizes, [F32] * 2, steps=5, v_bits=bits, null_pct=0.05, amp_pct=0.95))


def test_uncompressed_paths():
    log("compress_m only / compress_v only / neither")
    sizes = [6000, 200]
    _check(run_side_by_side(sizes, [F32] * 2, steps=5, compress_v=False))
    _check(run_side_by_side(sizes, [F32] * 2, steps=5, compress_m=False))
    _check(run_side_by_side(sizes, [F32] * 2, steps=5, compress_m=False, compress_v=False))


def test_grad_none_and_late_params():
    log("grad None on some steps")
    sizes = [5000, 300, 9000]
    _check(run_side_by_side(sizes, [F32] * 3, steps=6, grad_none=lambda s, i: (i == 1 and s % 2 == 0) or
                            (i == 2 and s < 2)))


def test_gpt2_block_shapes_few_steps():
    log("GPT-2 block (config 0 shapes), fp32, 3 steps")
    shapes = [(768,), (768,), (768, 2304), (2304,), (768, 768), (768,), (768,), (768,), (768, 3072), (3072,),
              (3072, 768), (768,)]
    sizes = [int(np.prod(s)) for s in shapes]
    _check(run_side_by_side(sizes, [F32] * len(sizes), steps=3, shapes=shapes, lr=6e-4, weight_decay=0.01))


def test_large_tensors_multi_workgroup_reductions():
    # 5M elements: 9768 quarter-tile partials (two alpha-reduction chunks of 8192);
    # 2.1M elements: 16391 blocks (three selection slices of 8192 ratios)
    log("bf16 5.0M + 2.1M elements, 3 steps (multi-chunk alpha, multi-slice selection)")
    sizes = [5_000_000 + 333, 8192 * 128 * 2 + 777]
    _check(run_side_by_side(sizes, [BF16] * 2, steps=3, lr=1e-3, weight_decay=0.1))


@pytest.mark.parametrize("dt", [F32, BF16])
def test_unaligned_parameter_views(dt):
    # parameters and gradients one element past a 16-byte boundary: every quarter
    # takes the bounds-checked path
    log(f"unaligned views dtype={dt}")
    sizes = [70_000, 4096 + 5, 300]
    _check(run_side_by_side(sizes, [dt] * 3, steps=4, offset=1, lr=1e-3, weight_decay=0.05))


def test_large_unaligned_tensor_spreads_over_workgroups():
    # 1.2M elements one past a 16-byte boundary: 586 tiles over 147 tail
    # workgroups (TAM_TAIL_TILES tiles each, the last one partial); a second,
    # smaller unaligned tensor follows in the tail grid
    log("large unaligned view")
    _check(run_side_by_side([1_200_001, 9000], [BF16, BF16], steps=2, offset=1, lr=1e-3, weight_decay=0.05))


@pytest.mark.parametrize("bits,pct", [(2, (0.10, 0.90)), (3, (0.05, 0.95)), (6, (0.10, 0.90)), (8, (0.05, 0.95))])
def test_ragged_multi_tensor_sweep(bits, pct):
    # the ragged-config pattern at a size the oracle finishes in seconds: 120 fp32
    # tensors log-uniform in [1, 2^14], mostly with tail blocks
    rng = np.random.default_rng(bits)
    sizes = [int(max(1, round(2 ** (14 * u)))) for u in rng.random(120)]
    log(f"ragged sweep: 120 tensors, {sum(sizes)} params, v_bits={bits}, pct={pct}")
    _check(run_side_by_side(sizes, [F32] * len(sizes), steps=3, v_bits=bits, null_pct=pct[0], amp_pct=pct[1],
                            lr=1e-3))


def test_sparse_heavy_tailed_gradients():
    # exact-zero gradient rows (a sparse embedding pattern) and Student-t(3) tails
    log("sparse rows of zeros + heavy tails, fp32, 4 steps")
    from turboadam_amd import TurboAdam
    from tests.helpers import from_torch, gpu_state, compare_states, to_torch

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(11)
    rows, cols = 400, 96
    sizes = [rows * cols, 5000]
    init = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]
    o_params = [a.copy() for a in init]
    g_params = [torch.nn.Parameter(to_torch(a, F32, (n,), dev)) for a, n in zip(init, sizes)]
    opt = TurboAdam(g_params, lr=6e-4, weight_decay=0.01)
    opt.philox_seed = 4242
    orc = O.OracleTurboAdam(o_params, dtypes=[F32, F32], seed=4242, lr=6e-4, weight_decay=0.01)
    bad = []
    for s in range(4):
        t = rng.standard_t(3, size=sizes[0]).astype(np.float32) * np.float32(1e-3)
        keep = rng.random(rows) < 0.05
        t = (t.reshape(rows, cols) * keep[:, None]).reshape(-1).astype(np.float32)
        g2 = (rng.standard_t(3, size=sizes[1]) * 1e-3).astype(np.float32)
        grads = [t, g2]
        for p, g, n in zip(g_params, grads, sizes):
            p.grad = to_torch(g, F32, (n,), dev)
        opt.step()
        orc.step(grads)
        torch.cuda.synchronize()
        for i, p in enumerate(g_params):
            where = f"step {s + 1} tensor {i}"
            if not np.array_equal(from_torch(p.data).view(np.uint32), o_params[i].view(np.uint32)):
                bad.append(f"{where}: param differs")
            bad += compare_states(gpu_state(opt, p), orc.state[i], where)
    _check(bad)


@pytest.mark.parametrize("dt", [F32, BF16, F16])
def test_error_feedback(dt):
    # CoState error feedback (fifth pass): tensors with tail blocks and one small
    # fp32-m tensor, residual compared bit for bit every step
    log(f"error feedback dtype={dt}, 5 steps")
    sizes = [5000, 4608 + 77, 300, 18509]
    _check(run_side_by_side(sizes, [dt] * len(sizes), steps=5, error_feedback=True, lr=1e-3, weight_decay=0.01))


def test_error_feedback_grad_none_unaligned_and_large():
    # a tensor without a gradient in some steps, unaligned views (bounds-checked
    # quarters), and a 2.1M-element tensor (many tiles, chunks and slices)
    log("error feedback: grad=None steps, unaligned views, 2.1M elements")
    _check(run_side_by_side([9000, 70_001], [BF16, F32], steps=4, error_feedback=True, offset=1,
                            grad_none=lambda s, i: i == 1 and s == 1, lr=1e-3, null_pct=0.05, amp_pct=0.95))
    _check(run_side_by_side([8192 * 128 * 2 + 777], [BF16], steps=3, error_feedback=True, lr=1e-3,
                            weight_decay=0.1))


def _nan_mask(a: np.ndarray, kind: str) -> np.ndarray:
    if a.dtype == np.float32:
        return np.isnan(a)
    if kind == "bf16":
        return (a & 0x7FFF) > 0x7F80
    if kind == "f16":
        return (a & 0x7FFF) > 0x7C00
    return np.zeros(a.shape, bool)


def _same(a: np.ndarray, b: np.ndarray, kind: str) -> np.ndarray:
    """Equal bit patterns, or NaN in both (NaN payloads are not part of parity)."""
    av = a.view(np.uint32) if a.dtype == np.float32 else a
    bv = b.view(np.uint32) if b.dtype == np.float32 else b
    return (av == bv) | (_nan_mask(a, kind) & _nan_mask(b, kind))


def _edge_run(dt, init, grads, **kw):
    """Step the GPU optimizer and the oracle through `grads` (per step, per
    tensor: fp32 arrays or None) from `init`; NaN-aware bit comparison."""
    from turboadam_amd import TurboAdam
    from tests.helpers import from_torch, gpu_state, to_bits, to_torch

    dev = torch.device("cuda:0")
    pkind = {BF16: "bf16", F16: "f16", F32: "f32"}[dt]
    o_params = [to_bits(a, dt) for a in init]
    g_params = [torch.nn.Parameter(to_torch(a.copy(), dt, (a.size,), dev)) for a in o_params]
    opt = TurboAdam(g_params, philox_seed=99, **kw)
    orc = O.OracleTurboAdam(o_params, dtypes=[dt] * len(init), seed=99, **kw)
    bad = []
    for s, gs in enumerate(grads):
        gb = [None if g is None else to_bits(g, dt) for g in gs]
        for p, g in zip(g_params, gb):
            p.grad = None if g is None else to_torch(g, dt, (g.size,), dev)
        opt.step()
        orc.step(gb)
        torch.cuda.synchronize()
        for i, p in enumerate(g_params):
            where = f"step {s + 1} tensor {i}"
            ok = _same(from_torch(p.data), o_params[i], pkind)
            if not ok.all():
                j = int(np.flatnonzero(~ok)[0])
                bad.append(f"{where}: param differs in {int((~ok).sum())} (first {j}: gpu {from_torch(p.data)[j]:#x} "
                           f"oracle {o_params[i][j]:#x})")
            if i not in orc.state:
                continue
            gst, ost = gpu_state(opt, p), orc.state[i]
            for k, b in ost.items():
                if k not in gst or not isinstance(b, np.ndarray) or k in ("has_ef",):
                    continue
                a = gst[k]
                kind = "f16" if k in ("amp", "scales") else "raw"
                if a.shape != b.shape or not _same(a, b, kind).all():
                    bad.append(f"{where}: {k} differs")
    return bad


def _edge_grads(rng, sizes, steps, scale, edit=None):
    out = []
    for s in range(steps):
        gs = [(rng.standard_normal(n) * scale).astype(np.float32) for n in sizes]
        if edit is not None:
            edit(s, gs)
        out.append(gs)
    return out


@pytest.mark.parametrize("dt", [BF16, F16])
def test_update_tiny_moments_zero_params(dt):
    # fl(-lr*m) and c*m in or near the subnormal range while bc1 = 1 - 0.99^t is
    # small, parameters exactly zero or tiny: the certificate's absolute terms
    log(f"edge: tiny moments, zero params, dtype={dt}")
    rng = np.random.default_rng(71)
    sizes = [4096 + 77, 2048]
    init = [np.zeros(sizes[0], np.float32), (rng.standard_normal(sizes[1]) * 1e-30).astype(np.float32)]
    scale = 1e-34 if dt == BF16 else 3e-6
    lr = 1e-3 if dt == BF16 else 1e-4
    grads = _edge_grads(rng, sizes, 4, scale)
    _check(_edge_run(dt, init, grads, lr=lr, betas=(0.99, 0.999)))


def test_update_zero_blocks_nan_and_inf_gradients():
    # a block of exact zeros at step 1 (v = 0: the q range fails), NaN of both
    # signs and infinities in later steps (NaN blocks, NaN parameters)
    log("edge: zero blocks, NaN / inf gradients, bf16")
    rng = np.random.default_rng(72)
    sizes = [4096 + 77, 5000]

    def edit(s, gs):
        if s == 0:
            gs[0][128:256] = 0.0
            gs[1][:512] = 0.0
        if s >= 1:
            gs[0][300] = np.nan
            gs[0][301] = -np.float32(np.nan)
            gs[0][700] = np.inf
            gs[1][1000] = -np.inf
    init = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]
    grads = _edge_grads(rng, sizes, 3, 1e-3, edit)
    _check(_edge_run(BF16, init, grads, lr=1e-3, weight_decay=0.1))


@pytest.mark.parametrize("eps", [0.0, -1e-8])
def test_update_eps_zero_and_negative(eps):
    log(f"edge: eps={eps}, bf16")
    rng = np.random.default_rng(73)
    sizes = [4096 + 77, 3000]
    init = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]
    grads = _edge_grads(rng, sizes, 3, 1e-4)
    _check(_edge_run(BF16, init, grads, lr=1e-3, eps=eps))


@pytest.mark.parametrize("betas", [(0.9, 1.5), (0.9, -0.5)])
def test_update_betas_outside_unit_interval(betas):
    # the reference does not validate betas: v may be negative (clamped path)
    log(f"edge: betas={betas}, bf16")
    rng = np.random.default_rng(74)
    sizes = [4096 + 77]
    init = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]
    grads = _edge_grads(rng, sizes, 3, 1e-3)
    _check(_edge_run(BF16, init, grads, lr=1e-3, betas=betas))


@pytest.mark.parametrize("dt", [BF16, F16])
def test_update_nonfinite_and_huge_params_beside_finite_ones(dt):
    # the 16-bit update certifies elements in pairs: NaN, +-inf and finite
    # values at or above 2^126 (f16: its largest finite values) in one or both
    # halves of a pair, next to ordinary values
    log(f"edge: non-finite and huge parameters in pairs, dtype={dt}")
    rng = np.random.default_rng(78)
    n = 4096 + 77
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    big = np.float32(2.0 ** 126 * 1.5) if dt == BF16 else np.float32(60000.0)
    p[10], p[21], p[22] = np.nan, np.nan, -np.float32(np.nan)  # NaN beside a finite value, NaN pair
    p[40], p[51], p[60:62] = np.inf, -np.inf, [np.inf, -np.inf]
    p[100:164:2] = big  # even halves of pairs
    p[201:265:2] = -big  # odd halves
    p[300:310] = big
    grads = _edge_grads(rng, [n], 3, 1e-3)
    _check(_edge_run(dt, [p], grads, lr=1e-3, weight_decay=0.1))


def test_update_near_overflow():
    # parameters near the bf16 maximum and updates near fp32 overflow
    log("edge: near-overflow parameters and updates, bf16")
    rng = np.random.default_rng(75)
    n = 4096 + 77
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    p[::7] = np.float32(3.3e38)
    p[3::7] = -np.float32(3.3e38)
    grads = _edge_grads(rng, [n], 3, 1.0)
    _check(_edge_run(BF16, [p], grads, lr=3e37))


def test_200_step_trajectory_bit_exact():
    # a long run: every packed state byte and every parameter bit after 50, 100,
    # 150 and 200 steps (mixed dtypes, tails, an fp32-m tensor)
    log("200 steps, mixed dtypes, bit-exact every 50 steps")
    sizes = [5000, 4096 + 77, 300, 20_000]
    _check(run_side_by_side(sizes, [BF16, F16, F32, F32], steps=200, check_every=50, lr=6e-4, weight_decay=0.01))


def test_200_step_trajectory_error_feedback_bit_exact():
    log("200 steps with error feedback, bf16, bit-exact every 50 steps")
    _check(run_side_by_side([9000, 4608 + 77], [BF16, BF16], steps=200, check_every=50, error_feedback=True,
                            lr=6e-4, weight_decay=0.01))


def test_param_groups_with_own_hyperparameters_and_lr_schedule():
    """Four groups, each with its own lr, betas, eps, weight decay, v_bits,
    thresholds and compression switches, and every group's lr changed before
    each step as a scheduler does (param_groups[i]["lr"] mutated): bit-exact
    against the oracle after every step."""
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    spec = [
        (dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, v_bits=4), [(70_001, BF16), (5000, F32)]),
        (dict(lr=3e-4, betas=(0.8, 0.99), eps=1e-6, weight_decay=0.0, v_bits=2, null_pct=0.05, amp_pct=0.95),
         [(20_000, F32), (300, BF16)]),
        (dict(lr=5e-4, betas=(0.95, 0.9999), eps=1e-7, weight_decay=0.1, v_bits=8, compress_m=False),
         [(9000, F16), (4000, F32)]),
        (dict(lr=1e-3, weight_decay=0.05, v_bits=3, compress_v=False), [(6000, F32), (12_345, BF16)]),
    ]
    sizes = [n for _, ts in spec for n, _ in ts]
    dts = [dt for _, ts in spec for _, dt in ts]
    rng = np.random.default_rng(51)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    g_params = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    o_params = [a.copy() for a in init]
    g_groups, o_groups, k = [], [], 0
    for hp, ts in spec:
        g_groups.append(dict(params=g_params[k:k + len(ts)], **hp))
        o_groups.append(dict(params=o_params[k:k + len(ts)], **hp))
        k += len(ts)
    opt = TurboAdam(g_groups, philox_seed=4242)
    orc = O.OracleTurboAdam(o_groups, dtypes=dts, seed=4242)
    sigmas = np.exp(np.log(1e-3) + rng.standard_normal(len(sizes)))
    drifts = [rng.standard_normal(n).astype(np.float32) for n in sizes]
    steps = 6
    for s in range(steps):
        scale = 0.1 + 0.9 * 0.5 * (1.0 + math.cos(math.pi * s / steps))  # cosine decay
        for gi, (hp, _) in enumerate(spec):
            opt.param_groups[gi]["lr"] = orc.param_groups[gi]["lr"] = hp["lr"] * scale
        grads = make_grads(rng, sizes, dts, sigmas, drifts)
        for p, g, dt, n in zip(g_params, grads, dts, sizes):
            p.grad = to_torch(g, dt, (n,), dev)
        opt.step()
        orc.step(grads)
        torch.cuda.synchronize()
        log(f"groups: step {s + 1}, lr scale {scale:.4f}")
        bad = []
        for i, p in enumerate(g_params):
            a, b = from_torch(p.data), o_params[i]
            if not np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                  b.view(np.uint32) if b.dtype == np.float32 else b):
                bad.append(f"step {s + 1} tensor {i}: params differ")
            bad += compare_states(gpu_state(opt, p), orc.state[i], f"step {s + 1} tensor {i}")
        assert not bad, "\n".join(bad[:20])


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("lmin,lmax", [(-69.0, -68.75), (-69.0, -67.0), (22.0, 22.125), (-0.25, 0.25),
                                       (-20.0, -19.9375)])
def test_requantisation_of_narrow_log_spans(bits, lmin, lmax):
    """Blocks whose v spans a narrow log range at large |ln v| (the state 1Q's
    repeated re-quantisation converges to): the certified index path is at
    its tightest there.  After one normal step both sides get the same
    synthetic v state (fp16 log bounds lmin, lmax; random indices), then take
    steps with gradients small enough to keep v in that range; bit-exact
    against the oracle after every step."""
    from turboadam_amd import TurboAdam

    dev = torch.device("cuda:0")
    sizes, dts = [40_000, 40_064, 3000], [F32, BF16, F32]
    rng = np.random.default_rng(61 + bits)
    init = [to_bits((rng.standard_normal(n) * 0.02).astype(np.float32), dt) for n, dt in zip(sizes, dts)]
    g_params = [torch.nn.Parameter(to_torch(a, dt, (n,), dev)) for a, dt, n in zip(init, dts, sizes)]
    o_params = [a.copy() for a in init]
    kw = dict(lr=1e-3, weight_decay=0.01, v_bits=bits)
    opt = TurboAdam(g_params, philox_seed=777 + bits, **kw)
    orc = O.OracleTurboAdam(o_params, dtypes=dts, seed=777 + bits, **kw)
    gscale = float(np.exp(0.5 * lmin)) * 1e-2  # (1 - beta2) g^2 ~ 1e-7 v: v stays in the span

    def grads():
        return [to_bits((rng.standard_normal(n) * gscale).astype(np.float32), dt) for n, dt in zip(sizes, dts)]

    def step(gs):
        for p, g, dt, n in zip(g_params, gs, dts, sizes):
            p.grad = to_torch(g, dt, (n,), dev)
        opt.step()
        orc.step(gs)
        torch.cuda.synchronize()

    step(grads())
    sc = np.array([lmin, lmax], dtype=np.float16).view(np.uint16)
    for i, (p, n) in enumerate(zip(g_params, sizes)):
        nb = (n + 127) // 128
        idx = rng.integers(0, 1 << bits, size=nb * 128, dtype=np.uint8)
        scales = np.tile(sc, nb)
        cv = opt.state[p]["compressed_v"]
        cv["indices"].copy_(torch.from_numpy(idx).to(dev))
        cv["scales"].copy_(torch.from_numpy(scales.view(np.int16).copy()).view(torch.float16).reshape(nb, 2).to(dev))
        orc.state[i]["indices"][:] = idx
        orc.state[i]["scales"][:] = scales
    for s in range(4):
        step(grads())
        bad = []
        for i, p in enumerate(g_params):
            a, b = from_torch(p.data), o_params[i]
            if not np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                                  b.view(np.uint32) if b.dtype == np.float32 else b):
                bad.append(f"step {s + 2} tensor {i}: params differ")
            bad += compare_states(gpu_state(opt, p), orc.state[i], f"step {s + 2} tensor {i}")
        log(f"narrow spans bits={bits} [{lmin}, {lmax}]: step {s + 2}, {len(bad)} mismatches")
        assert not bad, "\n".join(bad[:20])


def test_update_bf16_results_near_rounding_midpoints():
    # parameters in [1, 2) (bf16 spacing 2^-7) and lr = 2^-8: at step 1 the
    # update is -lr*sign(g)/(1 + eps/|g|), so p + u lands within a few fp32
    # units of a bf16 rounding midpoint, spread by eps/|g| across the certified
    # update's error bound: accepted and rejected elements side by side, every
    # one bit-exact
    log("edge: bf16 updates near rounding midpoints")
    rng = np.random.default_rng(76)
    sizes = [4096 * 3 + 77, 5000]
    init = [(1.0 + rng.integers(0, 128, n) / 128.0).astype(np.float32) for n in sizes]
    grads = _edge_grads(rng, sizes, 3, 1e-5)
    _check(_edge_run(BF16, init, grads, lr=2.0 ** -8, eps=1e-8))


def test_update_beta1_near_one():
    # bc1 = 1 - beta1^t near 2^-22 t: k_abs = fl(2^-147/bc1) and the
    # certificate's absolute error term k_abs*r are at their largest
    log("edge: beta1 = 1 - 2^-22, bf16")
    rng = np.random.default_rng(77)
    sizes = [4096 + 77, 3000]
    init = [(rng.standard_normal(n) * 0.02).astype(np.float32) for n in sizes]
    grads = _edge_grads(rng, sizes, 3, 1e-3)
    _check(_edge_run(BF16, init, grads, lr=1e-3, betas=(1.0 - 2.0 ** -22, 0.999)))
