"""CPU: pin the oracle (oracle/tam_oracle.c) before trusting it.

Each check is chosen so that a plausible slip in the oracle -- a wrong
Philox constant, a wrong rounding in the fp16 conversion, an inaccurate
transcendental, a dropped term, a transposed bit order, an off-by-one rank --
fails here.  Sources of truth: published known-answer vectors (Random123),
library routines (numpy fp16, torch bf16, torch.optim.Adam), exact arithmetic
(Python decimal / fractions) and the closed forms the reference's own tests
assert (tests/test_costate.py, tests/test_optimizer.py in the reference).
"""

import ctypes
import decimal
import math
from decimal import Decimal as D
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import oracle as O

L = O.lib()
P = O.ptr


# ---------------------------------------------------------------- Philox
KATS = [  # Random123 kat_vectors, philox4x32 R=10
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KATS)
def test_philox_known_answers(ctr, key, want):
    c = np.array(ctr, np.uint32)
    out = np.zeros(4, np.uint32)
    L.or_philox4x32_10(P(c), key[0], key[1], P(out))
    assert tuple(int(x) for x in out) == want


def test_philox_uniform_layout():
    # group t = e // 16: the three blocks with counters (3t + j, tid, step,
    # (3t + j) >> 32) as one little-endian 384-bit integer; element k = e % 16
    # takes the 24-bit integer with high 16 bits at [16k, 16k + 16) (the first
    # two blocks) and low 8 bits at [256 + 8k, 256 + 8k + 8) (the third) --
    # here as Python big-integer arithmetic over the KAT-pinned generator,
    # including a counter past 2^32.  The synthetic inputs use the same bits
    # with element k at [24k, 24k + 24).
    seed = 0x0123456789ABCDEF
    n = 16 * 5 + 7
    u = O.philox_uniforms(5, 9, seed, n)
    ui = O.input_uniforms(5, 9, seed, n)

    def block(c):
        ctr = np.array([c & 0xFFFFFFFF, 5, 9, c >> 32], np.uint32)
        out = np.zeros(4, np.uint32)
        L.or_philox4x32_10(P(ctr), seed & 0xFFFFFFFF, seed >> 32, P(out))
        return sum(int(w) << (32 * i) for i, w in enumerate(out))

    for e in range(n):
        t, k = divmod(e, 16)
        bits = sum(block(3 * t + j) << (128 * j) for j in range(3))
        hi, lo = (bits >> (16 * k)) & 0xFFFF, (bits >> (256 + 8 * k)) & 0xFF
        assert u[e] == np.float32(((hi << 8) | lo) * 2.0**-24), e
        assert ui[e] == np.float32(((bits >> (24 * k)) & 0xFFFFFF) * 2.0**-24), e
    assert (u >= 0).all() and (u < 1).all()
    # a group whose counters pass 2^32 (group t = 2^32 // 3 + 1): the slice
    # draws of a block0 offset reach it through or_fused_v_update
    t = (1 << 32) // 3 + 1
    bits = sum(block(3 * t + j) << (128 * j) for j in range(3))
    assert 3 * t > (1 << 32) and bits > 0


# ---------------------------------------------------------------- fp16 / bf16
def test_f16_rounding_matches_numpy():
    rng = np.random.default_rng(0)
    bits = np.concatenate([
        rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32),
        # every fp32 near each fp16 boundary: fp16 values, their midpoints and neighbours
        (np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
         .view(np.uint32)[:, None] + np.array([0, 1, 0xFFFFFFFF, 0x1000, 0xFFF, 0x1001], np.uint32)).ravel(),
    ])
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    want = x.astype(np.float16).view(np.uint16)
    f = L.or_f32_to_f16
    got = np.array([f(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[np.isfinite(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    f = L.or_f32_to_bf16
    got = np.array([f(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype,delta", [(torch.bfloat16, 2.0**-10), (torch.float16, 2.0**-13)])
def test_small_weight_decay_leaves_16bit_parameters_unchanged(dtype, delta):
    """The kernels skip decoupled weight decay on a 16-bit parameter when
    1 - delta <= c <= 1 (c = f32(1 - lr*wd)): R_p(fl(x*c)) == x for every
    finite 16-bit x and every such c.  Checked on all 65536 patterns at the
    bound, just inside it, at C3's lr*wd and at 1 - 2^-24; and the bound is
    not vacuous: at 4*delta some values change."""
    xs = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(dtype)
    xs = xs[torch.isfinite(xs)]
    x32 = xs.to(torch.float32)
    for c in (1.0 - delta, 1.0 - delta + 2.0**-24, 1.0 - delta / 3, float(np.float32(1.0 - 3e-4 * 0.1)),
              1.0 - 2.0**-24, 1.0):
        c32 = torch.tensor(c, dtype=torch.float32)
        assert float(c32) >= 1.0 - delta
        y = (x32 * c32).to(dtype)  # fp32 product (correctly rounded), then round to nearest even
        assert torch.equal(y.view(torch.int16), xs.view(torch.int16)), c
    y = (x32 * torch.tensor(1.0 - 4 * delta, dtype=torch.float32)).to(dtype)
    assert not torch.equal(y.view(torch.int16), xs.view(torch.int16))


# ---------------------------------------------------------------- log / exp
decimal.getcontext().prec = 50


def _round_f32(y: D) -> np.float32:
    """Correctly rounded fp32 of an exact Decimal (ties to even)."""
    f = np.float32(float(y))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda c: (abs(D(float(c)) - y), int(np.float32(c).view(np.uint32)) & 1))
    return np.float32(best)


def test_log_is_correctly_rounded():
    rng = np.random.default_rng(2)
    bits = np.concatenate([rng.integers(1, 0x7F800000, 6000, dtype=np.uint32),
                           np.arange(0x3F7FFFF0, 0x3F800010, dtype=np.uint32),  # around 1
                           np.array([1, 2, 0x007FFFFF, 0x00800000, 0x0036F9F6, 0x7F7FFFFF], np.uint32)])
    for b in bits:
        x = np.uint32(b).view(np.float32)
        if x == 1.0:
            assert L.or_logf(1.0) == 0.0
            continue
        want = _round_f32(D(float(x)).ln())
        assert np.float32(L.or_logf(float(x))) == want, hex(b)


def test_exp_is_correctly_rounded():
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.uniform(-104, 88.7, 6000), rng.uniform(-104, -87, 2000),
                         [-69.0625, -87.5, 0.0, 1e-7, -1e-7]]).astype(np.float32)
    for x in xs:
        want = _round_f32(D(float(x)).exp())
        assert np.float32(L.or_expf(float(x))) == want, float(x)


# ---------------------------------------------------------------- pairwise sums
def test_pairwise_sum_tree_and_padding():
    rng = np.random.default_rng(4)
    for n in [1, 2, 3, 7, 128, 129, 1000]:
        x = rng.standard_normal(n) * 10.0 ** rng.integers(-8, 8, n)
        P2 = 1 << max(0, (n - 1).bit_length())
        buf = np.zeros(P2)
        buf[:n] = x

        def tree(a):
            return a[0] if len(a) == 1 else tree(a[: len(a) // 2]) + tree(a[len(a) // 2:])

        got = L.or_pairwise_sum(P(np.ascontiguousarray(x)), n)
        assert got == tree(list(buf))
        exact = float(sum(Fraction(v) for v in x))
        assert abs(got - exact) <= 1e-12 * np.abs(x).sum()


# ---------------------------------------------------------------- CoState closed forms
def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _round_f32_q(q: Fraction) -> float:
    """The fp32 value nearest the rational q (ties to even), by integer arithmetic."""
    if q == 0:
        return 0.0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()  # 2^e <= a < 2^(e+2)
    if Fraction(2) ** (e + 1) <= a:
        e += 1
    quantum = Fraction(2) ** (max(e, -126) - 23)
    n, r = divmod(a, quantum)
    n = int(n)
    if r > quantum / 2 or (r == quantum / 2 and n % 2 == 1):
        n += 1
    v = float(n * quantum)
    return -v if q < 0 else v


def _contract_lane(xs, ys) -> float:
    """The reduction contract's fp32 partial of 8 products, in exact rational
    arithmetic rounded to fp32 after each operation: p_k = fma(x_2k, y_2k,
    fl(x_2k+1 y_2k+1)), then (p0 + p1) + (p2 + p3)."""
    F = Fraction
    p = []
    for k in range(4):
        t = _round_f32_q(F(float(xs[2 * k + 1])) * F(float(ys[2 * k + 1])))
        p.append(_round_f32_q(F(float(xs[2 * k])) * F(float(ys[2 * k])) + F(t)))
    return _round_f32_q(F(_round_f32_q(F(p[0]) + F(p[1]))) + F(_round_f32_q(F(p[2]) + F(p[3]))))


def _pair(v):
    return v[0] if len(v) == 1 else _pair(v[: len(v) // 2]) + _pair(v[len(v) // 2:])


def _contract_blocks(x, y):
    """Per 128-element block (zero padded): fp64 pairwise sum of the 16 lane partials."""
    n = x.size
    nb = (n + 127) // 128
    xp = np.zeros(nb * 128, np.float32); xp[:n] = x
    yp = np.zeros(nb * 128, np.float32); yp[:n] = y
    return [_pair([_contract_lane(xp[i:i + 8], yp[i:i + 8]) for i in range(b * 128, b * 128 + 128, 8)])
            for b in range(nb)]


def test_dot_and_norm_contract_against_a_rational_restatement():
    """alpha and block norms of the C oracle equal, bit for bit, the reduction
    contract evaluated in exact rational arithmetic with explicit fp32 rounding
    (an implementation that shares nothing with the oracle's fmaf / double
    code), including products that land exactly on an fp32 rounding midpoint
    where only the fused first level gives the right result."""
    rng = np.random.default_rng(41)
    # (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24: an fp32 midpoint; the tiny second
    # product decides its rounding inside the fma
    mid = np.float32(1 + 2.0 ** -12)
    cases = []
    for n in (8, 128, 300, 1000):
        m = _f32(rng.standard_normal(n) * 10.0 ** rng.integers(-3, 3, n))
        g = _f32(rng.standard_normal(n) * 10.0 ** rng.integers(-3, 3, n))
        cases.append((m, g))
    m = _f32(np.tile([mid, 1e-20, mid, -1e-20, mid, 0.0, -mid, 1e-30], 32))
    g = _f32(np.tile([mid, 1e-20, mid, 1e-20, mid, 0.0, mid, 1e-30], 32))
    cases.append((m, g))
    tie = _f32(np.tile([mid, 1e-20, 0, 0, 0, 0, 0, 0], 16))
    cases.append((tie, tie))
    for m, g in cases:
        n = m.size
        gg = _pair(_contract_blocks(g, g) + [0.0] * ((1 << max(0, ((n + 127) // 128 - 1).bit_length())) - (n + 127) // 128))
        mg = _pair(_contract_blocks(m, g) + [0.0] * ((1 << max(0, ((n + 127) // 128 - 1).bit_length())) - (n + 127) // 128))
        gg32, mg32 = np.float32(gg + 0.0), np.float32(mg + 0.0)
        want = mg32 / gg32 if gg32 > 0 else np.float32(0.0)
        d = np.empty_like(m)
        got = np.float32(L.or_decompose(P(m), P(g), n, P(d)))
        assert got.view(np.uint32) == np.float32(want).view(np.uint32), (n, got, want)
        # block norms: fp64 sqrt of the block sum of squares, rounded once
        nrm = np.zeros((n + 127) // 128, np.float32)
        signs = np.zeros((n + 7) // 8, np.uint8)
        amp = np.zeros(nrm.size, np.uint16)
        L.or_encode(P(m), n, ctypes.c_float(np.float32(math.sqrt(128))), P(signs), P(nrm), P(amp))
        want_n = _f32([math.sqrt(b) for b in _contract_blocks(m, m)])
        assert np.array_equal(nrm.view(np.uint32), want_n.view(np.uint32))
    # the last case exercises the fused first level: fl(mid^2) alone rounds
    # the midpoint to even (down), the fma with the tiny second product rounds up
    assert _contract_lane(tie[:8], tie[:8]) == 1 + 2.0 ** -11 + 2.0 ** -23
    assert float(np.float32(np.float32(mid * mid) + np.float32(np.float32(1e-20) * np.float32(1e-20)))) == \
        1 + 2.0 ** -11


def test_decompose_closed_forms():
    rng = np.random.default_rng(5)
    g = _f32(rng.standard_normal(256))
    m = _f32(3.0 * g)
    d = np.empty_like(m)
    a = L.or_decompose(P(m), P(g), 256, P(d))
    assert abs(a - 3.0) < 1e-6 and np.linalg.norm(d) < 1e-5
    g = np.zeros(256, np.float32); g[0] = 1.0
    m = np.zeros(256, np.float32); m[1] = 5.0
    a = L.or_decompose(P(m), P(g), 256, P(d))
    assert a == 0.0 and np.array_equal(d, m)
    g = np.zeros(128, np.float32)
    m = _f32(rng.standard_normal(128))
    d = np.empty_like(m)
    a = L.or_decompose(P(m), P(g), 128, P(d))
    assert a == 0.0 and np.array_equal(d, m)
    # alpha equals the exactly rounded m.g / g.g (dot products each rounded once)
    m = _f32(rng.standard_normal(3000)); g = _f32(rng.standard_normal(3000)); d = np.empty_like(m)
    a = L.or_decompose(P(m), P(g), 3000, P(d))
    mg = np.float32(float(sum(Fraction(float(x)) * Fraction(float(y)) for x, y in zip(m, g))))
    gg = np.float32(float(sum(Fraction(float(y)) ** 2 for y in g)))
    assert abs(np.float32(a) - np.float32(mg / gg)) <= 2 * abs(np.spacing(np.float32(a)))
    assert np.array_equal(d, _f32(m - _f32(np.float32(a) * g)))


def test_block_ratios_closed_forms():
    rng = np.random.default_rng(6)
    m = _f32(rng.standard_normal(256))
    r = np.empty(2, np.float32)
    zero = np.zeros(256, np.float32)
    mc = m.copy()
    L.or_block_ratios(P(zero), P(m), 256, P(r))
    assert (r == 0).all()
    L.or_block_ratios(P(mc), P(m), 256, P(r))
    assert np.allclose(r, 1.0, atol=1e-6)
    L.or_block_ratios(P(m), P(zero), 256, P(r))
    assert (r == 0).all()
    # ragged: 300 elements -> 3 blocks, norm over the zero-padded block
    d = _f32(rng.standard_normal(300)); mm = _f32(rng.standard_normal(300)); r3 = np.empty(3, np.float32)
    L.or_block_ratios(P(d), P(mm), 300, P(r3))
    ref = [np.linalg.norm(d[i * 128:(i + 1) * 128].astype(np.float64)) /
           np.linalg.norm(mm[i * 128:(i + 1) * 128].astype(np.float64)) for i in range(3)]
    assert np.allclose(r3, ref, rtol=1e-6)


def _thr(r, null_pct=0.10, amp_pct=0.90):
    r = _f32(r)
    lo, hi = O.ranks(r.size, null_pct, amp_pct)
    t0 = np.zeros(1, np.float32); t1 = np.zeros(1, np.float32)
    L.or_thresholds(P(r), r.size, lo, hi, P(t0), P(t1))
    return t0[0], t1[0]


def test_thresholds_order_statistics():
    t0, t1 = _thr(np.linspace(0, 1, 1000))
    # reference test: |tau0 - 0.1| < 0.02; exactly: sorted[int(0.1*1000)-1] = sorted[99]
    assert t0 == np.float32(np.linspace(0, 1, 1000)[99]) and t1 == np.float32(np.linspace(0, 1, 1000)[900])
    assert _thr(np.full(128, 0.5)) == (0.5, 0.5)
    assert _thr([0.42]) == (np.float32(0.42), np.float32(0.42))
    rng = np.random.default_rng(7)
    for nb in [2, 5, 10, 11, 4608, 10000]:
        r = rng.choice([0.0, 0.25, 0.5, 1.0, 2.0], size=nb) * rng.random(nb).round(1)  # many ties and zeros
        s = np.sort(_f32(r))
        lo, hi = max(0, int(0.1 * nb) - 1), min(nb - 1, int(0.9 * nb))
        assert _thr(r) == (s[lo], s[hi])
    # Python's int(0.1 * 4608) is 460 and int(0.9 * 4608) is 4147 (0.9 * 4608 = 4147.2):
    # ranks 459 and 4147
    assert O.ranks(4608, 0.10, 0.90) == (459, 4147)


def test_classify_boundaries():
    r = _f32([0.01, 0.1, 0.5, 0.9, 1.5])
    lab = np.empty(5, np.uint8)
    L.or_classify(P(r), 5, ctypes.c_float(0.1), ctypes.c_float(0.9), P(lab))
    assert lab.tolist() == [0, 1, 1, 2, 2]


def test_sign_packing_every_byte():
    # element 8j+k -> byte j, bit 7-k (MSB first), trailing bits of the last byte are 0
    vals = np.array([(b >> (7 - k)) & 1 for b in range(256) for k in range(8)], np.float32)
    delta = _f32(np.where(vals > 0, -1.0, 1.0))
    n = delta.size
    signs = np.zeros(n // 8, np.uint8); norms = np.zeros(n // 128, np.float32); amp = np.zeros(n // 128, np.uint16)
    L.or_encode(P(delta), n, ctypes.c_float(np.float32(math.sqrt(128))), P(signs), P(norms), P(amp))
    assert signs.tolist() == list(range(256))
    # ragged: 13 elements -> 2 bytes, padding bits zero
    d = _f32(-np.ones(13)); s2 = np.zeros(2, np.uint8); n2 = np.zeros(1, np.float32); a2 = np.zeros(1, np.uint16)
    L.or_encode(P(d), 13, ctypes.c_float(np.float32(math.sqrt(128))), P(s2), P(n2), P(a2))
    assert s2.tolist() == [0xFF, 0xF8]


def test_encode_norms_and_amplitudes():
    rng = np.random.default_rng(8)
    d = _f32(rng.standard_normal(384) * 1e-3)
    q = np.float32(math.sqrt(128))
    s = np.zeros(48, np.uint8); nrm = np.zeros(3, np.float32); amp = np.zeros(3, np.uint16)
    L.or_encode(P(d), 384, ctypes.c_float(q), P(s), P(nrm), P(amp))
    for b in range(3):
        exact = math.sqrt(float(sum(Fraction(float(v)) ** 2 for v in d[b * 128:(b + 1) * 128])))
        assert abs(nrm[b] - exact) <= abs(np.spacing(nrm[b]))
        assert amp[b] == np.float16(np.float32(nrm[b] / q)).view(np.uint16)


def test_decode_formulas_per_label():
    rng = np.random.default_rng(9)
    n = 384
    g = _f32(rng.standard_normal(n))
    signs = rng.integers(0, 256, n // 8, dtype=np.uint8)
    labels = np.array([0, 1, 2], np.uint8)
    norms = _f32([3.0, 5.5, 7.25])
    amp = np.array([np.float16(0.5), np.float16(0.125), np.float16(0.3)], np.float16).view(np.uint16)
    out = np.empty(n, np.float32)
    q = np.float32(math.sqrt(128))
    alpha = np.float32(1.5)
    L.or_decode_blocks(P(labels), P(signs), P(norms), P(amp), ctypes.c_float(alpha), P(g), n, ctypes.c_float(q),
                       P(out))
    bits = np.unpackbits(signs)  # MSB first
    sgn = (1.0 - 2.0 * bits).astype(np.float32)
    scale = np.repeat(_f32([0.0, norms[1] / q, np.float16(0.3)]), 128)
    want = _f32(_f32(alpha * g) + _f32(scale * sgn))
    assert np.array_equal(out, want)


def test_first_costate_step_is_one_minus_beta1_times_g():
    rng = np.random.default_rng(10)
    n = 4096
    p = _f32(rng.standard_normal(n) * 0.02)
    g = _f32(rng.standard_normal(n))
    opt = O.OracleTurboAdam([p], lr=0.0, compress_v=False)
    opt.step([g])
    st = opt.state[0]
    # after step 1: alpha = (m.g)/(g.g) with m = f32(0.1)*g -> alpha is 0.1 up to dot rounding
    assert abs(st["alpha"][0] - np.float32(0.1)) < 1e-6


def test_weight_decay_only_closed_form():
    # reference tests/test_optimizer.py:645-660: zero gradient, lr=1e-2, wd=0.1 -> x = 1*(1-1e-3)
    p = np.ones(100, np.float32)
    opt = O.OracleTurboAdam([p], lr=1e-2, weight_decay=0.1)
    opt.step([np.zeros(100, np.float32)])
    assert np.all(p == np.float32(np.float32(1.0) * np.float32(1.0 - 1e-2 * 0.1)))


def test_no_compression_equals_torch_adam():
    # reference tests/test_optimizer.py:250-285 (atol 1e-6); the oracle is tighter
    torch.manual_seed(7)
    grads = [[torch.randn(10, 10), torch.randn(20)] for _ in range(10)]
    tp = [torch.nn.Parameter(torch.ones(10, 10)), torch.nn.Parameter(torch.ones(20))]
    adam = torch.optim.Adam(tp, lr=1e-3, betas=(0.9, 0.999))
    op = [np.ones(100, np.float32), np.ones(20, np.float32)]
    orc = O.OracleTurboAdam(op, lr=1e-3, compress_m=False, compress_v=False)
    for gs in grads:
        for p, g in zip(tp, gs):
            p.grad = g.clone()
        adam.step()
        orc.step([g.reshape(-1).numpy().copy() for g in gs])
    for p, o in zip(tp, op):
        assert np.allclose(p.detach().reshape(-1).numpy(), o, atol=1e-6, rtol=0)


def test_v_update_invariants_and_unbiased_rounding():
    rng = np.random.default_rng(11)
    n = 128 * 64
    g = _f32(rng.standard_normal(n) * 1e-3)
    for bits in (2, 3, 4, 6, 8):
        idx = np.zeros(n, np.uint8)
        sc = np.full(2 * (n // 128), O.V_INIT_SCALE_BITS, np.uint16)
        v = np.empty(n, np.float32)
        L.or_fused_v_update(P(idx), P(sc), P(g), n, bits, ctypes.c_float(np.float32(0.999)),
                            ctypes.c_float(np.float32(0.001)), 3, 1, 99, P(v))
        assert idx.max() < 2**bits
        s = sc.view(np.float16).astype(np.float32).reshape(-1, 2)
        assert (s[:, 0] <= s[:, 1]).all()
        assert (v > 0).all()
    # unbiased stochastic rounding: average index over many Philox streams -> continuous position
    g = _f32(rng.standard_normal(128) * 1e-3)
    acc = np.zeros(128)
    T = 400
    for step in range(T):
        idx = np.zeros(128, np.uint8)
        sc = np.full(2, O.V_INIT_SCALE_BITS, np.uint16)
        v = np.empty(128, np.float32)
        L.or_fused_v_update(P(idx), P(sc), P(g), 128, 4, ctypes.c_float(np.float32(0.999)),
                            ctypes.c_float(np.float32(0.001)), 0, step + 1, 5, P(v))
        acc += idx
    lv = np.log(np.maximum(v, np.float32(1e-38)).astype(np.float64))
    s = sc.view(np.float16)
    lo = np.min(lv); hi = np.max(lv)
    cont = np.minimum((lv - lo) / (hi - lo) * 16, 15)
    assert abs((acc / T - cont).mean()) < 0.05


def test_block_slice_draws_as_the_whole_parameter():
    # Without CoState every block of a parameter updates independently; a
    # block-aligned slice stepped with its block offset (and the parameter's
    # tensor id) must reproduce those blocks of the whole parameter exactly.
    rng = np.random.default_rng(3)
    nb, b0, b1 = 40, 13, 29
    n = nb * O.BS
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    kw = dict(lr=1e-3, compress_m=False, v_bits=4)
    whole = O.OracleTurboAdam([p0.copy()], seed=77, tensor_ids=[5], **kw)
    part = O.OracleTurboAdam([p0[b0 * O.BS:b1 * O.BS].copy()], seed=77, tensor_ids=[5], block0=[b0], **kw)
    shifted = O.OracleTurboAdam([p0[b0 * O.BS:b1 * O.BS].copy()], seed=77, tensor_ids=[5], **kw)
    for _ in range(3):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        whole.step([g])
        part.step([g[b0 * O.BS:b1 * O.BS].copy()])
        shifted.step([g[b0 * O.BS:b1 * O.BS].copy()])
    sl = slice(b0 * O.BS, b1 * O.BS)
    w, s = whole.state[0], part.state[0]
    assert np.array_equal(whole.param_groups[0]["params"][0][sl].view(np.uint32),
                          part.param_groups[0]["params"][0].view(np.uint32))
    assert np.array_equal(w["indices"][sl], s["indices"])
    assert np.array_equal(w["scales"][2 * b0:2 * b1], s["scales"])
    assert np.array_equal(w["exp_avg"][sl].view(np.uint32), s["exp_avg"].view(np.uint32))
    # the offset matters: without it the slice draws other uniforms
    assert not np.array_equal(w["indices"][sl], shifted.state[0]["indices"])


def test_division_by_sqrt_block_as_fp64_product():
    # The kernels form fl(x / fl(sqrt(128))) (costate.py:306) as the fp32
    # rounding of x times the fp64 reciprocal; equal to the fp32 division for
    # every non-negative fp32 x (norms), checked exhaustively (negative x
    # follows by symmetry).
    c = np.float32(math.sqrt(128.0))
    r = 1.0 / float(c)
    step = 1 << 22  # 0x7F800000 is a multiple
    base = np.arange(step, dtype=np.uint32)
    xu = np.empty(step, np.uint32)
    prod = np.empty(step, np.float64)
    a = np.empty(step, np.float32)
    q = np.empty(step, np.float32)
    x = xu.view(np.float32)
    for start in range(0, 0x7F800000, step):
        np.add(base, np.uint32(start), out=xu)
        np.copyto(prod, x)  # exact widening, then one fp64 product
        np.multiply(prod, r, out=prod)
        np.copyto(a, prod, casting="unsafe")
        np.divide(x, c, out=q)
        assert np.array_equal(a.view(np.uint32), q.view(np.uint32)), hex(start)
