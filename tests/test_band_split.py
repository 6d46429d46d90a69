"""The bfloat16 split form of the coarse pass (csrc/frontend.hip, coarse_gemm_bf16_kernel and the
band derivation above mfma_tile_offset), restated in numpy and checked against its error bound:

    x = h + l + r,  h = bf16(x), l = bf16(x - h)  (round to nearest even),
    s' = (H0 + H1) + (L0 + L1)  over Dp = 32 ceil(Dq / 32) zero-padded dimensions, where H0 / H1
         accumulate h_c h_q of the even / odd 32-dim steps and L0 / L1 accumulate h_c l_q / l_c h_q,
         each step adding 32 exact float32 products to its float32 accumulator in any order,
    |s' - q.c| <= kappa sum |q_d c_d|,  kappa = (Dp + 4) 2^-23 (1 + 2^-5) + 3.125 2^-16.

The emulated sums use random addition orders inside each step.  Inputs: Gaussian, uniform
(the configs' value range) and two families of coherent low bits: every value just above a
bfloat16 tie (the dropped terms l_q l_c, ... all carry one sign: the largest error the split
leaves), or just below the next bfloat16 value (where a truncating split errs most).  Planted
mistakes must each break a bound, so the checks can fail: the float32 form's kappa
(Dq + 2) 2^-23 applied to the split sum, a truncating split, and a dropped L1 chain.
"""
import numpy as np
import pytest


def bf16_rne(x):
    """bfloat16 rounding of float32 x (as float32), nearest even; a finite value that would round
    to infinity is truncated instead (csrc/frontend.hip, bf16_rne)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    fin = (u & 0x7F800000) != 0x7F800000
    r = np.where(fin & ((r & 0x7F80) == 0x7F80), (u >> 16) & 0xFFFF, r)
    return (r.astype(np.uint32) << 16).view(np.float32)


def bf16_rtz(x):
    """Planted mistake: truncation instead of rounding."""
    return (np.asarray(x, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def split(x, rnd=bf16_rne):
    h = rnd(x)
    return h, rnd((np.asarray(x, np.float32) - h).astype(np.float32))


def kappa_split(Dq):
    NS = (Dq + 31) // 32
    return (32 * NS + 4) * 2.0 ** -23 * (1 + 2.0 ** -5) + 3.125 * 2.0 ** -16


def kappa_f32(Dq):
    return (Dq + 2) * 2.0 ** -23


def _step(acc, a, b, rng):
    """One matrix-core step: 32 exact products and the accumulator summed in float32, random order."""
    p = a.astype(np.float64) * b.astype(np.float64)
    p32 = p.astype(np.float32)
    assert np.array_equal(p32.astype(np.float64), p)  # bfloat16 x bfloat16 is exact in float32
    terms = np.concatenate([p32, np.array([acc], np.float32)])
    s = np.float32(0.0)
    for i in rng.permutation(terms.size):
        s = np.float32(s + terms[i])
    return s


def split_dot(q, c, rng, rnd=bf16_rne, drop_l1=False):
    """s' of the kernel's four chains for zero-padded rows q, c (length a multiple of 32)."""
    qh, ql = split(q, rnd)
    ch, cl = split(c, rnd)
    h = [np.float32(0.0), np.float32(0.0)]
    l0 = l1 = np.float32(0.0)
    for s in range(q.size // 32):
        sl = slice(32 * s, 32 * s + 32)
        h[s & 1] = _step(h[s & 1], ch[sl], qh[sl], rng)
        l0 = _step(l0, ch[sl], ql[sl], rng)
        if not drop_l1:
            l1 = _step(l1, cl[sl], qh[sl], rng)
    return np.float32(np.float32(h[0] + h[1]) + np.float32(l0 + l1))


def _coherent(rng, n):
    """Values whose low 16 bits sit just above the bfloat16 tie: h rounds up and
    x - h ~ -0.5 ulp_bf16(x) for every value."""
    v = rng.uniform(0.5, 200.0, n).astype(np.float32)
    u = (v.view(np.uint32) & np.uint32(0xFFFF0000)) | np.uint32(0x8000 + rng.integers(1, 0x100))
    return u.view(np.float32)


def _below_next(rng, n):
    """Values just below the next bfloat16 value: a truncating split leaves l ~ ulp_bf16(x) and
    r ~ 2^-8 l, all of one sign."""
    v = rng.uniform(0.5, 200.0, n).astype(np.float32)
    u = (v.view(np.uint32) & np.uint32(0xFFFF0000)) | np.uint32(0xFF00 + rng.integers(0, 0x100))
    return u.view(np.float32)


FAMILIES = ("gauss", "uniform", "coherent", "below_next")


def _rows(rng, kind, D):
    if kind == "gauss":
        return (rng.standard_normal((2, D)) * 100).astype(np.float32)
    if kind == "uniform":
        return np.stack([rng.uniform(0, 255, D), -0.5 * rng.uniform(0, 255, D)]).astype(np.float32)
    f = _coherent if kind == "coherent" else _below_next
    return np.stack([f(rng, D), f(rng, D)])


def _worst(kind, D, trials, **kw):
    """Largest |s' - q.c| / sum |q_d c_d| over random cases of one input family."""
    rng = np.random.default_rng([FAMILIES.index(kind), D])
    Dp = 32 * ((D + 31) // 32)
    worst = 0.0
    for _ in range(trials):
        q, c = _rows(rng, kind, D)
        qp = np.zeros(Dp, np.float32)
        cp = np.zeros(Dp, np.float32)
        qp[:D], cp[:D] = q, c
        prod = q.astype(np.float64) * c.astype(np.float64)  # exact in float64
        exact, den = float(prod.sum()), float(np.abs(prod).sum())
        worst = max(worst, abs(float(split_dot(qp, cp, rng, **kw)) - exact) / den)
    return worst


def test_split_components():
    """h and l are bfloat16, x - h is exact in float32, and the split's three bounds hold over
    every binade, ties, signs and zero; near FLT_MAX the split stays finite."""
    rng = np.random.default_rng(3)
    x = np.concatenate([
        (rng.standard_normal(20000) * np.exp2(rng.integers(-60, 60, 20000))).astype(np.float32),
        _coherent(rng, 2000),
        # exact ties: low half 0x8000, both parities of the kept bit
        ((rng.integers(0x3F800000, 0x47000000, 2000).astype(np.uint32) & np.uint32(0xFFFF0000))
         | np.uint32(0x8000)).view(np.float32),
        np.array([0.0, -0.0, 1.0, -3.5, 255.0, 3.0e38, -3.4e38], np.float32)])
    h, l = split(x)
    for t in (h, l):
        assert np.all((t.view(np.uint32) & 0xFFFF) == 0)
        assert np.all(np.isfinite(t))
    x64, h64, l64 = (t.astype(np.float64) for t in (x, h, l))
    assert np.array_equal((x - h).astype(np.float64), x64 - h64)  # exact residual
    big = np.abs(x64) > 1e38
    ok = ~big
    assert np.all(np.abs(x64 - h64)[ok] <= 2.0 ** -8 * np.abs(x64)[ok])
    assert np.all(np.abs(l64)[ok] <= 2.0 ** -8 * (1 + 2.0 ** -8) * np.abs(x64)[ok])
    assert np.all(np.abs(x64 - h64 - l64)[ok] <= 2.0 ** -16 * np.abs(x64)[ok])
    # ties round to the even bfloat16 neighbour
    tie = (x.view(np.uint32) & 0xFFFF) == 0x8000
    assert np.all((h[tie].view(np.uint32) >> 16) & 1 == 0)
    # a truncating split breaks the first bound (the planted mistake is visible)
    ht = bf16_rtz(x).astype(np.float64)
    assert np.any(np.abs(x64 - ht)[ok] > 2.0 ** -8 * np.abs(x64)[ok])


@pytest.mark.parametrize("D", [16, 100, 128])
def test_split_dot_within_kappa(D):
    """Every emulated kernel sum stays within kappa of the exact dot product."""
    for kind in FAMILIES:
        assert _worst(kind, D, 40) <= kappa_split(D), (kind, D)


def test_planted_mistakes_break_the_bounds():
    """The float32 form's kappa does not cover the split's dropped terms; a truncating split
    and a sum without the l_c h_q chain exceed even the split form's kappa."""
    D = 128
    assert _worst("coherent", D, 40) > kappa_f32(D)
    assert _worst("below_next", D, 40, rnd=bf16_rtz) > kappa_split(D)
    assert _worst("gauss", D, 10, drop_l1=True) > kappa_split(D)
