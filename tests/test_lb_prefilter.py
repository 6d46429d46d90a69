"""The integer arithmetic of the lower-bound pass's hi-plane prefilter (csrc/batch.hip,
lb_scan_kernel's tile and lb_prep_kernel), restated with int32 semantics in numpy and checked
on random and adversarial data: every (query, row) whose exact sum passes,
    S = 256 acc_hi + acc_lo + kq >= th,
also passes the prefilter h >= thh - cb with
    h   = acc_hi + ceil(kq_pre / 256)          (the hi-plane chain's start)
    thh = floor((th - 1) / 256) + 1            (the hi-plane form of th)
    cb  = ceil(fl(cn * lo_w) (1 + 2^-20))      (the row's lo allowance, 0 without row norms)
where, with row norms, kq_pre = kq, cn >= |c'|_2 (float32, rounded up) and lo_w >= the group's
largest |lo|_2 / 256 (float32, rounded up); without them kq_pre = kq + 128 sum |lo|, lo_w = 0.
Planted mistakes (floor for the start, no allowance, the allowance without the / 256 scale)
must each lose some passing pair, so the checks can fail.
"""
import numpy as np
import pytest
import torch

from trident_amd.index import round_up_f32


def _f32_up(x64):
    return round_up_f32(torch.as_tensor(np.asarray(x64, np.float64))).numpy()


def _case(rng, n_rows, n_q, D, adversarial):
    c = rng.integers(-128, 128, size=(n_rows, D)).astype(np.int64)      # codes - 128
    w = rng.integers(-32639, 32640, size=(n_q, D)).astype(np.int64)     # w_int
    hi = (w + 128) >> 8
    lo = w - 256 * hi                                                    # in [-128, 127]
    assert lo.min() >= -128 and lo.max() <= 127
    if adversarial:  # rows aligned with a query's lo plane: Cauchy-Schwarz nearly tight
        c[: n_q] = np.where(lo >= 0, 127, -128)
    acc_hi = c @ hi.T                                                    # [rows, q]
    acc_lo = c @ lo.T
    kq = rng.integers(-(1 << 26), 1 << 26, size=n_q)
    S = 256 * acc_hi + acc_lo + kq
    # thresholds near the sums, so that both outcomes occur
    th = S[:, rng.integers(0, n_q)] + rng.integers(-(1 << 16), 1 << 16, size=n_rows)
    return c, lo, acc_hi, kq, S, th


def _prefilter(c, lo, acc_hi, kq, th, norms, start="ceil", allowance=True):
    if norms:
        kq_pre = kq
        cn = _f32_up(np.sqrt((c * c).sum(1).astype(np.float64)) * (1.0 + 2.0 ** -50))
        lo_l2 = np.sqrt((lo * lo).sum(1).astype(np.float64)) * (1.0 + 2.0 ** -50)
        lo_w = _f32_up((lo_l2 / 256.0).max())
        p = (cn.astype(np.float32) * np.float32(lo_w)).astype(np.float32)
        cb = np.ceil((p + p * np.float32(2.0 ** -20)).astype(np.float32)).astype(np.int64)
    else:
        kq_pre = kq + 128 * np.abs(lo).sum(1)
        cb = np.zeros(len(c), np.int64)
    if not allowance:
        cb = np.zeros_like(cb)
        kq_pre = kq
    start_v = (kq_pre + 255) >> 8 if start == "ceil" else kq_pre >> 8
    h = acc_hi + start_v[None, :]
    thh = ((th - 1) >> 8) + 1 - cb
    return h >= thh[:, None]


@pytest.mark.parametrize("D", [64, 96, 128, 256])
@pytest.mark.parametrize("norms", [True, False])
def test_prefilter_keeps_every_exact_pass(D, norms):
    rng = np.random.default_rng(D + 7 * norms)
    n_pass = 0
    for rep in range(6):
        c, lo, acc_hi, kq, S, th = _case(rng, 256, 32, D, adversarial=rep % 2 == 1)
        exact = S >= th[:, None]
        pre = _prefilter(c, lo, acc_hi, kq, th, norms)
        assert not np.any(exact & ~pre)
        n_pass += int(exact.sum())
    assert n_pass > 100


def test_row_norms_reject_more_than_the_per_query_bound():
    rng = np.random.default_rng(11)
    c, lo, acc_hi, kq, S, th = _case(rng, 512, 32, 128, adversarial=False)
    a = _prefilter(c, lo, acc_hi, kq, th, True).sum()
    b = _prefilter(c, lo, acc_hi, kq, th, False).sum()
    assert a < b


@pytest.mark.parametrize("mistake", ["floor_start", "no_allowance", "unscaled"])
def test_planted_mistakes_lose_passes(mistake):
    rng = np.random.default_rng(5)
    lost = 0
    for rep in range(8):
        c, lo, acc_hi, kq, S, th = _case(rng, 256, 32, 128, adversarial=rep % 2 == 1)
        exact = S >= th[:, None]
        if mistake == "floor_start":
            pre = _prefilter(c, lo, acc_hi, kq, th, False, start="floor", allowance=False)
        elif mistake == "no_allowance":
            pre = _prefilter(c, lo, acc_hi, kq, th, True, allowance=False)
        else:  # lo_w as |lo| / 256^2: the allowance 256 times too small
            lo_l2 = np.sqrt((lo * lo).sum(1).astype(np.float64)).max()
            cn = np.sqrt((c * c).sum(1).astype(np.float64))
            cb = np.ceil(cn * lo_l2 / 65536.0).astype(np.int64)
            thh = ((th - 1) >> 8) + 1 - cb
            pre = (acc_hi + ((kq + 255) >> 8)[None, :]) >= thh[:, None]
        lost += int((exact & ~pre).sum())
    assert lost > 0, mistake
