"""Pins of the RoPE / SiLU / sampling oracles (CPU only).

Every check is independent of the oracle's own formula: known-answer vectors, the reference's
fixtures, closed forms, algebraic invariants or brute force over tiny inputs.
"""
import math

import numpy as np
import pytest
from scipy.special import expit

from oracle import layer_ops as olay
from oracle import sampling as osamp


# --------------------------------------------------------------------------- Philox
@pytest.mark.parametrize("ctr,key,want", [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
])
def test_philox4x32_10_known_answers(ctr, key, want):
    # Random123 kat_vectors for philox4x32 with 10 rounds.
    got = osamp.philox4x32_10(np.array(ctr, np.uint64), key)
    assert tuple(int(x) for x in got) == want


def test_gumbel_noise_is_uniform_in_distribution():
    g = osamp.gumbel_noise(200_000, 0, 7, 0).astype(np.float64)
    # Gumbel(0,1): mean = Euler-Mascheroni gamma, variance = pi^2/6.
    assert abs(g.mean() - 0.5772156649) < 0.01
    assert abs(g.var() - math.pi ** 2 / 6) < 0.03
    assert np.isfinite(g).all()


# --------------------------------------------------------------------------- joint filter
FIVE = np.array([4.0, 3.0, 2.0, 1.0, 0.0], np.float32)


@pytest.mark.parametrize("k,p,kept", [
    (-1, 1.0, {0, 1, 2, 3, 4}),
    (-1, 0.8, {0, 1}),        # sorted probs .636 .234 .086 ...: cumsum < .8 once -> keep 2
    (3, 0.9, {0, 1, 2}),      # top-3, and cumsum < .9 twice -> keep 3
    (1, 1.0, {0}),
])
def test_joint_filter_reference_fixture(k, p, kept):
    # sampling.rs:561-599 uses exactly these (top_k, top_p) pairs on [4, 3, 2, 1, 0].
    _, kk, pp = osamp.normalized(1.0, k, p, 5)
    keep = osamp.joint_keep(FIVE, kk, pp)
    assert set(np.flatnonzero(keep)) == kept
    dist = osamp.filtered_distribution(FIVE, kk, pp)
    e = np.exp(FIVE.astype(np.float64))
    idx = sorted(kept)
    want = np.zeros(5)
    want[idx] = e[idx] / e[idx].sum()
    np.testing.assert_allclose(dist, want, atol=1e-6)


def test_joint_filter_uses_original_mass():
    # sampling.rs:736-757: p=.5 keeps .4 and .3 on the ORIGINAL distribution; k=2 keeps both.
    s = np.log(np.array([0.4, 0.3, 0.2, 0.1], np.float32)).astype(np.float32)
    dist = osamp.filtered_distribution(s, 2, 0.5)
    np.testing.assert_allclose(dist, [4 / 7, 3 / 7, 0, 0], atol=1e-6)


def brute_keep(s, k, p):
    """Definition by enumeration: top-k keeps v when fewer than k values exceed it; top-p keeps
    v when it is >= the largest value whose mass-at-or-above reaches p (clamp: keep all)."""
    s = np.asarray(s, np.float32)
    probs = osamp.softmax_f32(s)
    n = len(s)
    keep = np.ones(n, bool)
    if k < n:
        keep &= np.array([np.sum(s > v) < k for v in s])
    if p < 1.0:
        # mass(x >= v) accumulated in descending sorted order, ties together.
        srt = np.sort(probs)[::-1]
        cums = np.cumsum(srt, dtype=np.float32)
        candidates = [srt[i] for i in range(n) if cums[i] >= np.float32(p)]
        cut = candidates[0] if candidates else srt[-1]
        keep &= probs >= cut
    return keep


@pytest.mark.parametrize("seed", range(12))
def test_joint_filter_matches_enumeration(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(2, 9))
    s = rng.integers(-3, 3, n).astype(np.float32) * np.float32(0.5)  # many ties
    for k in range(1, n + 1):
        for p in (0.05, 0.3, 0.5, 0.75, 0.9, 0.99, 1.0):
            np.testing.assert_array_equal(osamp.joint_keep(s, k, p), brute_keep(s, k, p))


def test_params_normalisation():
    assert osamp.normalized(0.7, 50, 0.9, 100) == (0.7, 50, 0.9)
    assert osamp.normalized(0.7, -1, float("nan"), 100) == (0.7, 100, 1.0)
    assert osamp.normalized(0.7, 0, 1.5, 100) == (0.7, 100, 1.0)
    assert osamp.normalized(0.7, 500, -0.1, 100) == (0.7, 100, 1.0)


def test_greedy_rows_reference_fixture():
    # sampling.rs:454-546: logits [[0.1, 2.0, 0.2], [3.0, 1.0, 0.5]] -> [1, 0] for temperature 0,
    # for top_k = 1 and for top_p = 0.
    logits = np.array([[0.1, 2.0, 0.2], [3.0, 1.0, 0.5]], np.float32)
    for t, k, p in ((0.0, -1, 1.0), (1.0, -1, 0.0)):
        ids, _ = osamp.sample_rows(logits, [t, t], [k, k], [p, p], 1, 0)
        assert ids.tolist() == [1, 0]
    ids, _ = osamp.sample_rows(logits, [1.0, 1.0], [1, 1], [1.0, 1.0], 1, 0)
    assert ids.tolist() == [1, 0]


def test_race_realises_the_filtered_distribution():
    rows = 4000
    logits = np.tile(FIVE, (rows, 1))
    for k, p in ((-1, 1.0), (-1, 0.8), (3, 0.9)):
        ids, _ = osamp.sample_rows(logits, [1.0] * rows, [k] * rows, [p] * rows, 12345, 3)
        _, kk, pp = osamp.normalized(1.0, k, p, 5)
        want = osamp.filtered_distribution(FIVE, kk, pp)
        freq = np.bincount(ids, minlength=5) / rows
        assert np.all(freq[want == 0] == 0)
        assert np.abs(freq - want).max() < 0.03, (k, p, freq, want)


def test_invalid_rows_give_sentinel():
    logits = np.array([[0.0, np.nan, 1.0], [-np.inf, -np.inf, -np.inf]], np.float32)
    ids, _ = osamp.sample_rows(logits, [1.0, 1.0], [-1, -1], [0.9, 1.0], 0, 0)
    assert ids.tolist() == [-1, -1]


def test_positive_infinity_makes_the_row_invalid():
    """The reference softmaxes the scaled row in torch (sampling.rs:261): a +inf entry gives
    inf - inf = NaN, so the whole distribution is NaN and the row is invalid (-1) for every
    filter; greedy rows take the raw argmax and are unaffected. An fp16 row scaled by a small
    temperature overflows to +inf the same way."""
    import torch
    row = torch.tensor([[0.0, float("inf"), 1.0, 2.0]])
    assert bool(torch.isnan(torch.softmax(row, -1)).all())
    half = torch.tensor([[1.0, 30.0, 2.0]], dtype=torch.float16)
    assert bool(torch.isinf(half / 1e-4).any())  # 3e5 > fp16 max
    logits = np.array([[0.0, np.inf, 1.0, 2.0]] * 4, np.float32)
    ids, _ = osamp.sample_rows(logits, [1.0, 1.0, 1.0, 0.0], [-1, 2, -1, -1], [1.0, 1.0, 0.9, 1.0],
                               0, 0)
    assert ids.tolist() == [-1, -1, -1, 1]
    h = np.array([[1.0, 30.0, 2.0]], np.float32)
    with np.errstate(over="ignore"):  # the fp16 cast overflows on purpose
        ids, _ = osamp.sample_rows(h, [1e-4], [-1], [1.0], 0, 0,
                                   lambda v: v.astype(np.float16).astype(np.float32))
    assert ids.tolist() == [-1]


# --------------------------------------------------------------------------- RoPE
def test_rope_reference_fixture_eager_formula():
    # ops.rs:498-530: q = arange(32).view(4,2,4), k = arange(16).view(4,1,4), positions
    # [0, 15, 3, 15], D = 4, theta 1e4; the eager formula recomputed here in float64.
    q = np.arange(32, dtype=np.float32).reshape(4, 2, 4)
    k = np.arange(16, dtype=np.float32).reshape(4, 1, 4)
    pos = np.array([0, 15, 3, 15])
    cos, sin = olay.rope_tables(16, 4, 10_000.0)
    for x in (q, k):
        got = olay.rope(x, pos, cos, sin)
        ang = pos[:, None].astype(np.float64) * (10_000.0 ** (-np.arange(0, 4, 2) / 4.0))[None]
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        x1, x2 = x[..., :2].astype(np.float64), x[..., 2:].astype(np.float64)
        want = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)
        np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-5)


def test_rope_invariants():
    rng = np.random.default_rng(0)
    cos, sin = olay.rope_tables(4096, 128, 1_000_000.0)
    x = rng.standard_normal((6, 3, 128)).astype(np.float32)
    # position 0 is the identity
    np.testing.assert_array_equal(olay.rope(x, np.zeros(6, np.int64), cos, sin), x)
    # every (i, i + 64) pair keeps its norm
    pos = rng.integers(0, 4096, 6)
    y = olay.rope(x, pos, cos, sin)
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = y[..., :64] ** 2 + y[..., 64:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-4, atol=1e-5)
    # q(m).k(n) depends only on m - n
    q = rng.standard_normal((1, 1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 1, 128)).astype(np.float32)
    dots = []
    for m, n in ((10, 3), (110, 103), (1010, 1003)):
        qm = olay.rope(q, np.array([m]), cos, sin)
        kn = olay.rope(k, np.array([n]), cos, sin)
        dots.append(float((qm * kn).sum()))
    np.testing.assert_allclose(dots, dots[0], rtol=1e-3, atol=1e-3)
    # positions outside the table leave rows untouched (fused_ops.cu:118-120)
    np.testing.assert_array_equal(olay.rope(x[:2], np.array([-1, 4096]), cos, sin), x[:2])


def test_silu_closed_form():
    rng = np.random.default_rng(1)
    gu = rng.standard_normal((5, 26)).astype(np.float32) * 4
    got = olay.silu_mul(gu)
    g, u = gu[:, :13].astype(np.float64), gu[:, 13:].astype(np.float64)
    np.testing.assert_allclose(got, g * expit(g) * u, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(olay.silu_mul(np.array([[0.0, 3.0]], np.float32)), [[0.0]])
    big = olay.silu_mul(np.array([[30.0, 1.0]], np.float32))
    assert abs(big[0, 0] - 30.0) < 1e-5
