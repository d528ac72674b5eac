"""Sampling oracle (test infrastructure only).

Restates, in numpy:
  src/engine/sampling.rs:29-41    SamplingParams::normalized (top_p outside [0, 1] -> 1)
  src/engine/sampling.rs:239-269  Sampler::sample: temperature <= 0 or top_p == 0 -> argmax;
                                  otherwise scale by 1/temperature, softmax in fp32, joint filter
  src/engine/sampling.rs:409-428  apply_joint_filters: both cutoffs on the ORIGINAL distribution,
                                  ties at the boundary kept (k-th value, cumsum crossing clamped
                                  to vocab-1)
and the library's own drawing rule (an exponential race): the survivor with the largest
s + Gumbel(u) wins, u from Philox4x32-10 keyed by the seed with counter (element/4, row, offset).
The reference draws with FlashInfer's Philox stream, which no test pins bit-for-bit
(sampling.rs:554-659 checks only support, frequencies and same-seed repeatability), so the
stream itself is this library's design; the distribution it realises is the reference's.

Pinned by: the Random123 known-answer vectors for Philox4x32-10, the reference's fixtures
(sampling.rs:454-546 greedy/top-k=1/top-p=0 rows, 554-659 support and frequencies for
[4, 3, 2, 1, 0], 736-757 the joint 3/7 case), and brute-force enumeration of the joint filter
on tiny rows.
"""
from __future__ import annotations

import numpy as np

_M0 = np.uint64(0xD2511F53)
_M1 = np.uint64(0xCD9E8D57)
_W0 = 0x9E3779B9
_W1 = 0xBB67AE85
_MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(counter: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox4x32-10 on uint32 counters [..., 4] with a 2-word key (Salmon et al., SC'11)."""
    c = np.asarray(counter, np.uint64) & _MASK
    c0, c1, c2, c3 = (c[..., i].copy() for i in range(4))
    k0, k1 = np.uint64(key[0] & 0xFFFFFFFF), np.uint64(key[1] & 0xFFFFFFFF)
    for r in range(10):
        if r:
            k0 = np.uint64((int(k0) + _W0) & 0xFFFFFFFF)
            k1 = np.uint64((int(k1) + _W1) & 0xFFFFFFFF)
        p0 = _M0 * c0
        p1 = _M1 * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & _MASK
        hi1, lo1 = p1 >> np.uint64(32), p1 & _MASK
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def normalized(temperature: float, top_k: int, top_p: float, vocab: int):
    """(temperature, effective k, effective p) as the kernel and sampling.rs:29-41 use them."""
    if not (np.isfinite(top_p) and 0.0 <= top_p <= 1.0):
        top_p = 1.0
    k = vocab if (top_k <= 0 or top_k > vocab) else int(top_k)
    return float(temperature), k, float(top_p)


def scaled_logits(row: np.ndarray, temperature: float, round_to=None) -> np.ndarray:
    """s = cast(logit * fp32(1 / T)); ``round_to`` casts to the logits dtype (None: fp32)."""
    inv_t = np.float32(1.0) / np.float32(temperature)
    s = (np.asarray(row, np.float32) * inv_t).astype(np.float32)
    return round_to(s) if round_to is not None else s


def softmax_f32(s: np.ndarray) -> np.ndarray:
    s = np.asarray(s, np.float32)
    m = np.max(s)
    e = np.exp((s - m).astype(np.float32)).astype(np.float32)
    return (e / np.sum(e, dtype=np.float32)).astype(np.float32)


def joint_keep(s: np.ndarray, top_k: int, top_p: float) -> np.ndarray:
    """Boolean survivors of apply_joint_filters (sampling.rs:411-428) on scaled logits s."""
    s = np.asarray(s, np.float32)
    vocab = s.shape[-1]
    remove = np.zeros(vocab, bool)
    if 0 < top_k < vocab:
        kth = np.sort(s)[::-1][top_k - 1]
        remove |= s < kth
    if top_p < 1.0:
        probs = softmax_f32(s)
        srt = np.sort(probs)[::-1]
        cums = np.cumsum(srt, dtype=np.float32)
        crossing = min(int(np.sum(cums < np.float32(top_p))), vocab - 1)
        remove |= probs < srt[crossing]
    return ~remove


def filtered_distribution(s: np.ndarray, top_k: int, top_p: float) -> np.ndarray:
    """softmax of the filtered logits (the reference test's `expected`, sampling.rs:569-576)."""
    keep = joint_keep(s, top_k, top_p)
    masked = np.where(keep, np.asarray(s, np.float32), -np.inf).astype(np.float32)
    return softmax_f32(masked)


def gumbel_noise(vocab: int, row: int, seed: int, offset: int) -> np.ndarray:
    """Per-element Gumbel variates of the race, float32 (same bit recipe as the kernel)."""
    groups = (vocab + 3) // 4
    ctr = np.zeros((groups, 4), np.uint64)
    ctr[:, 0] = np.arange(groups, dtype=np.uint64)
    ctr[:, 1] = row & 0xFFFFFFFF
    ctr[:, 2] = offset & 0xFFFFFFFF
    ctr[:, 3] = (offset >> 32) & 0xFFFFFFFF
    bits = philox4x32_10(ctr, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)).reshape(-1)[:vocab]
    u = ((bits >> np.uint32(9)).astype(np.float32) + np.float32(0.5)) * np.float32(2.0 ** -23)
    return (-np.log(-np.log(u.astype(np.float64)))).astype(np.float32)


def sample_rows(logits: np.ndarray, temperature, top_k, top_p, seed: int, offset: int,
                round_to=None) -> tuple[np.ndarray, list[float]]:
    """Token per row by the library's rule; also the race margin (best - runner-up key) per row,
    so a caller can tell a genuine mismatch from a float-level near tie."""
    logits = np.asarray(logits, np.float32)
    rows, vocab = logits.shape
    out = np.zeros(rows, np.int64)
    margins: list[float] = []
    for r in range(rows):
        t, k, p = normalized(float(temperature[r]), int(top_k[r]), float(top_p[r]), vocab)
        x = logits[r]
        if t <= 0 or p == 0.0:
            out[r] = int(np.argmax(x))
            margins.append(float("inf"))
            continue
        s = scaled_logits(x, t, round_to)
        # Invalid: NaN anywhere, no finite logit, or a +inf (the reference's softmax of the
        # scaled row, sampling.rs:261, is NaN throughout once inf - inf appears).
        if np.isnan(s).any() or np.isposinf(s).any() or not np.isfinite(s).any():
            out[r] = -1
            margins.append(float("inf"))
            continue
        keep = joint_keep(s, k, p) & np.isfinite(s)
        if k < vocab or p < 1.0:
            keep &= softmax_f32(s) > 0
        key = np.where(keep, s.astype(np.float64) + gumbel_noise(vocab, r, seed, offset), -np.inf)
        order = np.argsort(-key, kind="stable")
        out[r] = int(order[0])
        margins.append(float(key[order[0]] - key[order[1]]) if vocab > 1 else float("inf"))
    return out, margins
