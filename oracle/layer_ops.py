"""Decoder-layer elementwise oracle (test infrastructure only): RoPE and SiLU*up.

src/layers/ops.rs:65-97   HalfSplitRope::new: inv_freq = exp(arange(0, D, 2) * (-ln(theta) / D)),
                          freqs = positions x inv_freq, cos/sin tables in fp32 (GPU path)
src/layers/ops.rs:99-127  apply / rotate_half: [x1 c - x2 s, x2 c + x1 s] on the two halves
src/layers/fused_ops.cu:108-133  the GPU kernel: positions outside the table leave the row unchanged
src/layers/ops.rs:53-61   silu_and_mul: silu(gate) * up on a packed [T, 2W] input

Pinned by: the reference's own fixtures (ops.rs:483-530: the eager formula for reordered and last
positions), position 0 = identity, norm preservation of every rotated pair, R(a) R(b) = R(a + b),
and the relative-position property q(m).k(n) = q(m + s).k(n + s); silu against scipy.special.expit
and its closed-form points silu(0) = 0, silu(x) -> x.
"""
from __future__ import annotations

import numpy as np


def rope_tables(max_positions: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """fp32 cos/sin tables [max_positions, head_dim/2] (ops.rs:77-93, GPU cache kind Float)."""
    inv_freq = np.exp(np.arange(0, head_dim, 2, dtype=np.float32)
                      * np.float32(-(np.log(theta) / head_dim))).astype(np.float32)
    positions = np.arange(max_positions, dtype=np.float32)
    freqs = (positions[:, None] * inv_freq[None, :]).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def rotate_half(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """ops.rs:118-127 with cos/sin broadcast over heads; float32 result before the cast."""
    half = x.shape[-1] // 2
    x = np.asarray(x, np.float32)
    first, second = x[..., :half], x[..., half:]
    return np.concatenate([first * cos - second * sin, second * cos + first * sin],
                          axis=-1).astype(np.float32)


def rope(x: np.ndarray, positions: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate x [T, H, D] by per-token positions; out-of-table positions are left unchanged
    (fused_ops.cu:118-120)."""
    x = np.asarray(x, np.float32)
    out = x.copy()
    positions = np.asarray(positions, np.int64)
    valid = (positions >= 0) & (positions < cos.shape[0])
    idx = np.where(valid)[0]
    if idx.size:
        c = cos[positions[idx]][:, None, :]
        s = sin[positions[idx]][:, None, :]
        out[idx] = rotate_half(x[idx], c, s)
    return out


def silu_mul(gate_up: np.ndarray) -> np.ndarray:
    """silu(gate) * up in float32 (ops.rs:53-61)."""
    gate_up = np.asarray(gate_up, np.float32)
    w = gate_up.shape[-1] // 2
    g, u = gate_up[..., :w], gate_up[..., w:]
    return (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
