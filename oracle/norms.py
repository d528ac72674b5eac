"""Norm oracle (test infrastructure only), numpy fp32 in the reference's op order.

src/layers/ops.rs:8-18   rms_norm: x_f32 * rsqrt(mean(x_f32^2) + eps) * w_f32, cast
src/layers/ops.rs:22-35  add_rms_norm: s = x_f32 + r_f32; normalise s (unrounded);
                         residual <- cast(s)
src/layers/ops.rs:39-51  qk_norm: rms_norm per head of q with q_w and of k with k_w
Inputs are float32 arrays holding values already representable in the
activation dtype; outputs are float32 before the final cast (use
``oracle.bf16.round_to`` for the cast). The ``*_torch`` functions restate the
same op order in libtorch on CPU tensors of the activation dtype; they are the
timed CPU baseline, not a checker.
"""
from __future__ import annotations

import numpy as np


def rms_norm_f32(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, np.float32)
    var = np.mean(np.square(x, dtype=np.float32), axis=-1, keepdims=True, dtype=np.float32)
    scale = (1.0 / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return (x * scale * np.asarray(w, np.float32)).astype(np.float32)


def add_rms_norm_f32(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float):
    """Return (normalised sum before cast, fp32 sum before cast)."""
    s = (np.asarray(x, np.float32) + np.asarray(r, np.float32)).astype(np.float32)
    return rms_norm_f32(s, w, eps), s


def qk_norm_f32(q: np.ndarray, k: np.ndarray, qw: np.ndarray, kw: np.ndarray, eps: float):
    return rms_norm_f32(q, qw, eps), rms_norm_f32(k, kw, eps)


def rms_norm_torch(x, w, eps: float):
    """ops.rs:8-18 in libtorch: fp32 compute, cast back to x's dtype."""
    import torch

    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    return (xf * torch.rsqrt(var + eps) * w.float()).to(x.dtype)


def add_rms_norm_torch(x, r, w, eps: float):
    """ops.rs:22-35 in libtorch: returns (normalised, new residual)."""
    s = x.float() + r.float()
    return rms_norm_torch_f32(s, w, eps).to(x.dtype), s.to(x.dtype)


def rms_norm_torch_f32(s, w, eps: float):
    import torch

    var = s.pow(2).mean(-1, keepdim=True)
    return s * torch.rsqrt(var + eps) * w.float()


def qk_norm_torch(q, k, qw, kw, eps: float):
    """ops.rs:39-51 in libtorch: per-head RMSNorm of q and k."""
    return rms_norm_torch(q, qw, eps), rms_norm_torch(k, kw, eps)
