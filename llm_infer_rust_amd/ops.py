"""Shared norm operators on the gfx950 kernels.

Mirrors the reference's ``src/layers/ops.rs:8-51`` functions and the
validation of its ATen bridge ``src/layers/fused_ops_bridge.cpp:56-118``:

* ``rms_norm(x, weight, eps)`` returns a new contiguous tensor;
* ``add_rms_norm(x, residual, weight, eps)`` updates both buffers in place and
  returns ``(x, residual)``; the norm uses the unrounded fp32 sum;
* ``qk_norm(q, k, q_weight, k_weight, eps)`` normalises q and k views of a
  packed QKV buffer in place and returns ``(q, k)``; V is never written.

Only CUDA(HIP) bfloat16/float16 tensors are accepted; anything else raises.
"""
from __future__ import annotations

import torch

from . import _native
from ._native import NativeError, check, dtype_code, lib, stream_of


def _require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise NativeError(f"{what}: expected a GPU tensor")


def _check_weight(x: torch.Tensor, w: torch.Tensor, dim: int) -> None:
    if (not w.is_cuda or w.device != x.device or w.dtype != x.dtype or w.dim() != 1
            or w.size(0) != dim or not w.is_contiguous()):
        raise NativeError("invalid shared layer norm weight")


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * w over the last dim (fp32 math)."""
    _require_device(x, "rms_norm")
    dt = dtype_code(x)
    if x.dim() != 2 or x.stride(1) != 1:
        raise NativeError("invalid shared layer RMSNorm input")
    _check_weight(x, weight, x.size(1))
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    check(lib().mi355x_rms_norm(x.data_ptr(), weight.data_ptr(), out.data_ptr(), x.size(0), 1,
                                x.size(1), x.stride(0), 0, float(eps), dt, stream_of(x)),
          "rms_norm")
    return out


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                 eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """In place: residual <- round(x + residual); x <- round(rms(x + residual) * w)."""
    _require_device(x, "add_rms_norm")
    dt = dtype_code(x)
    if (x.dim() != 2 or x.stride(1) != 1 or not residual.is_cuda or residual.device != x.device
            or residual.dtype != x.dtype or residual.shape != x.shape or residual.stride(1) != 1
            or x.data_ptr() == residual.data_ptr()):
        raise NativeError("invalid shared layer fused add-RMSNorm inputs")
    _check_weight(x, weight, x.size(1))
    check(lib().mi355x_add_rms_norm(x.data_ptr(), residual.data_ptr(), weight.data_ptr(),
                                    x.size(0), x.size(1), x.stride(0), residual.stride(0),
                                    float(eps), dt, stream_of(x)), "add_rms_norm")
    return x, residual


def qk_norm(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
            eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """In-place per-head RMSNorm of q [T, Hq, D] and k [T, Hkv, D] views."""
    _require_device(q, "qk_norm")
    dt = dtype_code(q)
    if (q.dim() != 3 or k.dim() != 3 or q.size(0) != k.size(0) or q.size(2) != k.size(2)
            or q.device != k.device or q.dtype != k.dtype or q.stride(2) != 1
            or k.stride(2) != 1):
        raise NativeError("invalid shared layer query/key shapes or strides")
    _check_weight(q, q_weight, q.size(2))
    _check_weight(k, k_weight, k.size(2))
    check(lib().mi355x_qk_norm(q.data_ptr(), k.data_ptr(), q_weight.data_ptr(),
                               k_weight.data_ptr(), q.size(0), q.size(1), k.size(1), q.size(2),
                               q.stride(0), q.stride(1), k.stride(0), k.stride(1), float(eps),
                               dt, stream_of(q)), "qk_norm")
    return q, k


__all__ = ["rms_norm", "add_rms_norm", "qk_norm", "NativeError", "_native"]
