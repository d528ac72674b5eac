"""Shared norm operators on the gfx950 kernels.

Mirrors the reference's ``src/layers/ops.rs:8-51`` functions and the
validation of its ATen bridge ``src/layers/fused_ops_bridge.cpp:56-118``:

* ``rms_norm(x, weight, eps)`` returns a new contiguous tensor;
* ``add_rms_norm(x, residual, weight, eps)`` updates both buffers in place and
  returns ``(x, residual)``; the norm uses the unrounded fp32 sum;
* ``qk_norm(q, k, q_weight, k_weight, eps)`` normalises q and k views of a
  packed QKV buffer in place and returns ``(q, k)``; V is never written.

and ``src/layers/ops.rs:53-127``:

* ``silu_and_mul(gate_up)`` returns a new ``[T, W]`` tensor;
* ``HalfSplitRope`` holds fp32 cos/sin tables and rotates q/k in place;
* ``qk_norm_rope_store`` runs the decoder layer's qk_norm -> rope -> K/V store
  as one pass (``src/models/qwen3/model.rs:478-514``).

Only CUDA(HIP) bfloat16/float16 tensors are accepted; anything else raises.
"""
from __future__ import annotations

import math

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


def silu_and_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(gate) * up for a packed ``[T, 2W]`` input (ops.rs:53-61)."""
    _require_device(gate_up, "silu_and_mul")
    dt = dtype_code(gate_up)
    if gate_up.dim() != 2 or gate_up.size(1) % 2 != 0 or not gate_up.is_contiguous():
        raise NativeError("invalid SiLU input: expected a contiguous [T, 2W] tensor")
    width = gate_up.size(1) // 2
    if out is None:
        out = torch.empty((gate_up.size(0), width), dtype=gate_up.dtype, device=gate_up.device)
    elif (out.shape != (gate_up.size(0), width) or out.dtype != gate_up.dtype
          or not out.is_contiguous() or out.device != gate_up.device):
        raise NativeError("invalid SiLU output")
    check(lib().mi355x_silu_mul(gate_up.data_ptr(), out.data_ptr(), gate_up.size(0), width, dt,
                                stream_of(gate_up)), "silu_and_mul")
    return out


class HalfSplitRope:
    """Shared rotary tables (ops.rs:65-97): fp32 cos/sin ``[max_positions, D/2]`` on the GPU."""

    def __init__(self, max_positions: int, head_dim: int, rope_theta: float,
                 device: torch.device | str):
        if head_dim % 2 != 0 or max_positions <= 0:
            raise NativeError("invalid RoPE geometry")
        inv_freq = torch.exp(torch.arange(0, head_dim, 2, dtype=torch.float32)
                             * (-(math.log(rope_theta) / head_dim)))
        positions = torch.arange(max_positions, dtype=torch.float32)
        freqs = positions.unsqueeze(-1) * inv_freq.unsqueeze(0)
        self.cos = freqs.cos().to(device)
        self.sin = freqs.sin().to(device)
        self.half_dim = head_dim // 2
        self.max_positions = max_positions

    def apply(self, q: torch.Tensor, k: torch.Tensor,
              positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Rotate q [T, Hq, D] and k [T, Hkv, D] views in place; returns (q, k)."""
        return rope(q, k, positions, self.cos, self.sin)


def _check_heads(q: torch.Tensor, k: torch.Tensor, what: str) -> None:
    if (q.dim() != 3 or k.dim() != 3 or q.size(0) != k.size(0) or q.size(2) != k.size(2)
            or q.device != k.device or q.dtype != k.dtype or q.stride(2) != 1
            or k.stride(2) != 1):
        raise NativeError(f"invalid {what} query/key shapes or strides")


def _check_positions(q: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
                     sin: torch.Tensor) -> None:
    if (positions.dtype != torch.int64 or positions.dim() != 1 or positions.numel() != q.size(0)
            or not positions.is_contiguous() or positions.device != q.device):
        raise NativeError("RoPE positions must be a contiguous int64 vector, one per token")
    half = q.size(2) // 2
    for table in (cos, sin):
        if (table.dtype != torch.float32 or table.dim() != 2 or table.size(1) != half
                or not table.is_contiguous() or table.device != q.device):
            raise NativeError("RoPE tables must be contiguous fp32 [max_positions, D/2]")


def rope(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor,
         sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """In-place half-split RoPE (fused_ops.cu:108-133 semantics)."""
    _require_device(q, "rope")
    dt = dtype_code(q)
    _check_heads(q, k, "RoPE")
    _check_positions(q, positions, cos, sin)
    check(lib().mi355x_rope(q.data_ptr(), k.data_ptr(), positions.data_ptr(), cos.data_ptr(),
                            sin.data_ptr(), q.size(0), q.size(1), k.size(1), q.size(2),
                            q.stride(0), q.stride(1), k.stride(0), k.stride(1), cos.size(0), dt,
                            stream_of(q)), "rope")
    return q, k


def qk_norm_rope_store(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       q_weight: torch.Tensor | None, k_weight: torch.Tensor | None, eps: float,
                       positions: torch.Tensor | None, rope_tables: HalfSplitRope | None,
                       attention=None, write_loc: torch.Tensor | None = None) -> None:
    """qk_norm -> rope -> K/V store in one pass; q and k are rewritten in place.

    ``attention`` is a bound ``kv_cache.BaseAttention`` (its caches, reserved slot and error
    word are used); the store is skipped when it is None or ``write_loc`` is None, as
    ``BaseAttention.write_kv`` skips it."""
    _require_device(q, "qk_norm_rope_store")
    dt = dtype_code(q)
    _check_heads(q, k, "QK-norm/RoPE")
    if v.shape != k.shape or v.stride(2) != 1 or v.dtype != k.dtype:
        raise NativeError("K/V input must have matching (tokens, kv_heads, head_dim) shapes")
    if (q_weight is None) != (k_weight is None):
        raise NativeError("q_weight and k_weight go together")
    if q_weight is not None:
        _check_weight(q, q_weight, q.size(2))
        _check_weight(k, k_weight, k.size(2))
    cos = sin = None
    max_pos = 0
    if rope_tables is not None:
        if positions is None:
            raise NativeError("RoPE needs positions")
        cos, sin, max_pos = rope_tables.cos, rope_tables.sin, rope_tables.max_positions
        _check_positions(q, positions, cos, sin)
    kc = vc = errors = None
    reserved, capacity, index64 = -1, 0, False
    if attention is not None and write_loc is not None and attention.is_bound():
        kc, vc = attention.cache_tensors()
        if kc.size(2) != k.size(1) or kc.size(3) != k.size(2) or kc.dtype != k.dtype:
            raise NativeError("K/V input head shape does not match the bound cache")
        if (write_loc.dim() != 1 or write_loc.numel() != k.size(0) or not write_loc.is_contiguous()
                or write_loc.dtype not in (torch.int32, torch.int64)
                or write_loc.device != k.device):
            raise NativeError("invalid KV store locations")
        reserved = attention.reserved_write_slot()
        capacity = kc.size(0) * kc.size(1)
        index64 = write_loc.dtype == torch.int64
        errors = attention.error_word()

    def ptr(t):
        return None if t is None else t.data_ptr()

    check(lib().mi355x_qk_norm_rope_store(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), ptr(q_weight), ptr(k_weight),
        ptr(positions) if rope_tables is not None else None, ptr(cos), ptr(sin), max_pos,
        ptr(kc), ptr(vc), ptr(write_loc) if kc is not None else None, index64, capacity,
        reserved, ptr(errors), q.size(0), q.size(1), k.size(1), q.size(2), q.stride(0),
        q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1), float(eps), dt,
        stream_of(q)), "qk_norm_rope_store")


def linear_qk_norm_rope_store(x: torch.Tensor, weight: torch.Tensor, q_heads: int,
                              k_heads: int, q_weight: torch.Tensor, k_weight: torch.Tensor,
                              eps: float, positions: torch.Tensor, rope_tables: HalfSplitRope,
                              attention, write_loc: torch.Tensor | None) -> torch.Tensor:
    """The decoder layer's ``qkv = linear(x, W_qkv)`` followed by ``qk_norm_rope_store`` on its
    q/k/v head views; returns ``qkv`` ``[T, (Hq + 2 Hkv) 128]``. Decode-sized products with a
    bound cache run as one projection plus one pass that also sums the split-K partials
    (``mi355x_linear_qk_norm_rope_store``, bit-identical to the two steps); everything else
    runs the two steps."""
    m, k = (x.shape if x.dim() == 2 else (0, 0))
    n = weight.size(0)
    if q_heads <= 0 or k_heads <= 0 or n % (q_heads + 2 * k_heads):
        raise NativeError("QKV weight rows must be (q_heads + 2 k_heads) * head_dim")
    d = n // (q_heads + 2 * k_heads)  # head_dim
    fused = (x.is_cuda and x.dim() == 2 and x.stride(1) == 1 and x.stride(0) % 8 == 0
             and weight.is_contiguous() and d == 128
             and uses_decode_kernel(m, n, k) and attention is not None
             and write_loc is not None and attention.is_bound() and rope_tables is not None)
    if not fused:
        qkv = linear(x, weight)
        t = qkv.size(0)
        qk_norm_rope_store(qkv[:, :q_heads * d].view(t, q_heads, d),
                           qkv[:, q_heads * d:(q_heads + k_heads) * d].view(t, k_heads, d),
                           qkv[:, (q_heads + k_heads) * d:].view(t, k_heads, d), q_weight,
                           k_weight, eps, positions, rope_tables, attention, write_loc)
        return qkv
    _require_device(x, "linear_qk_norm_rope_store")
    dt = dtype_code(x)
    if weight.dtype != x.dtype or weight.device != x.device or weight.size(1) != k:
        raise NativeError("invalid linear operands: expected x [M, K] and weight [N, K]")
    qkv = torch.empty((m, n), dtype=x.dtype, device=x.device)
    q_view = qkv[:, :q_heads * d].view(m, q_heads, d)
    _check_weight(q_view, q_weight, d)
    _check_weight(q_view, k_weight, d)
    cos, sin, max_pos = rope_tables.cos, rope_tables.sin, rope_tables.max_positions
    _check_positions(q_view, positions, cos, sin)
    kc, vc = attention.cache_tensors()
    if (kc.size(2) != k_heads or kc.size(3) != d or kc.dtype != x.dtype
            or kc.device != x.device):
        raise NativeError("K/V input head shape does not match the bound cache")
    if (write_loc.dim() != 1 or write_loc.numel() != m or not write_loc.is_contiguous()
            or write_loc.dtype not in (torch.int32, torch.int64) or write_loc.device != x.device):
        raise NativeError("invalid KV store locations")
    cus = _native.device_cus(x.device)
    need = lib().mi355x_linear_workspace_bytes(m, n, k, cus, -1, -1)
    ws = torch.empty(max(int(need), 16), dtype=torch.uint8, device=x.device) if need else None
    check(lib().mi355x_linear_qk_norm_rope_store(
        x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), qkv.data_ptr(), n, m, k,
        q_heads, k_heads, None if ws is None else ws.data_ptr(), int(need), cus,
        q_weight.data_ptr(), k_weight.data_ptr(), positions.data_ptr(), cos.data_ptr(),
        sin.data_ptr(), max_pos, kc.data_ptr(), vc.data_ptr(), write_loc.data_ptr(),
        write_loc.dtype == torch.int64, kc.size(0) * kc.size(1),
        attention.reserved_write_slot(),
        None if attention.error_word() is None else attention.error_word().data_ptr(), float(eps), dt,
        stream_of(x)), "linear_qk_norm_rope_store")
    return qkv


# Decode batches (at most this many rows) with an output of at most DECODE_MAX_N
# columns go to the gfx950 projection kernel; long-K products (K > 4096) only from
# DECODE_LONG_K_MIN_ROWS rows up. Everything else stays on hipBLASLt through
# F.linear. The bounds come from timing both on MI355X at the Qwen3-8B shapes: the
# kernel wins on QKV, o_proj and down (1.2-2.8x at 64-256 rows); hipBLASLt keeps the
# lm_head and prefill-sized products, and gate_up goes to the fused gate_up + SiLU entry
# (``linear_silu_mul``).
DECODE_MAX_ROWS = 256
DECODE_MAX_N = 8192
DECODE_LONG_K_MIN_ROWS = 32


def uses_decode_kernel(rows: int, n: int, k: int) -> bool:
    """Whether ``linear`` routes an ``[rows, k] x [n, k]^T`` product to the gfx950 kernel."""
    return (0 < rows <= DECODE_MAX_ROWS and n <= DECODE_MAX_N and n % 4 == 0 and k % 64 == 0
            and (k <= 4096 or rows >= DECODE_LONG_K_MIN_ROWS))


def decode_linear(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None,
                  config: int = -1, splits: int = -1) -> torch.Tensor:
    """``x @ weight.T`` on the gfx950 projection kernel (fp32 accumulation, one rounding).

    x ``[M, K]`` with unit column stride, weight ``[N, K]`` contiguous, same 16-bit
    dtype. When the kernel splits K, its fp32 partials live in a workspace taken from
    the caching allocator (safe under HIP graph capture). ``config``/``splits`` force a
    tiling (tuning and tests); -1 lets the library choose. Replaces the decode-time
    ``x.matmul(w.T)`` of ``src/layers/linear.rs:5-7``."""
    _require_device(x, "decode_linear")
    dt = dtype_code(x)
    if (x.dim() != 2 or weight.dim() != 2 or x.stride(1) != 1 or not weight.is_contiguous()
            or weight.dtype != x.dtype or weight.device != x.device
            or weight.size(1) != x.size(1)):
        raise NativeError("invalid linear operands: expected x [M, K] and weight [N, K]")
    m, k = x.shape
    n = weight.size(0)
    if out is None:
        out = torch.empty((m, n), dtype=x.dtype, device=x.device)
    elif (out.shape != (m, n) or out.dtype != x.dtype or out.stride(1) != 1
          or out.device != x.device):
        raise NativeError("invalid linear output")
    cus = _native.device_cus(x.device)
    need = lib().mi355x_linear_workspace_bytes(m, n, k, cus, config, splits)
    if need < 0:
        raise NativeError("invalid linear shape")
    ws = torch.empty(max(int(need), 16), dtype=torch.uint8, device=x.device) if need else None
    check(lib().mi355x_linear(x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0),
                              out.data_ptr(), out.stride(0), m, n, k,
                              None if ws is None else ws.data_ptr(), int(need), cus, config,
                              splits, dt, stream_of(x)), "decode_linear")
    return out


def linear_add_rms_norm(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                        norm_weight: torch.Tensor,
                        eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """``y = linear(x, weight)`` then ``add_rms_norm(y, residual, norm_weight, eps)``,
    returning ``(normed, residual)`` with ``residual`` updated in place. Decode-sized
    products run as one projection plus one fused reduce/residual/norm pass (bit-identical
    to the two separate steps); everything else runs the two steps."""
    m, k = (x.shape if x.dim() == 2 else (0, 0))
    n = weight.size(0)
    if (x.is_cuda and x.dim() == 2 and x.stride(1) == 1 and weight.is_contiguous()
            and uses_decode_kernel(m, n, k) and n % 8 == 0 and 128 < n // 8 <= 1024
            and x.stride(0) % 8 == 0 and residual.dim() == 2 and residual.shape == (m, n)
            and residual.stride(1) == 1 and residual.dtype == x.dtype
            and residual.device == x.device and residual.stride(0) % 8 == 0):
        _require_device(x, "linear_add_rms_norm")
        dt = dtype_code(x)
        _check_weight(x, norm_weight, n)
        if weight.dtype != x.dtype or weight.device != x.device or weight.size(1) != k:
            raise NativeError("invalid linear operands: expected x [M, K] and weight [N, K]")
        out = torch.empty((m, n), dtype=x.dtype, device=x.device)
        cus = _native.device_cus(x.device)
        need = lib().mi355x_linear_workspace_bytes(m, n, k, cus, -1, -1)
        ws = torch.empty(max(int(need), 16), dtype=torch.uint8, device=x.device) if need else None
        check(lib().mi355x_linear_add_rms_norm(
            x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), residual.data_ptr(),
            residual.stride(0), norm_weight.data_ptr(), float(eps), out.data_ptr(), n, m, n, k,
            None if ws is None else ws.data_ptr(), int(need), cus, dt, stream_of(x)),
            "linear_add_rms_norm")
        return out, residual
    return add_rms_norm(linear(x, weight), residual, norm_weight, eps)


def uses_silu_kernel(rows: int, width: int, k: int) -> bool:
    """Whether ``linear_silu_mul`` runs the fused gate_up + SiLU kernel for
    ``[rows, k] x [2 width, k]^T``."""
    return 0 < rows <= DECODE_MAX_ROWS and width % 4 == 0 and k % 64 == 0


def decode_linear_silu_mul(x: torch.Tensor, weight: torch.Tensor,
                           out: torch.Tensor | None = None, config: int = -1) -> torch.Tensor:
    """``silu_and_mul(x @ weight.T)`` in one gfx950 launch: weight ``[2 W, K]`` (gate rows,
    then up rows), result ``[M, W]``, bit-identical to ``decode_linear`` (unsplit) followed
    by ``silu_and_mul``."""
    _require_device(x, "decode_linear_silu_mul")
    dt = dtype_code(x)
    if (x.dim() != 2 or weight.dim() != 2 or x.stride(1) != 1 or not weight.is_contiguous()
            or weight.dtype != x.dtype or weight.device != x.device
            or weight.size(1) != x.size(1) or weight.size(0) % 2 != 0):
        raise NativeError("invalid gate_up operands: expected x [M, K] and weight [2W, K]")
    m, k = x.shape
    width = weight.size(0) // 2
    if out is None:
        out = torch.empty((m, width), dtype=x.dtype, device=x.device)
    elif (out.shape != (m, width) or out.dtype != x.dtype or out.stride(1) != 1
          or out.device != x.device):
        raise NativeError("invalid gate_up output")
    check(lib().mi355x_linear_silu_mul(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                       weight.stride(0), out.data_ptr(), out.stride(0), m,
                                       width, k, _native.device_cus(x.device), config, dt,
                                       stream_of(x)), "decode_linear_silu_mul")
    return out


def linear_silu_mul(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """The MLP's ``silu_and_mul(linear(x, gate_up))`` (``mlp.rs``, ``ops.rs:53-61``):
    decode-sized products in one fused launch, the rest as the two steps."""
    if (x.is_cuda and x.dim() == 2 and x.stride(1) == 1 and weight.is_contiguous()
            and weight.size(0) % 2 == 0
            and uses_silu_kernel(x.size(0), weight.size(0) // 2, x.size(1))):
        return decode_linear_silu_mul(x, weight)
    return silu_and_mul(linear(x, weight))


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``x @ weight.T``: decode-sized products on the gfx950 kernel, the rest on
    hipBLASLt (``src/layers/linear.rs:5-7``)."""
    if (x.is_cuda and x.dim() == 2 and x.stride(1) == 1 and weight.is_contiguous()
            and uses_decode_kernel(x.size(0), weight.size(0), x.size(1))):
        return decode_linear(x, weight)
    return torch.nn.functional.linear(x, weight)


__all__ = ["rms_norm", "add_rms_norm", "qk_norm", "silu_and_mul", "linear_silu_mul",
           "HalfSplitRope", "rope", "qk_norm_rope_store", "decode_linear", "linear",
           "linear_add_rms_norm", "decode_linear_silu_mul",
           "uses_decode_kernel", "NativeError",
           "_native"]
