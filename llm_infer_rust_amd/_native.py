"""ctypes binding of libmi355x_attn.so (the C ABI declared in include/mi355x_attn.h).

The library is the only compute path: if it is missing or fails to load,
every op raises. There is no CPU or PyTorch fallback.

``torch`` is imported before the library is opened so that the library binds to
the HIP runtime torch already loaded (same soname), giving one runtime per
process.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede loading the HIP library)

# MI355X_ATTN_LIB overrides the library path (for comparing builds of the same sources).
LIB_PATH = Path(os.environ.get("MI355X_ATTN_LIB",
                               Path(__file__).resolve().parent / "libmi355x_attn.so"))

c_void_p = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_i32 = ctypes.c_int32
c_int = ctypes.c_int
c_bool = ctypes.c_bool
c_double = ctypes.c_double
c_char_p = ctypes.c_char_p
c_u64 = ctypes.c_uint64
P_i32 = ctypes.POINTER(ctypes.c_int32)
P_i64 = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes). Keep in the order of include/mi355x_attn.h.
SIGNATURES: dict[str, tuple] = {
    "mi355x_attn_error": (c_char_p, []),
    "mi355x_attn_abi_version": (c_int, []),
    "mi355x_store_kv": (c_char_p, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                   c_bool, c_void_p, c_void_p]),
    "mi355x_rms_norm": (c_char_p, [c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64, c_i64,
                                   c_i64, c_double, c_int, c_void_p]),
    "mi355x_add_rms_norm": (c_char_p, [c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64,
                                       c_i64, c_double, c_int, c_void_p]),
    "mi355x_qk_norm": (c_char_p, [c_void_p, c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64,
                                  c_i64, c_i64, c_i64, c_i64, c_i64, c_double, c_int, c_void_p]),
    "mi355x_decode_prepare": (c_void_p, [c_void_p, c_void_p, c_i64, c_i64, c_i64, c_void_p,
                                         c_i64, c_i64, c_i64, c_i64, c_i64, c_bool, c_void_p,
                                         c_i64, c_void_p]),
    "mi355x_decode_run": (c_char_p, [c_void_p, c_void_p, c_i64, c_i64, c_void_p, c_void_p,
                                     c_void_p, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                     c_void_p]),
    "mi355x_decode_plan_drop": (None, [c_void_p]),
    "mi355x_decode_workspace_allocations": (c_u64, [c_void_p]),
    "mi355x_decode_plan_info": (c_char_p, [c_void_p, P_i64]),
    "mi355x_decode_plan_read": (c_char_p, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                           c_void_p, c_void_p]),
    "mi355x_decode_schedule": (c_i64, [c_void_p, c_i64, c_i64, c_i64, c_void_p, c_i64, c_void_p,
                                       P_i64]),
    "mi355x_decode_items_capacity": (c_i64, [c_i64, c_i64, c_i64]),
    "mi355x_prefill_prepare": (c_void_p, [c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64,
                                          c_void_p, c_void_p, c_i64, c_i64, c_i64, c_i64,
                                          c_void_p]),
    "mi355x_prefill_run": (c_char_p, [c_void_p, c_void_p, c_i64, c_i64, c_void_p, c_i64, c_i64,
                                      c_void_p, c_i64, c_i64, c_void_p, c_i64, c_i64, c_i64,
                                      c_i64, c_i64, c_i64, c_i64, c_void_p]),
    "mi355x_prefill_plan_drop": (None, [c_void_p]),
    "mi355x_prefill_workspace_allocations": (c_u64, [c_void_p]),
    "mi355x_prefill_plan_info": (c_char_p, [c_void_p, P_i64]),
    "mi355x_prefill_plan_read": (c_char_p, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "mi355x_prefill_schedule": (c_i64, [c_void_p, c_void_p, c_i64, c_i64, c_i64, c_void_p,
                                        c_i64]),
    "mi355x_rope": (c_char_p, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_i64, c_i64,
                               c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_int, c_void_p]),
    "mi355x_qk_norm_rope_store": (c_char_p, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                             c_void_p, c_void_p, c_void_p, c_i64, c_void_p,
                                             c_void_p, c_void_p, c_bool, c_i64, c_i64, c_void_p,
                                             c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                             c_i64, c_i64, c_i64, c_double, c_int, c_void_p]),
    "mi355x_linear_qk_norm_rope_store": (c_char_p, [c_void_p, c_i64, c_void_p, c_i64,
                                                    c_void_p, c_i64, c_i64, c_i64, c_i64, c_i64,
                                                    c_void_p, c_i64, c_i32, c_void_p, c_void_p,
                                                    c_void_p, c_void_p, c_void_p, c_i64,
                                                    c_void_p, c_void_p, c_void_p, c_bool, c_i64,
                                                    c_i64, c_void_p, c_double, c_int,
                                                    c_void_p]),
    "mi355x_silu_mul": (c_char_p, [c_void_p, c_void_p, c_i64, c_i64, c_int, c_void_p]),
    "mi355x_linear": (c_char_p, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_i64,
                                 c_i64, c_i64, c_void_p, c_i64, c_i32, c_i32, c_i32, c_i64,
                                 c_void_p]),
    "mi355x_linear_add_rms_norm": (c_char_p, [c_void_p, c_i64, c_void_p, c_i64, c_void_p,
                                              c_i64, c_void_p, c_double, c_void_p, c_i64,
                                              c_i64, c_i64, c_i64, c_void_p, c_i64, c_i32,
                                              c_i64, c_void_p]),
    "mi355x_linear_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i32, c_i32, c_i32]),
    "mi355x_linear_noalloc": (c_char_p, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64,
                                         c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i64,
                                         c_void_p]),
    "mi355x_linear_silu_mul": (c_char_p, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64,
                                          c_i64, c_i64, c_i64, c_i32, c_i32, c_i64,
                                          c_void_p]),
    "mi355x_sample": (c_char_p, [c_void_p, c_i64, c_i64, c_i64, c_int, c_void_p, c_void_p,
                                 c_void_p, c_u64, c_u64, c_void_p, c_void_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeError(RuntimeError):
    """Raised when a native entry point reports an error."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeError(
                    f"{LIB_PATH.name} is not built; run `python -m llm_infer_rust_amd.build` "
                    "(the HIP library is the only compute path)")
            handle = ctypes.CDLL(os.fspath(LIB_PATH), mode=ctypes.RTLD_LOCAL)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def check(err: bytes | None, what: str) -> None:
    if err is not None:
        raise NativeError(f"{what} failed: {err.decode(errors='replace')}")


def last_error() -> str:
    return lib().mi355x_attn_error().decode(errors="replace")


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current stream on the tensor's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return 0
    if t.dtype == torch.float16:
        return 1
    raise NativeError(f"expected bfloat16 or float16 tensor, got {t.dtype}")


_CUS: dict[int, int] = {}


def device_cus(device: torch.device) -> int:
    """Compute units of a GPU (cached per device index)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _CUS:
        _CUS[index] = torch.cuda.get_device_properties(index).multi_processor_count
    return _CUS[index]


# ---------------------------------------------------------------------------
# Releasing native plans. Dropping a plan frees device buffers and waits on its upload event
# (hipFree, hipEventSynchronize), which a stream capture in progress does not allow: a plan
# finalized by the garbage collector in the middle of a HIP graph capture would invalidate the
# capture. Such a plan's handle is parked and released at the next safe point instead (the
# next plan release or creation outside a capture, or an explicit release_deferred()).
# ---------------------------------------------------------------------------
_deferred: list[tuple[str, int]] = []
_deferred_lock = threading.Lock()


def _capturing() -> bool:
    """True while this thread's current HIP stream is being captured into a graph."""
    try:
        return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
    except Exception:  # interpreter shutdown
        return False


def release_deferred() -> None:
    """Release the plan handles parked during a capture (no-op while one is in progress)."""
    if _capturing():
        return
    while True:
        with _deferred_lock:
            if not _deferred:
                return
            name, handle = _deferred.pop()
        getattr(lib(), name)(handle)


def release_handle(drop_entry: str, handle: int) -> None:
    """Drop a native plan through `drop_entry` now, or after the capture in progress."""
    if _capturing():
        with _deferred_lock:
            _deferred.append((drop_entry, handle))
        return
    release_deferred()
    getattr(lib(), drop_entry)(handle)


def deferred_count() -> int:
    with _deferred_lock:
        return len(_deferred)
