"""Token sampling on the gfx950 sampling kernel.

Mirrors ``src/engine/sampling.rs``:

* ``SamplingParams`` with ``normalized()`` (``:8-47``);
* ``Sampler.sample_batch(logits, params)`` -> list of ids, raising
  ``SamplingError`` for an invalid distribution (``:281-372``, ``sampled_ids``);
* ``Sampler.defer_batch(logits, params)`` -> ``PendingSample`` whose ids are
  copied into pinned host memory behind an event (the reference's ``Readback``,
  ``:193-237``); ``relay()`` gives the device ids clamped at 0 for the next
  step's embedding, ``finish()`` waits and validates.

Unlike the reference, which groups rows by identical parameters and launches
one FlashInfer call per group (``:343-371``), one kernel launch serves the
whole heterogeneous batch: the parameters travel as per-row device arrays.
The random stream is (seed, offset): ``manual_seed`` resets both and every
sampling launch advances the offset by one.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace

import torch

from ._native import NativeError, check, lib, stream_of


class SamplingError(RuntimeError):
    """Invalid logits shape, parameter count mismatch or invalid distribution."""


@dataclass(frozen=True)
class SamplingParams:
    temperature: float = 0.0
    top_k: int = -1
    top_p: float = 1.0
    ignore_eos: bool = False
    max_tokens: int = 1024

    def normalized(self) -> "SamplingParams":
        top_p = self.top_p if (math.isfinite(self.top_p) and 0.0 <= self.top_p <= 1.0) else 1.0
        return replace(self, max_tokens=max(self.max_tokens, 1), top_p=top_p)


_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _validate_logits(logits: torch.Tensor) -> None:
    if logits.dim() != 2 or logits.size(1) <= 0:
        raise SamplingError(f"logits must be 2-D (num_reqs, vocab_size), got {list(logits.shape)}")
    if not logits.is_cuda:
        raise NativeError("sampling requires GPU logits")
    if logits.dtype not in _DTYPES:
        raise NativeError(f"unsupported logits dtype {logits.dtype}")
    if logits.stride(1) != 1:
        raise NativeError("logits rows must be contiguous")


class PendingSample:
    """One in-flight sampling launch; ids land in pinned host memory behind an event."""

    def __init__(self, ids: torch.Tensor, logits: torch.Tensor):
        self.ids = ids
        self._logits = logits  # keeps the input alive until the copy has run
        self._host = torch.empty(ids.shape, dtype=ids.dtype, pin_memory=True)
        self._host.copy_(ids, non_blocking=True)
        self._event = torch.cuda.Event()
        self._event.record(torch.cuda.current_stream(ids.device))

    def relay(self) -> torch.Tensor:
        """Device ids with the -1 sentinel clamped to 0, safe to feed an embedding."""
        return self.ids.clamp_min(0)

    def ready(self) -> bool:
        return self._event.query()

    def finish(self) -> list[int]:
        self._event.synchronize()
        ids = self._host.tolist()
        if any(i < 0 for i in ids):
            raise SamplingError("invalid probability distribution")
        return ids


class Sampler:
    """Samples one next-token id per logits row, whole batch in one launch."""

    def __init__(self, seed: int = 0):
        self.manual_seed(seed)
        self._param_key: tuple | None = None
        self._param_objs: tuple | None = None
        self._params: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None

    def manual_seed(self, seed: int) -> None:
        self.seed = int(seed) & (2 ** 64 - 1)
        self.offset = 0

    def _device_params(self, params_list, device: torch.device):
        # A decode step usually passes the very objects of the previous step (each running
        # request keeps its SamplingParams, which are frozen): reuse the device arrays after
        # an identity check instead of normalising every row again on the host.
        objs = self._param_objs
        if (objs is not None and self._param_key is not None and self._param_key[0] == device
                and len(objs) == len(params_list)
                and all(a is b for a, b in zip(params_list, objs))):
            return self._params
        normalized = [p.normalized() for p in params_list]
        key = (device, tuple((p.temperature, p.top_k, p.top_p) for p in normalized))
        self._param_objs = tuple(params_list)
        if key != self._param_key:
            n = len(normalized)
            host = torch.empty(3 * n, dtype=torch.float32, pin_memory=True)
            host[:n] = torch.tensor([p.temperature for p in normalized], dtype=torch.float32)
            host[2 * n:] = torch.tensor([p.top_p for p in normalized], dtype=torch.float32)
            ks = torch.tensor([p.top_k for p in normalized], dtype=torch.int32)
            host[n:2 * n] = ks.view(torch.float32)  # bit-copy the int32 top-k
            dev = host.to(device, non_blocking=True)
            self._params = (dev[:n], dev[n:2 * n].view(torch.int32), dev[2 * n:])
            self._param_key = key
        return self._params

    def sample_batch_device(self, logits: torch.Tensor, params_list, *,
                            out: torch.Tensor | None = None) -> torch.Tensor:
        """Device int64 ids [rows]; an invalid distribution yields -1 in its row."""
        _validate_logits(logits)
        rows = logits.size(0)
        if rows != len(params_list):
            raise SamplingError(
                f"SamplingParams count ({len(params_list)}) must equal logits rows ({rows})")
        if out is None:
            out = torch.empty(rows, dtype=torch.int64, device=logits.device)
        if rows == 0:
            return out
        temperature, top_k, top_p = self._device_params(params_list, logits.device)
        check(lib().mi355x_sample(logits.data_ptr(), rows, logits.size(1), logits.stride(0),
                                  _DTYPES[logits.dtype], temperature.data_ptr(),
                                  top_k.data_ptr(), top_p.data_ptr(), self.seed, self.offset,
                                  out.data_ptr(), stream_of(logits)), "sample")
        self.offset += 1
        return out

    def sample_batch(self, logits: torch.Tensor, params_list) -> list[int]:
        return self.defer_batch(logits, params_list).finish()

    def defer_batch(self, logits: torch.Tensor, params_list) -> PendingSample:
        return PendingSample(self.sample_batch_device(logits, params_list), logits)


__all__ = ["SamplingParams", "Sampler", "PendingSample", "SamplingError"]
