"""Tensors derived once from a caller's parameters (transposed router weights, weights
converted from another layout), cached per source tensor and version.

An entry lives as long as the source's base tensor (a weak identity-keyed map), so
freed storage whose address is reused by a new tensor can never hit an old entry.
Each entry records the signature of every input it was made from (base identity,
view geometry, dtype, version counter) and holds those bases, so the identities it
compares stay valid while it exists; an in-place update bumps the version and makes
the entry stale.  Inference tensors have no version counter: they are never cached, and
nothing made while a HIP graph is being captured on the current stream is kept.
"""

from __future__ import annotations

from typing import Callable, Optional, Sequence

import torch
from torch import Tensor
from torch.utils.weak import WeakIdKeyDictionary

_ENTRIES: "WeakIdKeyDictionary" = WeakIdKeyDictionary()


def _base(t: Tensor) -> Tensor:
    return t._base if t._base is not None else t


def _signature(t: Optional[Tensor]):
    if t is None:
        return None
    return (id(_base(t)), t.storage_offset(), tuple(t.shape), tuple(t.stride()), t.dtype,
            t.device, t._version)


def _capturing(inputs: Sequence[Optional[Tensor]]) -> bool:
    """A HIP graph is being captured on the current stream: what make() allocates then
    belongs to the graph's private pool, so it is used by the call and not kept (an
    entry made before the capture is still used)."""
    t = next((t for t in inputs if t is not None), None)
    return t is not None and t.is_cuda and torch.cuda.is_current_stream_capturing()


def derived(tag: str, inputs: Sequence[Optional[Tensor]], make: Callable[[], object]):
    """``make()`` computed from ``inputs`` (the first one is the key), cached until any
    input is freed, replaced by another tensor or modified in place."""
    key = inputs[0]
    if any(t is not None and t.is_inference() for t in inputs):
        with torch.no_grad():
            return make()
    sig = (tag,) + tuple(_signature(t) for t in inputs)
    slot = _ENTRIES.get(_base(key))
    hit = None if slot is None else slot.get(tag)
    if hit is not None and hit[0] == sig:
        return hit[2]
    with torch.no_grad():
        value = make()
    if _capturing(inputs):  # the value lives in the graph's pool: used, not kept
        return value
    if slot is None:
        slot = {}
        _ENTRIES[_base(key)] = slot
    slot[tag] = (sig, [None if t is None else _base(t) for t in inputs], value)
    return value


def clear() -> None:
    _ENTRIES.clear()


def transposed_rows(router_weights: Tensor) -> Tensor:
    """router_weights [H, E] -> contiguous [E, H] rows (a view when the storage already
    is [E, H], as for ``W.T`` of a contiguous [E, H] parameter)."""
    w = router_weights.t()
    if w.is_contiguous():
        return w
    return derived("router_rows", (router_weights,), lambda: w.contiguous())
