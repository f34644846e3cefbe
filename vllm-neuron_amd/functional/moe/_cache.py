"""Tensors derived once from a caller's parameters (transposed router weights, weights
converted from another layout), cached per source tensor and version.

An entry lives only as long as the source's base tensor: the map is keyed weakly by that
base, and the entry refers to its other inputs' bases through weak references too, so a
cached value never keeps any of the tensors it was made from alive.  When the key's base
is freed, the entry and the value go with it.  Each entry records the signature of every
input it was made from (base identity, view geometry, dtype, version counter) together
with a weak reference to each base; a hit requires every reference to be alive and to
name the very base the caller passes, so freed storage whose address (or ``id``) is
reused by a new tensor can never hit an old entry, and an in-place update (a version
bump) makes the entry stale.  A value that is itself a view of the key's base would keep
the key alive, and is therefore returned without being cached.  Inference tensors have
no version counter: they are never cached, and nothing made while a HIP graph is being
captured on the current stream is kept.
"""

from __future__ import annotations

import weakref
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


def _tensors(value):
    """The tensors a cached value holds (a tensor, or a tuple / named tuple of them)."""
    if isinstance(value, Tensor):
        return [value]
    if isinstance(value, (tuple, list)):
        return [t for v in value for t in _tensors(v)]
    return []


def _refs_alive(refs, inputs) -> bool:
    """Every input's base is still the object the entry was made from."""
    for r, t in zip(refs, inputs):
        if (r is None) != (t is None):
            return False
        if r is not None and r() is not _base(t):
            return False
    return True


def derived(tag: str, inputs: Sequence[Optional[Tensor]], make: Callable[[], object]):
    """``make()`` computed from ``inputs`` (the first one is the key), cached until any
    input is freed, replaced by another tensor or modified in place."""
    key = inputs[0]
    if any(t is not None and t.is_inference() for t in inputs):
        with torch.no_grad():
            return make()
    kb = _base(key)
    sig = (tag,) + tuple(_signature(t) for t in inputs)
    slot = _ENTRIES.get(kb)
    hit = None if slot is None else slot.get(tag)
    if hit is not None and hit[0] == sig and _refs_alive(hit[1], inputs):
        return hit[2]
    with torch.no_grad():
        value = make()
    if _capturing(inputs):  # the value lives in the graph's pool: used, not kept
        return value
    if any(_base(t) is kb for t in _tensors(value)):  # a view of the key would pin it
        return value
    if slot is None:
        slot = {}
        _ENTRIES[kb] = slot
    refs = [None if t is None else weakref.ref(_base(t)) for t in inputs]
    slot[tag] = (sig, refs, value)
    return value


def discard(key: Tensor) -> None:
    """Drop every value cached for ``key``'s base (its content is about to change)."""
    _ENTRIES.pop(_base(key), None)


def entries() -> int:
    """Number of live source tensors with cached values."""
    return len(_ENTRIES)


def clear() -> None:
    _ENTRIES.clear()


def transposed_rows(router_weights: Tensor) -> Tensor:
    """router_weights [H, E] -> contiguous [E, H] rows (a view when the storage already
    is [E, H], as for ``W.T`` of a contiguous [E, H] parameter)."""
    w = router_weights.t()
    if w.is_contiguous():
        return w
    return derived("router_rows", (router_weights,), lambda: w.contiguous())
