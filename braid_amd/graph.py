"""Graph capture of the decode step per batch bucket, with scratch-slot padding.

Mirrors ``GraphedDecoder`` (braid/model/graph.py:51-192) for the GDN path:
one graph per batch bucket, captured against static input buffers and a
static slot buffer that the caller's values are copied into before replay.
The kernels read ``slot_idx`` from device memory, so reassigning sequences to
slots is a copy into that buffer, never a re-capture. On ROCm,
``torch.cuda.CUDAGraph`` is a hipGraph: a replay launches the whole step's
kernels with one host call.

A batch of B rows replays the smallest bucket >= B; rows B..bucket-1 are
padding. Padded rows run the full arithmetic on the slots they name, so they
must name scratch slots that no live sequence owns (``pad_slots``), or they
corrupt a live sequence's state (graph.py:15-19). Their inputs are zeroed;
with a zero gate ``z`` the readout of a padded row is exactly 0, so it does
not move the per-tensor FP8 scale of the live rows either.

Under capture the kernels skip their eager slot-map validation (a device to
host copy is illegal while capturing), which is also what lets several padded
rows share one scratch slot. A replay therefore trusts the slot buffer, and
``step`` validates what it copies in (``validate=True``, the default): every
slot in ``[0, max_slots)``, live slots distinct, and no pad slot equal to a
live one. An out-of-range slot would make the kernels write outside the pool,
and a repeated live slot would let two rows race on one state slab; the eager
entry points reject both, and so does ``step``. The check reads the slots on
the host (one small device-to-host copy when they live on the GPU, the same
synchronisation an eager launch pays); ``validate=False`` skips it for
callers that guarantee the contract themselves.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable, Optional, Sequence

import torch

from braid_amd.cache import GDNCache

# The reference's ladder (graph.py:48): buckets above the pool size are never
# captured.
DEFAULT_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 96, 128)


def usable_buckets(buckets: Sequence[int], max_slots: int) -> tuple:
    usable = tuple(b for b in sorted(set(buckets)) if 0 < b <= max_slots)
    if not usable:
        raise ValueError(f"no bucket fits: buckets={tuple(buckets)}, cache has {max_slots} slots")
    return usable


def bucket_for(sizes: Sequence[int], batch: int) -> int:
    """Smallest bucket holding ``batch`` rows (graph.py:143-148)."""
    for b in sizes:
        if b >= batch:
            return b
    raise ValueError(f"batch {batch} exceeds the largest bucket {max(sizes)}")


def _map(fn: Callable, obj: Any) -> Any:
    if isinstance(obj, torch.Tensor):
        return fn(obj)
    if isinstance(obj, dict):
        return {k: _map(fn, v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return type(obj)(_map(fn, v) for v in obj)
    return obj


def _zip_copy(dst: Any, src: Any, rows: int, pad: bool) -> None:
    """Copy src's leading ``rows`` rows into dst's; with ``pad``, zero the
    rest of dst."""
    if isinstance(dst, torch.Tensor):
        if src.shape[0] != rows or src.shape[1:] != dst.shape[1:]:
            raise ValueError(f"input of shape {tuple(src.shape)} does not fit the static "
                             f"buffer {tuple(dst.shape)} at {rows} rows")
        dst[:rows].copy_(src)
        if pad:
            dst[rows:].zero_()
        return
    if isinstance(dst, dict):
        if set(dst) != set(src):
            raise ValueError(f"inputs {sorted(src)} do not match the captured {sorted(dst)}")
        for k in dst:
            _zip_copy(dst[k], src[k], rows, pad)
        return
    if len(dst) != len(src):
        raise ValueError("input lists do not match the captured inputs")
    for d, s in zip(dst, src):
        _zip_copy(d, s, rows, pad)


@dataclass
class _Bucket:
    graph: torch.cuda.CUDAGraph
    inputs: Any               # static inputs, leading dim = size
    slots: torch.Tensor       # [size] int64, static
    slots_i32: torch.Tensor   # [size] int32, static, same values
    outputs: Any              # static outputs
    size: int


class GraphedDecoder:
    """Captures ``step(inputs, view)`` once per bucket and replays it.

    ``make_inputs(size)`` returns the static input buffers for one bucket (a
    tensor, or dicts / lists of them, each with leading dimension ``size``).
    ``step`` must read its rows' slots from ``view.slots_i32`` and allocate
    only through torch (the capture gives it a private memory pool).
    """

    def __init__(self, step: Callable, cache: GDNCache, make_inputs: Callable,
                 buckets: Sequence[int] = DEFAULT_BUCKETS, warmup: int = 3):
        self.step_fn = step
        self.cache = cache
        self.warmup = warmup
        self.sizes = usable_buckets(buckets, cache.max_slots)
        self.buckets = {b: self._capture(b, make_inputs(b)) for b in self.sizes}

    def _capture(self, size: int, inputs: Any) -> _Bucket:
        cache = self.cache
        dev = cache.slots.device
        slots = torch.arange(size, dtype=torch.long, device=dev)
        slots_i32 = slots.to(torch.int32)
        view = GDNCache(layers=cache.layers, slots=slots, lengths=cache.lengths,
                        max_slots=cache.max_slots, slots_i32=slots_i32)
        # Warm-up steps are real steps on slots 0..size-1; their rows are saved
        # and put back, so capture leaves no mark on the pool (graph.py:103-116).
        saved = cache.snapshot_slots(slots)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(self.warmup):
                self.step_fn(inputs, view)
        torch.cuda.current_stream().wait_stream(side)
        cache.restore_slots(saved)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outputs = self.step_fn(inputs, view)
        cache.restore_slots(saved)
        return _Bucket(graph=graph, inputs=inputs, slots=slots, slots_i32=slots_i32,
                       outputs=outputs, size=size)

    def check_slots(self, slots: torch.Tensor, pad_slots: Optional[torch.Tensor],
                    n_pad: int) -> None:
        """Raise ValueError unless every live slot lies in ``[0, max_slots)``
        and is distinct, and the ``n_pad`` pad slots used lie in range and
        name no live slot. The messages follow the eager entry points'."""
        n = self.cache.max_slots
        live = [int(s) for s in slots.reshape(-1).tolist()]
        pads = [] if n_pad == 0 else [int(s) for s in pad_slots.reshape(-1)[:n_pad].tolist()]
        if len(pads) < n_pad:
            raise ValueError(f"pad_slots holds {len(pads)} slots; {n_pad} rows are padding")
        for i, s in enumerate(live):
            if not 0 <= s < n:
                raise ValueError(f"slot_idx[{i}] = {s} is out of range [0, {n})")
        if len(set(live)) != len(live):
            dup = next(s for s in live if live.count(s) > 1)
            raise ValueError(f"slot_idx has duplicate slot {dup}; two live rows sharing one "
                             f"state slab is silent cross-sequence corruption. Slots must be "
                             f"distinct.")
        for i, s in enumerate(pads):
            if not 0 <= s < n:
                raise ValueError(f"pad_slots[{i}] = {s} is out of range [0, {n})")
        clash = set(pads) & set(live)
        if clash:
            raise ValueError(f"pad slot {min(clash)} is also a live slot; padded rows would "
                             f"advance that sequence's state")

    def step(self, inputs: Any, slots: torch.Tensor,
             pad_slots: Optional[torch.Tensor] = None, validate: bool = True) -> Any:
        """Copy ``inputs`` (leading dim B) and ``slots`` [B] into the bucket's
        static buffers, point the padded rows at ``pad_slots``, replay, and
        return the outputs cut to B rows (graph.py:150-192). With
        ``validate`` the slots are checked first (``check_slots``)."""
        B = int(slots.shape[0])
        size = bucket_for(self.sizes, B)
        buck = self.buckets[size]
        if B < size and pad_slots is None:
            raise ValueError(f"batch {B} pads bucket {size}; pass pad_slots for the "
                             f"{size - B} scratch rows, or the padding will advance live slots")
        if validate:
            self.check_slots(slots, pad_slots, size - B)
        _zip_copy(buck.inputs, inputs, B, pad=B < size)
        buck.slots[:B].copy_(slots)
        if B < size:
            buck.slots[B:].copy_(pad_slots[: size - B])
        buck.slots_i32.copy_(buck.slots)
        buck.graph.replay()
        return _map(lambda t: t[:B] if t.dim() > 0 and t.shape[0] == size else t, buck.outputs)
