"""Slot-pooled recurrent state of the GDN layers: the layout contract the kernels
read.

Mirrors ``RecurrentCache`` and the GDN half of ``Cache`` (braid/model/cache.py:
97-232). Attention's KV pool is not part of this path and is not rebuilt.

Layout (what ``include/braid_gdn.h`` takes):

* ``state`` ``[max_slots, n_heads, state_size, head_dim]``, fp32 / fp16 / bf16,
  head_dim fastest (cache.py:127-128). One (slot, head) tile is one contiguous
  ``state_size x head_dim`` block; a kernel addresses it as
  ``(slot * n_heads + h) * state_size * head_dim``.
* ``conv`` ``[max_slots, conv_channels, conv_kernel]`` fp32, the last K
  **pre-convolution** inputs per channel, oldest first (cache.py:100-104 and
  braid/kernels/csrc/conv1d_decode.cu:21-27). The reference kept this pool in
  the activation dtype for its torch path; both conv kernels here take fp32,
  as the reference's CUDA conv did, so fp32 is the only accepted dtype.
* The batch addresses the pools through ``slots_i32`` (int32, on the device):
  the kernels gather by slot, so one captured graph serves every assignment.

Nothing here computes on the CPU: the pools live wherever ``device`` says,
and the kernels that read them run only on the GPU.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from braid_amd.config import GDNConfig

STATE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


class RecurrentCache:
    """One GDN layer's conv window and delta-rule state, pooled by slot
    (braid/model/cache.py:97-138)."""

    def __init__(self, g: GDNConfig, max_slots: int, device: str | torch.device,
                 state_dtype: torch.dtype = torch.float32,
                 conv_dtype: torch.dtype = torch.float32):
        if state_dtype not in STATE_DTYPES:
            raise ValueError(f"state_dtype {state_dtype} is not one of fp32 / fp16 / bf16")
        if conv_dtype != torch.float32:
            raise ValueError("the conv kernels take an fp32 conv pool, "
                             f"got conv_dtype {conv_dtype}")
        if max_slots <= 0:
            raise ValueError(f"max_slots must be positive, got {max_slots}")
        self.conv = torch.zeros(max_slots, g.conv_channels, g.conv_kernel, device=device,
                                dtype=conv_dtype)
        self.state = torch.zeros(max_slots, g.n_heads, g.state_size, g.head_dim,
                                 device=device, dtype=state_dtype)

    def reset(self, slot: int) -> None:
        """Zero one slot, so a new sequence never starts from the previous
        occupant's state (cache.py:132-137)."""
        self.conv[slot].zero_()
        self.state[slot].zero_()


@dataclass
class GDNCache:
    """Every GDN layer's pools plus the batch's slot assignment and per-slot
    lengths (braid/model/cache.py:140-232, GDN layers only).

    ``slots`` (int64) and ``slots_i32`` hold the same assignment; the int32 copy
    is what the kernels take, kept alongside because a cast allocates and an
    allocation inside graph capture is a capture failure (cache.py:150-153).
    """

    layers: list
    slots: torch.Tensor
    lengths: torch.Tensor
    max_slots: int
    slots_i32: Optional[torch.Tensor] = None

    def __post_init__(self) -> None:
        if self.slots_i32 is None:
            self.slots_i32 = self.slots.to(torch.int32)

    @classmethod
    def allocate(cls, g: GDNConfig, max_slots: int, device: str | torch.device,
                 state_dtype: torch.dtype = torch.float32,
                 n_layers: Optional[int] = None) -> "GDNCache":
        n = g.n_gdn_layers if n_layers is None else n_layers
        return cls(layers=[RecurrentCache(g, max_slots, device, state_dtype) for _ in range(n)],
                   slots=torch.arange(max_slots, device=device),
                   lengths=torch.zeros(max_slots, dtype=torch.int64, device=device),
                   max_slots=max_slots)

    def reset_slot(self, slot: int) -> None:
        for lyr in self.layers:
            lyr.reset(slot)
        self.lengths[slot] = 0

    def select(self, slots: Sequence[int] | torch.Tensor) -> "GDNCache":
        """A view addressing ``slots`` as batch rows 0..B-1; every pool is
        shared, only the assignment changes (cache.py:182-194)."""
        idx = (slots if isinstance(slots, torch.Tensor)
               else torch.tensor(list(slots), dtype=torch.int64, device=self.slots.device))
        idx = idx.to(self.slots.device)
        return GDNCache(layers=self.layers, slots=idx, lengths=self.lengths,
                        max_slots=self.max_slots, slots_i32=idx.to(torch.int32))

    def snapshot(self) -> list:
        """Copy every mutable pool and the lengths (cache.py:196-208)."""
        out = [self.lengths.clone()]
        for lyr in self.layers:
            out += [lyr.conv.clone(), lyr.state.clone()]
        return out

    def restore(self, snap: list) -> None:
        it = iter(snap)
        self.lengths.copy_(next(it))
        for lyr in self.layers:
            lyr.conv.copy_(next(it))
            lyr.state.copy_(next(it))

    def snapshot_slots(self, slots: torch.Tensor) -> tuple:
        """Copy only the rows of ``slots`` (and their lengths). A decode step
        touches nothing else, so this is what graph capture needs to undo its
        warm-up steps: 2 MiB per slot and layer at fp16 instead of the whole
        pool."""
        idx = slots.to(self.slots.device, torch.int64)
        rows = [(lyr.conv.index_select(0, idx), lyr.state.index_select(0, idx))
                for lyr in self.layers]
        return idx.clone(), self.lengths.index_select(0, idx), rows

    def restore_slots(self, snap: tuple) -> None:
        idx, lengths, rows = snap
        self.lengths.index_copy_(0, idx, lengths)
        for lyr, (conv, state) in zip(self.layers, rows):
            lyr.conv.index_copy_(0, idx, conv)
            lyr.state.index_copy_(0, idx, state)

    @property
    def batch_lengths(self) -> torch.Tensor:
        """Committed token count of each row of the current assignment."""
        return self.lengths.index_select(0, self.slots)

    def bytes(self) -> int:
        return sum(lyr.conv.numel() * lyr.conv.element_size()
                   + lyr.state.numel() * lyr.state.element_size() for lyr in self.layers)
