"""One continuous-batching tick on a shared state pool: prefill chunks for new
sequences and one decode token for running ones, run side by side.

The reference's scheduler step (braid/serve/scheduler.py:246-274) runs a tick's
prefill chunks (one ragged forward over the rows still prefilling) and then its
decode (the rows that are not), one after the other on one stream. Here the
decode launch goes on a second stream forked from the caller's, so the two
kernels overlap: the prefill scan is a latency-bound serial chain (one
workgroup per CU at a tick's sizes), and the decode, a memory stream, fills the
CUs' remaining issue slots and the HBM beside it. On MI355X (config 4: 96
decode rows + 4 x 256 prefill tokens, fp16 pool, graph-replayed) the tick takes
129 us against 156 us in sequence; the prefill alone takes 119 us.

The prefill is captured first, and that order matters: the graph's branches
start in capture order, and a large decode asks for enough LDS to hold two of
its workgroups per CU, so a decode that started first would keep the prefill's
workgroups off the CUs until it drained (measured: 205 us for the tick with the
decode captured first).

The two launches touch disjoint slots (the decode takes only rows that are no
longer prefilling, scheduler.py:267), so their order does not change a bit:
outputs and pool equal the sequential tick's. That disjointness is the caller's
contract, as it is the scheduler's; an eager tick checks it when asked
(check_slots), a captured one cannot read the slot maps and does not. The fork
and join are stream waits, so a captured tick is two parallel graph branches.
An eager tick runs the two in sequence: each eager launch synchronises its
stream to validate its slots.
"""
from __future__ import annotations

from typing import Optional

import torch

from braid_amd.kernels.loader import load_gdn


class MixedTick:
    """``tick(pool, prefill, decode)`` with ``prefill`` the arguments of
    ``gdn_prefill_raw`` after the pool (slots, q, k, v, a_raw, b_raw, A,
    dt_bias, y, seq_lens, and optionally plan_lens: the host lengths a
    captured tick plans its ragged prefill from) and ``decode`` those of
    ``gdn_decode_raw`` (slots, q, k, v, a_raw, b_raw, A, dt_bias, y), as
    dicts with those names. The prefill runs on the caller's current stream,
    the decode on this object's side stream; the caller's stream waits for
    both before it goes on."""

    PREFILL = ("slots", "q", "k", "v", "a_raw", "b_raw", "A", "dt_bias", "y", "seq_lens")
    DECODE = ("slots", "q", "k", "v", "a_raw", "b_raw", "A", "dt_bias", "y")

    def __init__(self, kern=None, device: Optional[torch.device] = None,
                 check_slots: bool = False):
        self.kern = kern if kern is not None else load_gdn()
        self.side = torch.cuda.Stream(device=device)
        self.check_slots = check_slots

    @staticmethod
    def _check_disjoint(pre_slots: torch.Tensor, dec_slots: torch.Tensor) -> None:
        if pre_slots.is_cuda and torch.cuda.is_current_stream_capturing():
            return
        both = torch.cat([pre_slots.reshape(-1), dec_slots.reshape(-1).to(pre_slots.dtype)])
        both = both.tolist()  # one copy to the host
        n = pre_slots.numel()
        shared = set(both[:n]) & set(both[n:])
        if shared:
            raise RuntimeError(
                f"a tick's prefill and decode rows share slot(s) {sorted(shared)}; "
                "the two launches run side by side, so their slots must be distinct")

    def __call__(self, pool: torch.Tensor, prefill: dict, decode: dict) -> None:
        pre = [prefill[k] for k in self.PREFILL]
        plan = {"plan_lens": prefill["plan_lens"]} if "plan_lens" in prefill else {}
        dec = [decode[k] for k in self.DECODE]
        if not torch.cuda.is_current_stream_capturing():
            # Eager: in sequence, on the caller's stream. Each eager launch
            # validates its slots on the host, which synchronises its stream,
            # so two eager branches would not overlap anyway (measured 298 us
            # side by side against 216 us in sequence at config 4). In
            # sequence, shared slots do not race; check_slots verifies the
            # contract a captured tick relies on (one more copy to the host,
            # about 28 us at config 4).
            if self.check_slots:
                self._check_disjoint(prefill["slots"], decode["slots"])
            self.kern.gdn_prefill_raw(pool, *pre, **plan)
            self.kern.gdn_decode_raw(pool, *dec)
            return
        if self.side.device != pool.device:
            raise RuntimeError(f"this MixedTick's side stream is on {self.side.device}, "
                               f"the pool on {pool.device}")
        main = torch.cuda.current_stream(pool.device)
        self.side.wait_stream(main)
        # The prefill first (see the module docstring): its workgroups must
        # hold their CUs before the decode's arrive.
        self.kern.gdn_prefill_raw(pool, *pre, **plan)
        with torch.cuda.stream(self.side):
            self.kern.gdn_decode_raw(pool, *dec)
        main.wait_stream(self.side)
