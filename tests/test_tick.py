"""MixedTick's host-side contract (CPU): a tick's prefill and decode rows run
side by side, so an eager tick refuses slot maps that share a slot. The GPU
behaviour (outputs and pool equal to the sequential tick's, eager and
captured, every bucket) is tested with config 4 in test_configs_gpu.py."""
import pytest
import torch

from braid_amd.tick import MixedTick


def test_disjoint_slot_maps_pass():
    MixedTick._check_disjoint(torch.tensor([96, 97, 98, 99], dtype=torch.int32),
                              torch.arange(96, dtype=torch.int32))


def test_a_shared_slot_is_refused():
    with pytest.raises(RuntimeError, match=r"share slot\(s\) \[7\]"):
        MixedTick._check_disjoint(torch.tensor([7, 100], dtype=torch.int32),
                                  torch.arange(8, dtype=torch.int32))
