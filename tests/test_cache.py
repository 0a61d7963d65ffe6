"""The state-pool layout contract and the bucket ladder, on the CPU (pools are
plain tensors; nothing here runs a kernel). Follows the reference's
tests/test_slot_indirection.py and braid/model/cache.py:97-232 semantics."""
from __future__ import annotations

import pytest
import torch

from braid_amd.cache import GDNCache, RecurrentCache
from braid_amd.config import GDNConfig
from braid_amd.graph import DEFAULT_BUCKETS, _zip_copy, bucket_for, usable_buckets

G = GDNConfig(n_heads=4, head_dim=128, state_size=128, n_groups=2, n_gdn_layers=3)


def test_layout_matches_the_kernel_contract():
    c = RecurrentCache(G, 5, "cpu", torch.float16)
    assert tuple(c.state.shape) == (5, 4, 128, 128) and c.state.dtype == torch.float16
    assert tuple(c.conv.shape) == (5, 2 * 2 * 128 + 4 * 128, 4) and c.conv.dtype == torch.float32
    assert c.state.is_contiguous() and c.conv.is_contiguous()
    # one (slot, head) tile is one contiguous 128x128 block
    assert c.state.stride() == (4 * 128 * 128, 128 * 128, 128, 1)
    assert (c.state == 0).all() and (c.conv == 0).all()


def test_rejected_dtypes():
    with pytest.raises(ValueError, match="fp32 / fp16 / bf16"):
        RecurrentCache(G, 2, "cpu", torch.float64)
    with pytest.raises(ValueError, match="fp32 conv pool"):
        RecurrentCache(G, 2, "cpu", torch.float16, conv_dtype=torch.bfloat16)


def _filled(state_dtype=torch.float32, slots=6):
    cache = GDNCache.allocate(G, slots, "cpu", state_dtype)
    gen = torch.Generator().manual_seed(0)
    for lyr in cache.layers:
        lyr.state.copy_(torch.randn(lyr.state.shape, generator=gen))
        lyr.conv.copy_(torch.randn(lyr.conv.shape, generator=gen))
    cache.lengths.copy_(torch.arange(slots) * 7)
    return cache


def test_reset_slot_zeroes_exactly_one_slot_in_every_layer():
    cache = _filled()
    before = cache.snapshot()
    cache.reset_slot(2)
    after = cache.snapshot()
    assert after[0][2] == 0 and torch.equal(after[0][[0, 1, 3, 4, 5]], before[0][[0, 1, 3, 4, 5]])
    for b, a in zip(before[1:], after[1:]):
        assert (a[2] == 0).all()
        keep = [0, 1, 3, 4, 5]
        assert torch.equal(a[keep], b[keep])


def test_select_shares_pools_and_carries_int32_slots():
    cache = _filled()
    view = cache.select([4, 1])
    assert view.layers is cache.layers and view.lengths is cache.lengths
    assert view.slots.tolist() == [4, 1] and view.slots_i32.dtype == torch.int32
    assert view.slots_i32.tolist() == [4, 1]
    assert view.batch_lengths.tolist() == [28, 7]


def test_snapshot_restore_round_trip():
    cache = _filled(torch.bfloat16)
    snap = cache.snapshot()
    for lyr in cache.layers:
        lyr.state.add_(1)
        lyr.conv.mul_(3)
    cache.lengths.add_(5)
    cache.restore(snap)
    for s, t in zip(snap, cache.snapshot()):
        assert torch.equal(s, t)


def test_slot_snapshot_restores_only_its_rows():
    cache = _filled(torch.float16)
    full = cache.snapshot()
    part = cache.snapshot_slots(torch.tensor([0, 3]))
    for lyr in cache.layers:
        lyr.state.zero_()
        lyr.conv.zero_()
    cache.lengths.zero_()
    cache.restore_slots(part)
    now = cache.snapshot()
    assert now[0].tolist() == [0, 0, 0, 21, 0, 0]
    for f, n in zip(full[1:], now[1:]):
        assert torch.equal(n[[0, 3]], f[[0, 3]])
        assert (n[[1, 2, 4, 5]] == 0).all()


def test_bytes():
    cache = GDNCache.allocate(G, 3, "cpu", torch.float16)
    per_layer = 3 * 4 * 128 * 128 * 2 + 3 * G.conv_channels * 4 * 4
    assert cache.bytes() == 3 * per_layer


def test_bucket_ladder():
    assert DEFAULT_BUCKETS == (1, 2, 4, 8, 16, 32, 64, 96, 128)
    sizes = usable_buckets(DEFAULT_BUCKETS, 100)
    assert sizes == (1, 2, 4, 8, 16, 32, 64, 96)
    assert [bucket_for(sizes, b) for b in (1, 3, 5, 17, 64, 65, 96)] == [1, 4, 8, 32, 64, 96, 96]
    with pytest.raises(ValueError, match="exceeds the largest bucket 96"):
        bucket_for(sizes, 97)
    with pytest.raises(ValueError, match="no bucket fits"):
        usable_buckets((8, 16), 4)


def test_static_input_copy_pads_with_zeros_and_checks_shapes():
    dst = {"x": [torch.full((4, 3), 9.0)], "y": torch.full((4, 2), 9.0)}
    _zip_copy(dst, {"x": [torch.ones(2, 3)], "y": torch.ones(2, 2)}, 2, pad=True)
    assert dst["x"][0].tolist() == [[1, 1, 1]] * 2 + [[0, 0, 0]] * 2
    assert dst["y"][2:].abs().sum() == 0
    with pytest.raises(ValueError, match="does not fit"):
        _zip_copy(dst, {"x": [torch.ones(2, 4)], "y": torch.ones(2, 2)}, 2, pad=True)
    with pytest.raises(ValueError, match="do not match"):
        _zip_copy(dst, {"x": [torch.ones(2, 3)]}, 2, pad=True)


def test_replayed_step_validates_its_slots():
    """A graph replay skips the kernels' eager slot checks, so GraphedDecoder
    checks what step() copies into the static slot buffer: range, distinct
    live slots, pad slots in range and apart from the live ones."""
    from types import SimpleNamespace

    from braid_amd.graph import GraphedDecoder

    gd = GraphedDecoder.__new__(GraphedDecoder)
    gd.cache = SimpleNamespace(max_slots=10)
    gd.check_slots(torch.tensor([3, 1, 2]), torch.tensor([9]), 1)
    gd.check_slots(torch.tensor([3, 1, 2]), torch.tensor([9, 9, 9]), 3)  # scratch may repeat
    with pytest.raises(ValueError, match=r"slot_idx\[1\] = 10 is out of range \[0, 10\)"):
        gd.check_slots(torch.tensor([3, 10]), None, 0)
    with pytest.raises(ValueError, match=r"slot_idx\[0\] = -1 is out of range"):
        gd.check_slots(torch.tensor([-1]), None, 0)
    with pytest.raises(ValueError, match="duplicate slot 3.*distinct"):
        gd.check_slots(torch.tensor([3, 1, 3]), None, 0)
    with pytest.raises(ValueError, match="pad slot 1 is also a live slot"):
        gd.check_slots(torch.tensor([3, 1]), torch.tensor([1, 9]), 2)
    with pytest.raises(ValueError, match=r"pad_slots\[0\] = 12 is out of range"):
        gd.check_slots(torch.tensor([3, 1]), torch.tensor([12]), 1)
    with pytest.raises(ValueError, match="pad_slots holds 1 slots; 2 rows"):
        gd.check_slots(torch.tensor([3, 1]), torch.tensor([9]), 2)
