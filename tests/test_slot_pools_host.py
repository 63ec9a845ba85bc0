"""Host logic of the engine slot pools (rows f-2 / f-3), on the CPU: the
routing ``GDNSlotPools.bind`` builds for the kernels, and
``install_slot_pool_patch`` on an object shaped like the reference's
``SlotPoolCache`` (engine/runtime/kv_cache.py:220-340: ``layers`` whose GDN
entries carry ``_pool_conv_states`` / ``_pool_recurrent_states``, and
``set_batch`` / ``commit_batch`` / ``batch``).  No kernel runs here."""
import types

import pytest
import torch

from engine.runtime import GDN_PAD_SLOT, GDNSlotPools, install_slot_pool_patch


def pools(num_slots=6, layers=(0, 2), max_batch=None):
    return GDNSlotPools.allocate(layers, num_slots, conv_dim=16, num_v_heads=2, head_k_dim=4, head_v_dim=4,
                                 device=torch.device("cpu"), max_batch=max_batch)


def test_bind_routes_rows_and_pads_repeats_and_out_of_range():
    p = pools()
    p.bind(torch.tensor([3, 1, 3, 7, -2, 0]), is_prefill=False)
    assert p.slots().tolist() == [3, 1, GDN_PAD_SLOT, GDN_PAD_SLOT, GDN_PAD_SLOT, 0]
    assert p.has_state().tolist() == [True] * 6 and p.decode
    p.bind(torch.tensor([5]), is_prefill=True)
    assert p.slots().tolist() == [5] and p.has_state().tolist() == [False] and not p.decode
    assert p._slots[1:].eq(GDN_PAD_SLOT).all()  # rows past the batch never address a slot


def test_bind_keeps_the_slot_buffer_in_place():
    p = pools(max_batch=4)
    ptr = p._slots.data_ptr()
    for ids in ([1, 2], [0, 1, 2, 3], [5]):
        p.bind(torch.tensor(ids), is_prefill=False)
        assert p.slots().data_ptr() == ptr  # what a captured graph reads
    with pytest.raises(ValueError):
        p.bind(torch.arange(5), is_prefill=False)


def test_verify_only_on_decode_and_commit_needs_a_verify_step():
    p = pools()
    with pytest.raises(ValueError):
        p.bind(torch.tensor([1]), is_prefill=True, verify_tokens=4)
    p.bind(torch.tensor([1, 2]), is_prefill=False)
    with pytest.raises(RuntimeError):
        p.commit_verify(torch.tensor([1, 1]))
    p.bind(torch.tensor([1, 2]), is_prefill=False, verify_tokens=4)
    assert p.snapshots(0).shape == (2, 4, 2, 4, 4) and p.verify_tokens == 4


def test_pool_shapes_are_checked():
    conv = {0: torch.zeros(4, 16, 4, dtype=torch.bfloat16)}
    with pytest.raises(ValueError):
        GDNSlotPools(conv, {0: torch.zeros(4, 2, 4, 4, dtype=torch.bfloat16)})  # recurrent pool must be fp32
    with pytest.raises(ValueError):
        GDNSlotPools(conv, {0: torch.zeros(5, 2, 4, 4)})  # slot counts differ
    with pytest.raises(ValueError):
        GDNSlotPools(conv, {1: torch.zeros(4, 2, 4, 4)})  # layer sets differ


class RefShapedCache:
    """Attribute-level stand-in for the reference SlotPoolCache: the cache
    calls set_batch / commit_batch around each forward and its GDN layers
    hold the pools under these names (kv_cache.py:171-182, 296-321)."""

    def __init__(self, num_slots=5):
        lin = lambda: types.SimpleNamespace(  # noqa: E731
            _pool_conv_states=torch.zeros(num_slots, 16, 4, dtype=torch.bfloat16),
            _pool_recurrent_states=torch.zeros(num_slots, 2, 4, 4))
        self.layers = [lin(), lin(), types.SimpleNamespace(k=torch.zeros(1)), lin()]
        self.num_slots = num_slots
        self.batch = None
        self.gathered = 0

    def set_batch(self, batch):  # the reference gathers here
        self.batch = batch
        self.gathered += 1

    def commit_batch(self):
        raise AssertionError("the patched cache has nothing to scatter")


def test_patch_routes_the_reference_cache_through_the_pools():
    cache = RefShapedCache()
    p = install_slot_pool_patch(cache)
    assert cache.gdn_slot_pools is p and sorted(p.rec) == [0, 1, 3]
    assert p.rec[3] is cache.layers[3]._pool_recurrent_states  # the cache's own tensors, not copies
    batch = types.SimpleNamespace(slot_ids=torch.tensor([2, 0, 2]), is_prefill=False)
    cache.set_batch(batch)
    assert cache.batch is batch and cache.gathered == 0
    assert p.slots().tolist() == [2, 0, GDN_PAD_SLOT]
    cache.commit_batch()
