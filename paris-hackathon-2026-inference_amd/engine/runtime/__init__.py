"""Engine-side plumbing around the GDN kernels: slot-indexed state pools
and the speculative-verify rollback (:mod:`engine.runtime.slot_pools`)."""
from .slot_pools import GDN_PAD_SLOT, GDNSlotPools, install_slot_pool_patch

__all__ = ["GDN_PAD_SLOT", "GDNSlotPools", "install_slot_pool_patch"]
