"""Kernel-side slot indexing for the engine's GDN state pools, and the
speculative-verify rollback.

The reference's ``SlotPoolCache`` (engine/runtime/kv_cache.py:220-560) keeps
each GDN layer's state as two slot pools -- conv ``[slots, conv_dim, 4]``
bf16 and recurrent ``[slots, Hv, K, V]`` fp32 (``_LinearAttentionSlotLayer``,
:134-212) -- and around every forward copies the batch's rows out
(``index_select(...).clone()``, :189-193) and back (``index_copy_``,
:195-208): extra passes over the whole state every step, and a fresh
allocation every step that its CUDA-graph runner has to work around
(cuda_graphs.py:36-71).  Here the GDN layer forward hands the pools and the
batch's slot ids to the kernels, which read and update ``pool[slot]`` in
place:

* :class:`GDNSlotPools` holds the pools of every GDN layer and one
  persistent slot-id buffer; :meth:`GDNSlotPools.bind` routes the next
  forward (outside any captured graph; the graph reads the buffer).
* :func:`install_slot_pool_patch` puts a reference ``SlotPoolCache`` on
  that path: its ``set_batch`` / ``commit_batch`` stop gathering and
  scattering, and ``gated_delta_net_forward`` finds the pools through
  ``cache.gdn_slot_pools``.
* Speculative verify (no reference implementation; spec_decode.py:81-87 and
  :99-103 record that GDN rollback "requires saving state snapshots"): a
  forward bound with ``verify_tokens=T`` records, per GDN layer, the state
  after each of the T tokens and the conv history of the step;
  :meth:`GDNSlotPools.commit_verify` then rolls every layer back to the
  state after each sequence's accepted tokens.
"""
from __future__ import annotations

from typing import Dict, Iterable, Optional, Tuple

import torch

from ..kernels.state_pool import gdn_conv_state_commit, gdn_state_commit

# A slot id the kernels treat as "no slot": zero state, nothing written.
GDN_PAD_SLOT = -1


class GDNSlotPools:
    """The GDN half of a slot-pool cache.

    ``conv_pools[layer]`` ``[slots, C, S]`` (bf16, fp16 or fp32) and
    ``rec_pools[layer]`` ``[slots, Hv, K, V]`` fp32 are the pools of each GDN
    layer (the cache's own tensors, not copies).  ``max_batch`` bounds the
    rows of one forward (graph buckets included).
    """

    def __init__(self, conv_pools: Dict[int, torch.Tensor], rec_pools: Dict[int, torch.Tensor],
                 max_batch: Optional[int] = None):
        if not rec_pools or set(conv_pools) != set(rec_pools):
            raise ValueError("need conv and recurrent pools for the same, non-empty set of layers")
        self.conv = dict(conv_pools)
        self.rec = dict(rec_pools)
        first = next(iter(self.rec.values()))
        self.device = first.device
        self.num_slots = int(first.shape[0])
        for i in self.rec:
            r, c = self.rec[i], self.conv[i]
            if r.dtype != torch.float32 or r.dim() != 4 or not r.is_contiguous():
                raise ValueError(f"layer {i}: recurrent pool must be contiguous fp32 [slots, Hv, K, V]")
            if c.dim() != 3 or not c.is_contiguous() or c.dtype not in (torch.bfloat16, torch.float16, torch.float32):
                raise ValueError(f"layer {i}: conv pool must be contiguous [slots, C, S] bf16, fp16 or fp32")
            if r.shape[0] != self.num_slots or c.shape[0] != self.num_slots:
                raise ValueError(f"layer {i}: pools hold different slot counts")
            if r.device != self.device or c.device != self.device:
                raise ValueError(f"layer {i}: pools on different devices")
        self.max_batch = int(max_batch or self.num_slots)
        self._slots = torch.full((self.max_batch,), GDN_PAD_SLOT, dtype=torch.int64, device=self.device)
        self._has_state = torch.zeros(self.max_batch, dtype=torch.bool, device=self.device)
        self.batch_size = 0
        self.decode = False
        self.verify_tokens = 0
        self._snap: Dict[int, torch.Tensor] = {}
        self._hist: Dict[int, torch.Tensor] = {}
        self._verify_len = 0

    @classmethod
    def allocate(cls, layer_ids: Iterable[int], num_slots: int, conv_dim: int = 8192, conv_kernel: int = 4,
                 num_v_heads: int = 32, head_k_dim: int = 128, head_v_dim: int = 128,
                 device: Optional[torch.device] = None, conv_dtype: torch.dtype = torch.bfloat16,
                 max_batch: Optional[int] = None) -> "GDNSlotPools":
        """Zeroed pools with the reference cache's shapes and dtypes (kv_cache.py:175-182)."""
        device = device or torch.device("cuda")
        conv, rec = {}, {}
        for i in layer_ids:
            conv[i] = torch.zeros(num_slots, conv_dim, conv_kernel, dtype=conv_dtype, device=device)
            rec[i] = torch.zeros(num_slots, num_v_heads, head_k_dim, head_v_dim, dtype=torch.float32,
                                 device=device)
        return cls(conv, rec, max_batch)

    # ------------------------------------------------------------- routing
    def bind(self, slot_ids: torch.Tensor, is_prefill: bool, verify_tokens: int = 0) -> None:
        """Route the next forward: batch row b uses ``pool[slot_ids[b]]``.

        A row whose slot repeats an earlier row's (the CUDA-graph runner pads
        a bucket by repeating row 0, cuda_graphs.py:473-497) or lies outside
        ``[0, num_slots)`` becomes ``GDN_PAD_SLOT``: the kernels give it a zero
        state and write nothing, so padding can never race a real row for a
        slot or reach past a pool.  ``is_prefill`` rows start from a zero
        state (the reference's prefill ignores what the slot held); decode
        rows continue from their slot.  ``verify_tokens=T`` (decode only)
        makes the forward record what :meth:`commit_verify` needs.
        """
        ids = slot_ids.to(device=self.device, dtype=torch.int64).reshape(-1)
        b = ids.numel()
        if b > self.max_batch:
            raise ValueError(f"batch of {b} rows exceeds max_batch={self.max_batch}")
        if verify_tokens and is_prefill:
            raise ValueError("verify_tokens applies to decode steps only")
        if int(verify_tokens) < 0:
            raise ValueError(f"verify_tokens={verify_tokens} must be >= 0 (0: no verify step)")
        ok = (ids >= 0) & (ids < self.num_slots)
        if b > 1:
            earlier = torch.tril(ids.unsqueeze(0) == ids.unsqueeze(1), diagonal=-1).any(dim=1)
            ok &= ~earlier
        self._slots[:b].copy_(torch.where(ok, ids, torch.full_like(ids, GDN_PAD_SLOT)))
        self._slots[b:].fill_(GDN_PAD_SLOT)
        self._has_state.fill_(not is_prefill)
        self.batch_size = b
        self.decode = not is_prefill
        if verify_tokens:
            self._ensure_verify_buffers(int(verify_tokens))
        self.verify_tokens = int(verify_tokens)

    def slots(self) -> torch.Tensor:
        """Slot ids of the bound batch (a view of the persistent buffer)."""
        return self._slots[: self.batch_size]

    def has_state(self) -> torch.Tensor:
        """Per row: continue from the slot's state (decode) or start from zero (prefill)."""
        return self._has_state[: self.batch_size]

    def layer(self, layer_idx: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """(conv pool, recurrent pool) of a GDN layer."""
        if layer_idx not in self.rec:
            raise KeyError(f"layer {layer_idx} has no GDN pools")
        return self.conv[layer_idx], self.rec[layer_idx]

    def reset_slot(self, slot_id: int) -> None:
        """Zero a slot in every layer (the reference's ``reset_slot``, kv_cache.py:210-212)."""
        for i in self.rec:
            self.conv[i][slot_id].zero_()
            self.rec[i][slot_id].zero_()

    # ------------------------------------------------------------- speculative verify
    def _ensure_verify_buffers(self, t: int) -> None:
        if t == self._verify_len:
            return
        for i in self.rec:
            c, r = self.conv[i], self.rec[i]
            self._snap[i] = torch.empty((self.max_batch, t) + tuple(r.shape[1:]), dtype=torch.float32,
                                        device=self.device)
            self._hist[i] = torch.empty((self.max_batch, c.shape[1], c.shape[2] + t), dtype=c.dtype,
                                        device=self.device)
        self._verify_len = t

    def snapshots(self, layer_idx: int) -> torch.Tensor:
        """``[B, T, Hv, K, V]``: the verify step's state after each token."""
        return self._snap[layer_idx][: self.batch_size]

    def record_conv(self, layer_idx: int, x: torch.Tensor) -> None:
        """Keep a verify step's conv history before the conv kernel moves the
        windows on: the rows' current windows, then the step's inputs
        ``x`` ``[B, C, T]`` (pre-conv)."""
        c = self.conv[layer_idx]
        s = c.shape[2]
        hist = self._hist[layer_idx][: self.batch_size]
        hist[:, :, :s].copy_(c.index_select(0, self.slots().clamp(min=0)))
        hist[:, :, s:].copy_(x)

    def commit_verify(self, accepted_len: torch.Tensor) -> None:
        """Roll every GDN layer back to the state after each row's first
        ``accepted_len[b]`` verify tokens (1 = only the last real token; T =
        the whole draft accepted): the recurrent state from the step's
        snapshots, the conv window from its history."""
        if not self.verify_tokens:
            raise RuntimeError("commit_verify without a bound verify step")
        acc = accepted_len.to(device=self.device, dtype=torch.int32).reshape(-1)
        if acc.numel() != self.batch_size:
            raise ValueError(f"accepted_len has {acc.numel()} entries for {self.batch_size} rows")
        acc = acc.clamp(min=0, max=self.verify_tokens)
        slots = self.slots()
        for i in self.rec:
            gdn_state_commit(self.rec[i], slots, self.snapshots(i), acc)
            gdn_conv_state_commit(self.conv[i], slots, self._hist[i][: self.batch_size], acc)
        self.verify_tokens = 0


def install_slot_pool_patch(cache, max_batch: Optional[int] = None) -> GDNSlotPools:
    """Put a reference ``SlotPoolCache`` (engine/runtime/kv_cache.py:220) on
    kernel-side slot indexing and return its :class:`GDNSlotPools`.

    The cache's GDN layers (those with ``_pool_conv_states`` /
    ``_pool_recurrent_states``, :171-182) keep their pools; ``set_batch``
    (:296-307) binds the batch's slot ids instead of gathering, and
    ``commit_batch`` (:309-321) has nothing left to scatter.  Full-attention
    layers are untouched (they write their pools in ``update``).  Run the
    model with :func:`engine.kernels.install_gdn_layer_patch` so that the GDN
    layers' forward reads ``cache.gdn_slot_pools``.
    """
    conv, rec = {}, {}
    for i, layer in enumerate(cache.layers):
        if hasattr(layer, "_pool_recurrent_states") and hasattr(layer, "_pool_conv_states"):
            conv[i] = layer._pool_conv_states
            rec[i] = layer._pool_recurrent_states
    pools = GDNSlotPools(conv, rec, max_batch)

    def set_batch(batch) -> None:
        cache.batch = batch
        pools.bind(batch.slot_ids, batch.is_prefill)

    def commit_batch() -> None:
        return None

    cache.set_batch = set_batch
    cache.commit_batch = commit_batch
    cache.gdn_slot_pools = pools
    return pools
