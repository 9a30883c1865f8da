"""Decode-state cache for serving the lane-shared delta rule.

The reference keeps no recurrent cache (GDN3LinearAttn.forward swallows
cache_params, gdn3/gdn3_upgrade.py:725), so a serving loop there re-runs the
whole prefix.  Here every sequence owns a slot of one state pool
[n_slots, H, M, D, D] float32 in HBM (64 KB per chain at D = 128):

  * ``prefill`` runs the chunked forward (gdnx_delta_chunk_fwd) over a
    prompt from the slots' current states and writes the final states back;
  * ``step`` advances one token for a batch whose rows name their slots
    (gdnx_delta_decode_step_slots, one HBM read and write of each state), so
    sequences join and leave the batch without moving states;
  * ``alloc`` / ``free`` / ``reset`` manage the slots on the host.

The arithmetic is the HIP kernels'; the pool gathers and scatters of the
prefill are device copies.
"""
from __future__ import annotations

import torch

from . import ops


class DecodeStateCache:
    def __init__(self, n_slots: int, H: int, M: int, D: int, device="cuda"):
        self.pool = torch.zeros(n_slots, H, M, D, D, dtype=torch.float32, device=device)
        self.n_slots, self.H, self.M, self.D = n_slots, H, M, D
        self._free = list(range(n_slots - 1, -1, -1))

    # ---- slots ----
    def alloc(self, n: int = 1) -> list:
        """n free slots, zero-initialised."""
        if n > len(self._free):
            raise RuntimeError(f"decode cache full: {n} slots asked, {len(self._free)} free")
        slots = [self._free.pop() for _ in range(n)]
        self.reset(slots)
        return slots

    def free(self, slots) -> None:
        for s in slots:
            if not 0 <= s < self.n_slots or s in self._free:
                raise ValueError(f"slot {s} is not allocated")
            self._free.append(s)

    def reset(self, slots) -> None:
        idx = torch.as_tensor(list(slots), dtype=torch.long, device=self.pool.device)
        self.pool.index_fill_(0, idx, 0.0)

    def _slot_tensor(self, slots):
        if isinstance(slots, torch.Tensor):
            return slots.to(device=self.pool.device, dtype=torch.int32).contiguous()
        return torch.as_tensor(list(slots), dtype=torch.int32, device=self.pool.device)

    # ---- compute ----
    def prefill(self, slots, q, k, v, a_e, a_w, log_g):
        """Chunked forward of q, k, v [B,T,H,D] and a_e, a_w, log_g
        [B,T,H,M] for the B sequences in ``slots``, starting from their
        cached states; the final states go back to the slots.  Returns y
        [B,T,H,M,D]."""
        idx = torch.as_tensor(list(slots), dtype=torch.long, device=self.pool.device)
        state0 = self.pool.index_select(0, idx)
        y, s_out, _ = ops.delta_chunk_fwd(q.contiguous(), k.contiguous(), v.contiguous(), a_e.float().contiguous(),
                                          a_w.float().contiguous(), log_g.float().contiguous(), state0,
                                          return_state=True)
        self.pool.index_copy_(0, idx, s_out)
        return y

    def step(self, slots, q, k, v, a_e, a_w, log_g, out=None):
        """One token for each row s of q, k, v [NS,H,D] and a_e, a_w, log_g
        [NS,H,M], advancing slot slots[s] (-1: an empty row, y = 0).
        Returns y [NS,H,M,D]."""
        return ops.delta_decode_step_slots(q.contiguous(), k.contiguous(), v.contiguous(), a_e.float().contiguous(),
                                           a_w.float().contiguous(), log_g.float().contiguous(), self.pool,
                                           self._slot_tensor(slots), out=out)
