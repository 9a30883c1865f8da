"""Decode-state cache for serving the recurrences one token at a time.

The reference keeps no recurrent cache (GDN3LinearAttn.forward swallows
cache_params, gdn3/gdn3_upgrade.py:725; KMD2NativeAttn re-runs its scan), so a
serving loop there re-runs the whole prefix.  Here every sequence owns a slot
of a state pool in HBM, and three state kinds are kept:

  * ``"dense"``: the lane-shared delta rule with one log-decay per chain
    (the GDN3 dense regime, KMD-2 with a per-token decay): S [n_slots, H, M,
    D, D] float32, prefill through gdnx_delta_chunk_fwd, steps through
    gdnx_delta_decode_step_slots;
  * ``"chan"``: the KMD-2 native state with a decay per key channel
    (research/kernel_ab/ref_scan.py:24-48): S [n_slots, H, 1, D, D], prefill
    through gdnx_delta_chan_fwd, steps through gdnx_delta_decode_step_chan;
  * ``"gdn3"``: the GDN3 Kronecker-residual state of the reference layer
    (gdn3/_reference_recurrence.py:52-55): A, B, U, Vb per (slot, head, lane)
    plus each slot's token count, prefill through gdnx_gdn3_chunk_fwd_state,
    steps through gdnx_gdn3_decode_step (compaction when a slot's token count
    reaches a multiple of the compaction interval).  The compaction sketch has
    one row block per slot, so a sequence's compactions do not depend on the
    other sequences in its batch.

``step`` advances one token for a batch whose rows name their slots (-1: an
empty row, y = 0); sequences join and leave without moving states.  The
arithmetic is the HIP kernels'; the pool gathers and scatters of a prefill
are device copies.
"""
from __future__ import annotations

import torch

from . import gdn3, ops

KINDS = ("dense", "chan", "gdn3")


class DecodeStateCache:
    def __init__(self, n_slots: int, H: int, M: int, D: int, device="cuda", kind: str = "dense", *,
                 R: int = 4, P: int = 16, factors=None, slow_decay: float = 0.97, compact_every=None,
                 compact_mode: str = "svd"):
        if kind not in KINDS:
            raise ValueError(f"kind must be one of {KINDS}, got {kind!r}")
        if kind == "chan" and M != 1:
            raise ValueError("the per-channel (KMD-2) state has one chain per head: M must be 1")
        self.kind, self.n_slots, self.H, self.M, self.D = kind, n_slots, H, M, D
        self.device = torch.device(device)
        self._free = list(range(n_slots - 1, -1, -1))
        if kind == "gdn3":
            if factors is None:
                factors = (16, 16, 8, 8) if D == 128 else (8, 8, 8, 8)
            a_v, a_k, b_v, b_k = factors
            self.R, self.P, self.factors, self.slow_decay = R, P, tuple(factors), slow_decay
            self.compact_every = P if compact_every is None else int(compact_every)
            self.compact_mode = ops.compact_mode_code(compact_mode)
            dev = self.device
            self.A = torch.zeros(n_slots, H, M, R, a_v, a_k, device=dev)
            self.B = torch.zeros(n_slots, H, M, R, b_v, b_k, device=dev)
            self.U = torch.zeros(n_slots, H, M, D, P, device=dev)
            self.Vb = torch.zeros(n_slots, H, M, D, P, device=dev)
            qw = ops.sketch_width(R, a_v * a_k, b_v * b_k, self.compact_mode)
            self.sketch = gdn3.default_sketch(n_slots * H * M, b_v * b_k, qw, dev)
            self.pos = [0] * n_slots          # tokens each slot has seen
        else:
            self.pool = torch.zeros(n_slots, H, M, D, D, dtype=torch.float32, device=self.device)

    # ---- slots ----
    def alloc(self, n: int = 1) -> list:
        """n free slots, zero-initialised."""
        if n > len(self._free):
            raise RuntimeError(f"decode cache full: {n} slots asked, {len(self._free)} free")
        slots = [self._free.pop() for _ in range(n)]
        self.reset(slots)
        return slots

    def free(self, slots) -> None:
        """Return slots to the pool; the whole list is checked before any is freed."""
        slots = [int(s) for s in slots]
        free = set(self._free)
        if len(set(slots)) != len(slots):
            raise ValueError(f"slots {slots} name a slot twice")
        for s in slots:
            if not 0 <= s < self.n_slots or s in free:
                raise ValueError(f"slot {s} is not allocated")
        self._free.extend(slots)

    def reset(self, slots) -> None:
        slots = [int(s) for s in slots]
        idx = torch.as_tensor(slots, dtype=torch.long, device=self.device)
        if self.kind == "gdn3":
            for t in (self.A, self.B, self.U, self.Vb):
                t.index_fill_(0, idx, 0.0)
            for s in slots:
                self.pos[s] = 0
        else:
            self.pool.index_fill_(0, idx, 0.0)

    def state(self, slot: int):
        """The state of one slot (views): S [H, M, D, D], or (A, B, U, Vb)
        with leading dims [H, M] for the gdn3 kind."""
        if self.kind == "gdn3":
            return self.A[slot], self.B[slot], self.U[slot], self.Vb[slot]
        return self.pool[slot]

    def _slot_tensor(self, slots):
        """The slots as an int32 device tensor, after checking on the host that
        no live slot is named twice (two rows advancing one state would race in
        the kernels).  A tensor is read back for the check (one sync)."""
        host = [int(s) for s in (slots.tolist() if isinstance(slots, torch.Tensor) else slots)]
        live = [s for s in host if 0 <= s < self.n_slots]
        if len(set(live)) != len(live):
            raise ValueError(f"slots {host} name a slot twice (rows sharing a slot would race)")
        if isinstance(slots, torch.Tensor):
            return slots.to(device=self.device, dtype=torch.int32).contiguous()
        return torch.as_tensor(host, dtype=torch.int32, device=self.device)

    # ---- compute ----
    def prefill(self, slots, q, k, v, a_e, a_w, log_g):
        """Chunked forward over a prompt for the B sequences in ``slots``,
        from their cached states; the final states go back to the slots.

        dense: q, k, v [B,T,H,D], a_e, a_w, log_g [B,T,H,M].
        chan:  q, k, v [B,T,H,D], a_e, a_w [B,T,H], log_g [B,T,H,D].
        gdn3:  q, k, v [B,T,H,(M,)D], a_e = b_gates, a_w = w_gates
               ([B,T,H,M] or [B,T,H,M,D]), log_g = the multiplicative decay
               [B,T,H,M]; every slot of the call must hold the same number
               of tokens.
        Returns y [B,T,H,M,D] ([B,T,H,D] for chan)."""
        slots = [int(s) for s in slots]
        idx = torch.as_tensor(slots, dtype=torch.long, device=self.device)
        if self.kind == "gdn3":
            t0 = self.pos[slots[0]]
            if any(self.pos[s] != t0 for s in slots):
                raise ValueError("gdn3 prefill: the slots of one call must hold equal token counts "
                                 f"(got {[self.pos[s] for s in slots]})")
            Bn, HM = len(slots), self.H * self.M
            st0 = tuple(t.index_select(0, idx).reshape(Bn * HM, *t.shape[3:]) for t in (self.A, self.B, self.U,
                                                                                            self.Vb))
            G = self.sketch.view(self.n_slots, HM, *self.sketch.shape[1:]).index_select(0, idx)
            with torch.no_grad():
                y, st, _ = gdn3.gdn3_recurrent_state(q, k, v, a_e, a_w, log_g, R=self.R, P=self.P,
                                                     factors=self.factors, slow_decay=self.slow_decay,
                                                     compact_every=self.compact_every,
                                                     sketch=G.reshape(Bn * HM, *G.shape[2:]), return_state=True,
                                                     state0=st0, t0=t0, compact_mode=self.compact_mode)
            for pool, s_new in zip((self.A, self.B, self.U, self.Vb), st):
                pool.index_copy_(0, idx, s_new.view(Bn, self.H, self.M, *s_new.shape[1:]))
            T = log_g.shape[1]
            for s in slots:
                self.pos[s] += T
            return y
        state0 = self.pool.index_select(0, idx)
        if self.kind == "chan":
            y, s_out, _ = ops.delta_chan_fwd(*(t.float().contiguous() for t in (q, k, v, a_e, a_w, log_g)),
                                             state0[:, :, 0].contiguous())
            self.pool.index_copy_(0, idx, s_out.unsqueeze(2))
            return y
        y, s_out, _ = ops.delta_chunk_fwd(q.contiguous(), k.contiguous(), v.contiguous(), a_e.float().contiguous(),
                                          a_w.float().contiguous(), log_g.float().contiguous(), state0,
                                          return_state=True)
        self.pool.index_copy_(0, idx, s_out)
        return y

    def step(self, slots, q, k, v, a_e, a_w, log_g, out=None):
        """One token for each row s, advancing slot slots[s] (-1: an empty
        row, y = 0).  dense: q, k, v [NS,H,D], a_e, a_w, log_g [NS,H,M].
        chan: the same with log_g [NS,H,M,D] (M = 1).  gdn3: q, k, v
        [NS,H,(M,)D], a_e = b_gates, a_w = w_gates ([NS,H,M] or [NS,H,M,D]),
        log_g = the multiplicative decay [NS,H,M].  Returns y [NS,H,M,D]."""
        st = self._slot_tensor(slots)
        if self.kind == "gdn3":
            host = st.tolist() if isinstance(slots, torch.Tensor) else [int(s) for s in slots]
            pos = torch.tensor([self.pos[s] if 0 <= s < self.n_slots else 0 for s in host], dtype=torch.int32,
                               device=self.device)
            with torch.no_grad():
                y = gdn3.gdn3_decode_step(q, k, v, a_e, a_w, log_g, (self.A, self.B, self.U, self.Vb), pos,
                                          R=self.R, P=self.P, factors=self.factors, slow_decay=self.slow_decay,
                                          compact_every=self.compact_every, sketch=self.sketch, slots=st,
                                          compact_mode=self.compact_mode)
            for s in host:
                if 0 <= s < self.n_slots:
                    self.pos[s] += 1
            return y
        if self.kind == "chan":
            return ops.delta_decode_step_chan(q.contiguous(), k.contiguous(), v.contiguous(),
                                              a_e.float().contiguous(), a_w.float().contiguous(),
                                              log_g.float().contiguous(), self.pool, st, out=out)
        return ops.delta_decode_step_slots(q.contiguous(), k.contiguous(), v.contiguous(), a_e.float().contiguous(),
                                           a_w.float().contiguous(), log_g.float().contiguous(), self.pool, st,
                                           out=out)
