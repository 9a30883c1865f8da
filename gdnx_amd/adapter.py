"""Drop-in method for GDN3LinearAttn: the recurrence on the HIP kernels.

The reference's boundary is a bound method,
``GDN3LinearAttn._gdn3_recurrent_state(self, q_features, k_features,
v_features, b_gates, w_gates, decay_factors) -> [B,T,H,M,V] float32``
(gdn3/gdn3_upgrade.py:403-411, called from ``forward`` at :834-837).  It reads
the layer's ``R, P, a_k, b_k, a_v, b_v, slow_decay, compact_mode`` and leaves
the summed compaction error in ``self._last_comp_err`` (:525-528: a detached
device tensor, or a Python float when GDN3_SYNC_COMP_ERR=1).

``gdn3_recurrent_state_method`` is that method; ``install(cls)`` binds it on a
class (the reference's GDN3LinearAttn, a subclass, or any object with those
attributes).  Lane-expanded q/k/v (stride-0 views over M, as the layer builds
them at :785-787) are read once per head.  y is differentiable in q, k, v,
the gates and the decay (P = 16, 32 or 64); the compaction error is not.
"""
from __future__ import annotations

import os

import torch

from . import gdn3

COMPACT_MODES = ("svd", "sketch", "sketch_noqr")


def _check_layer(layer):
    missing = [a for a in ("R", "P", "a_k", "b_k", "a_v", "b_v", "slow_decay") if not hasattr(layer, a)]
    if missing:
        raise AttributeError(f"layer lacks the GDN3 attributes {missing}")
    mode = str(getattr(layer, "compact_mode", "svd")).lower()
    if mode not in COMPACT_MODES:
        raise NotImplementedError(f"compact_mode {mode!r} is not supported (one of {COMPACT_MODES})")
    return mode


def gdn3_recurrent_state_method(self, q_features, k_features, v_features, b_gates, w_gates, decay_factors):
    """GDN3LinearAttn._gdn3_recurrent_state on the GPU (see the module doc)."""
    mode = _check_layer(self)
    y, _, err = gdn3.gdn3_recurrent_state(
        q_features, k_features, v_features, b_gates, w_gates, decay_factors, R=self.R, P=self.P,
        factors=(self.a_v, self.a_k, self.b_v, self.b_k), slow_decay=self.slow_decay,
        compact_every=self.P, return_state=True, compact_mode=mode)
    if os.environ.get("GDN3_SYNC_COMP_ERR", "0") == "1":
        self._last_comp_err = float(err)
    else:
        self._last_comp_err = err.detach()
    return y.float()


def install(cls) -> None:
    """Bind gdn3_recurrent_state_method as cls._gdn3_recurrent_state."""
    cls._gdn3_recurrent_state = gdn3_recurrent_state_method
