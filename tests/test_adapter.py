"""Host logic of the layer-method adapter and the compaction-mode names (CPU
only: every failure here is raised before any device work)."""
import types

import pytest
import torch

from gdnx_amd import adapter, ops


def _layer(**over):
    attrs = dict(R=4, P=16, a_v=16, a_k=16, b_v=8, b_k=8, slow_decay=0.97, compact_mode="svd")
    attrs.update(over)
    return types.SimpleNamespace(**attrs)


def test_adapter_rejects_a_layer_without_the_gdn3_attributes():
    layer = _layer()
    del layer.b_k
    x = torch.zeros(1)
    with pytest.raises(AttributeError, match="b_k"):
        adapter.gdn3_recurrent_state_method(layer, x, x, x, x, x, x)


@pytest.mark.parametrize("mode", ["qr", "rsvd", ""])
def test_adapter_rejects_unknown_compaction_modes(mode):
    x = torch.zeros(1)
    with pytest.raises(NotImplementedError, match="compact_mode"):
        adapter.gdn3_recurrent_state_method(_layer(compact_mode=mode), x, x, x, x, x, x)


def test_adapter_install_binds_the_method():
    class Layer:
        pass
    adapter.install(Layer)
    assert Layer._gdn3_recurrent_state is adapter.gdn3_recurrent_state_method


def test_compaction_mode_names_and_sketch_widths():
    assert ops.compact_mode_code("svd") == 0
    assert ops.compact_mode_code("SKETCH") == 1 and ops.compact_mode_code("sketch_noqr") == 1
    assert ops.compact_mode_code(1) == 1
    for bad in ("qr", 2, -1):
        with pytest.raises(Exception):
            ops.compact_mode_code(bad)
    assert ops.sketch_width(4, 256, 64) == 8
    assert ops.sketch_width(4, 256, 64, "sketch") == 4
    assert ops.sketch_width(6, 4, 64, "svd") == 4
