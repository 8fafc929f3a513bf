"""CPU checks of the torch.library registration (no device work): the
path's entry points are custom ops of the ``glm53`` namespace whose shape
functions give the output shapes and dtypes under FakeTensor, so
torch.compile can trace a model through them without a graph break."""

from __future__ import annotations

import pytest

from conftest import submodule

torch = pytest.importorskip("torch")


def test_ops_are_registered():
    submodule("ops")
    for name in ("block_fp8_linear", "router_topk", "moe_decode", "moe_prefill"):
        assert hasattr(torch.ops.glm53, name), name


def test_fake_shapes_and_dtypes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    submodule("ops")
    with FakeTensorMode():
        x = torch.empty((2, 5, 256), dtype=torch.bfloat16)
        w = torch.empty((384, 256), dtype=torch.uint8)
        s = torch.empty((3, 2), dtype=torch.float32)
        y = torch.ops.glm53.block_fp8_linear(x, w, s, None)
        assert y.shape == (2, 5, 384) and y.dtype == torch.bfloat16
        rw = torch.empty((32, 256), dtype=torch.float32)
        rb = torch.empty((32,), dtype=torch.float32)
        ids, sc = torch.ops.glm53.router_topk(x, rw, rb, 8, 2.5, True)
        assert ids.shape == (2, 5, 8) and ids.dtype == torch.int32
        assert sc.shape == (2, 5, 8) and sc.dtype == torch.float32
        one = torch.empty((1, 1, 256), dtype=torch.bfloat16)
        assert torch.ops.glm53.moe_decode(one, 7, None, None).shape == one.shape
        assert torch.ops.glm53.moe_prefill(x, 7, ids, sc).shape == x.shape


def test_unknown_owner_raises():
    ops = submodule("ops")
    with pytest.raises(RuntimeError, match="no longer exists"):
        ops._owner(10 ** 9)
