"""The custom-operator registration and the per-block compile helpers, on the CPU: every
``difflet_rocm::*`` operator has a schema and a fake implementation that gives the real one's
output shape and dtype (checked under FakeTensorMode, where no kernel runs), and the compile
helpers wrap exactly the repeated blocks. The compiled GPU path is test_gpu_compile.py."""

from __future__ import annotations

import pytest
import torch
import torch.nn as nn
from torch._subclasses.fake_tensor import FakeTensorMode

from difflet_amd.backends.rocm import compile as rc
from difflet_amd.backends.rocm.ops_impl import library  # noqa: F401  (registers the ops)

OPS = ("attention", "linear", "fp8_linear", "rms_norm", "layer_norm", "rope")


def test_every_op_is_registered_with_a_schema():
    for name in OPS:
        op = getattr(torch.ops.difflet_rocm, name).default
        assert op._schema.name == f"difflet_rocm::{name}"
        # functional: no argument is written
        assert not any(a.alias_info is not None and a.alias_info.is_write
                       for a in op._schema.arguments), name


def test_fake_implementations_give_shapes_and_dtypes():
    ops = torch.ops.difflet_rocm
    with FakeTensorMode():
        bf = dict(dtype=torch.bfloat16)
        q = torch.empty(1, 4, 300, 128, **bf)
        kv = torch.empty(1, 4, 77, 128, **bf)
        o = ops.attention(q, kv, kv, 0.1, False, None, None, None)
        assert o.shape == (1, 4, 300, 128) and o.dtype == torch.bfloat16
        o = ops.attention(q.reshape(4, 300, 128), kv.reshape(4, 77, 128),
                          kv.reshape(4, 77, 128).half(), 1.0, True, None, None, None)
        assert o.shape == (4, 300, 128) and o.dtype == torch.float16
        x = torch.empty(33, 384, **bf)
        y = ops.linear(x, torch.empty(100, 384, **bf), None, 99)
        assert y.shape == (33, 99) and y.dtype == torch.bfloat16
        y = ops.fp8_linear(x, torch.empty(256, 384, dtype=torch.uint8),
                           torch.empty(256, dtype=torch.float32), None, False)
        assert y.shape == (33, 256) and y.dtype == torch.bfloat16
        h = torch.empty(2, 9, 4, 128, dtype=torch.float32)
        assert ops.rms_norm(h, None, 1e-6).shape == h.shape
        assert ops.layer_norm(x, None, None, 1e-6).dtype == torch.bfloat16
        r = ops.rope(q, torch.empty(300, 128), torch.empty(300, 128), 1)
        assert r.shape == q.shape and r.dtype == q.dtype


class _Flux(nn.Module):
    def __init__(self):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([nn.Linear(4, 4) for _ in range(2)])
        self.single_transformer_blocks = nn.ModuleList([nn.Linear(4, 4) for _ in range(3)])
        self.proj_out = nn.Linear(4, 4)


class _Wan(nn.Module):
    def __init__(self):
        super().__init__()
        self.blocks = nn.ModuleList([nn.Linear(4, 4)])


def test_repeated_blocks_and_compile_blocks():
    flux = _Flux()
    assert [len(b) for b in rc.repeated_blocks(flux)] == [2, 3]
    assert [len(b) for b in rc.repeated_blocks(_Wan())] == [1]
    outer = nn.Module()
    outer.transformer = _Flux()
    assert len(rc.repeated_blocks(outer)) == 2
    n = rc.compile_repeated_blocks_(flux, mode="default")
    assert n == 5
    assert all(type(b).__name__ == "OptimizedModule" for bl in rc.repeated_blocks(flux) for b in bl)
    assert isinstance(flux.proj_out, nn.Linear)  # the module around the blocks stays eager
    with pytest.raises(ValueError, match="repeated block lists"):
        rc.compile_repeated_blocks_(nn.Linear(2, 2))


def test_compile_options_extend_the_mode():
    blocks = nn.ModuleList([nn.Linear(2, 2)])
    assert rc.compile_blocks([blocks], dynamic=False, options={"max_autotune": False}) == 1
    assert rc.COMPILE_MODE == "max-autotune-no-cudagraphs"
