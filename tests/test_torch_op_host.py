"""The registered torch operator's host side, on any host: its schema is
registered, its fake (meta) implementation gives the output's shape and
dtype without a device, and bad operands are refused before any device call.
The operator's results are checked against the oracle in
tests/test_gpu_torch.py."""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def torch_ops():
    from fused3s_amd import torch_ops
    return torch_ops


def test_operator_is_registered(torch_ops):
    op = torch.ops.fused3s.attention_fwd
    schema = str(op.default._schema)
    for arg in ("Tensor q", "Tensor k", "Tensor v", "Tensor window_offsets",
                "Tensor block_col", "Tensor? tile_mask", "Tensor? window_order", "float scale"):
        assert arg in schema, schema
    assert schema.endswith("-> Tensor")


def test_fake_implementation_gives_the_output_shape(torch_ops):
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        q = torch.empty((37, 3, 64), dtype=torch.float16, device="cuda")
        offs = torch.empty(4, dtype=torch.int32, device="cuda")
        bcol = torch.empty(9, dtype=torch.int32, device="cuda")
        mask = torch.empty((9, 16), dtype=torch.int16, device="cuda")
        o = torch.ops.fused3s.attention_fwd(q, q, q, offs, bcol, mask, None, 0.5)
        assert tuple(o.shape) == (37, 3, 64) and o.dtype == torch.float32


def test_bad_operands_are_refused_before_any_device_call(torch_ops):
    op = torch.ops.fused3s.attention_fwd
    offs = torch.zeros(3, dtype=torch.int32)
    bcol = torch.zeros(1, dtype=torch.int32)
    q16 = torch.zeros(33, 1, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="float16 CUDA"):
        op(q16.float(), q16, q16, offs, bcol, None, None, 1.0)
    with pytest.raises(ValueError, match="float16 CUDA"):
        op(q16, q16, q16, offs, bcol, None, None, 1.0)          # not on a device
    with pytest.raises(ValueError, match=r"\[n, H, 64\]"):
        op(torch.zeros(33, 1, 32, dtype=torch.float16), q16, q16, offs, bcol, None, None, 1.0)
    with pytest.raises(RuntimeError, match="forward-only"):
        op(q16.clone().requires_grad_(), q16, q16, offs, bcol, None, None, 1.0)


def test_index_narrowing(torch_ops):
    with pytest.raises(ValueError, match="int32 range"):
        torch_ops._cuda_i32(torch.tensor([0, 2**31], dtype=torch.int64), "col_idx")
    with pytest.raises(ValueError, match="int32 \\(or int64\\)"):
        torch_ops._cuda_i32(torch.tensor([0.0, 1.0]), "row_ptr")
