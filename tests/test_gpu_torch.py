"""The PyTorch-ROCm binding (fused3s_amd.torch_ops): the fused pass on torch
tensors and torch's stream, checked against the CPU oracle, and the
graph-transformer layer (QKV GEMM -> fused attention -> output GEMM) against
an fp32 restatement of the same layer on the CPU.

Tolerances: the attention alone is held to the north-star bar (max abs 2e-3,
normwise max rel 1e-2) on the fp16 Q/K/V it was given.  The whole layer
differs from the fp32 restatement also by its fp16 GEMMs (rounded
projections and output), so it is held to max abs <= 1e-2 * max|y| + 2e-3.
"""
from __future__ import annotations

import numpy as np
import pytest
# Imported at collection, before any test loads libf3s_hip.so: the library
# then binds to torch's HIP runtime and the process holds only one.
import torch  # noqa: F401

import _oracle as orc
from conftest import GOLDEN, random_csr, rng

pytestmark = pytest.mark.gpu

ABS_TOL = 2e-3
REL_TOL = 1e-2


def close(got: np.ndarray, want: np.ndarray, what: str, abs_tol=ABS_TOL, rel_tol=REL_TOL):
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    diff = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max())
    scale = float(np.abs(want).max())
    print(f"  {what}: max_abs={diff:.3e} max_rel={diff / scale:.3e}", flush=True)
    assert diff <= abs_tol and diff / scale <= rel_tol, what


@pytest.fixture(scope="module")
def torch_ops(gpu):
    import torch
    assert torch.cuda.is_available(), "torch sees no ROCm device"
    from fused3s_amd import torch_ops
    return torch_ops


def oracle_attention(rp, ci, q, k, v, scale):
    n, H, d = q.shape
    f = lambda t: t.detach().float().cpu().numpy()   # fp16 -> fp32 exactly
    return orc.masked_attention(n, d, H, f(q), f(k), f(v), rp, ci, scale)


@pytest.mark.parametrize("case,H", [("cora", 1), ("random", 4)])
def test_attention_on_torch_tensors(torch_ops, case, H):
    import torch
    if case == "cora":
        import fused3s_amd as f3s
        g = f3s.load_csr_graph(str(GOLDEN / "cora"))
        rp, ci = g.row_ptr, g.col_ind
    else:
        rp, ci = random_csr(3000, 12, 21)
    n = len(rp) - 1
    graph = torch_ops.TorchGraph(rp, ci, heads=H)
    gen = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(n, H, 64, generator=gen).half().cuda() for _ in range(3))
    out = graph.attention(q, k, v, scale=0.125)
    torch.cuda.synchronize()
    close(out.cpu().numpy(), oracle_attention(rp, ci, q, k, v, 0.125), f"{case} H={H}")
    # same call on a side stream, into a caller-provided output
    s = torch.cuda.Stream()
    out2 = torch.full_like(out, float("nan"))
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        graph.attention(q, k, v, scale=0.125, out=out2)
    s.synchronize()
    assert torch.equal(out2.cpu(), out.cpu()), "side-stream pass differs"


def test_graph_transformer_layer(torch_ops):
    import torch
    rp, ci = random_csr(2048, 10, 22)
    n, H, in_dim = len(rp) - 1, 2, 96
    torch.manual_seed(3)
    layer = torch_ops.GraphTransformerLayer(in_dim, heads=H).cuda().half()
    graph = torch_ops.TorchGraph(rp, ci, heads=H)
    x = (torch.randn(n, in_dim) * 0.5).half()
    y = layer(x.cuda(), graph)
    torch.cuda.synchronize()
    assert y.shape == (n, in_dim) and y.dtype == torch.float16

    # fp32 restatement on the CPU: projections in fp32, Q/K/V rounded to fp16
    # as the layer hands them to the fused pass, oracle attention, fp32 W_o
    with torch.no_grad():
        Wqkv, bqkv = layer.qkv.weight.float().cpu(), layer.qkv.bias.float().cpu()
        Wo, bo = layer.proj.weight.float().cpu(), layer.proj.bias.float().cpu()
        qkv = (x.float() @ Wqkv.T + bqkv).half().view(n, 3, H, 64)
        q, k, v = (qkv[:, i].contiguous() for i in range(3))
        o = oracle_attention(rp, ci, q, k, v, 64 ** -0.5)
        yr = (torch.from_numpy(o).view(n, H * 64) @ Wo.T + bo).numpy()
    close(y.float().cpu().numpy(), yr, "layer", abs_tol=1e-2 * float(np.abs(yr).max()) + 2e-3,
          rel_tol=1.0)


def test_rejects_grad_and_bad_inputs(torch_ops):
    import torch
    rp, ci = random_csr(64, 3, 23)
    graph = torch_ops.TorchGraph(rp, ci, heads=1)
    q = torch.zeros(64, 1, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="forward-only"):
        graph.attention(q.clone().requires_grad_(), q, q)
    with pytest.raises(ValueError, match="float16"):
        graph.attention(q.float(), q, q)
    with pytest.raises(ValueError, match="shape"):
        graph.attention(q[:32], q, q)


@pytest.mark.parametrize("H", [1, 3])
def test_registered_operator(torch_ops, H):
    """torch.ops.fused3s.attention_fwd (the drop-in launch as a torch
    operator) on the block-sparse form of to_block_sparse: the converter's
    tensors equal the oracle converter's bit for bit, both semantics meet
    the oracle in the descending and natural orders, the operator's schema
    and fake (meta) implementation pass torch.library.opcheck, and bad
    operands raise."""
    import torch
    rp, ci = random_csr(1500, 9, 24)
    n = len(rp) - 1
    offs, bcol, mask = torch_ops.to_block_sparse(torch.from_numpy(rp),
                                                 torch.from_numpy(ci).long())   # int64 narrowed
    w_offs, w_bcol, w_mask = orc.convert(n, rp, ci)
    assert np.array_equal(offs.cpu().numpy(), w_offs)
    assert np.array_equal(bcol.cpu().numpy(), w_bcol)
    assert np.array_equal(mask.cpu().numpy().view(np.uint16), w_mask)
    order = torch.from_numpy(orc.window_order(w_offs)).cuda()
    gen = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(n, H, 64, generator=gen).half().cuda() for _ in range(3))
    f = lambda t: t.float().cpu().numpy()
    want_m = orc.masked_attention(n, 64, H, f(q), f(k), f(v), rp, ci, 0.25)
    want_d = orc.tile_dense_attention(n, 64, H, f(q), f(k), f(v), w_offs, w_bcol, 0.25, fast=True)
    op = torch.ops.fused3s.attention_fwd
    for o_arg in (order, None):
        got_m = op(q, k, v, offs, bcol, mask, o_arg, 0.25)
        got_d = op(q, k, v, offs, bcol, None, o_arg, 0.25)
        torch.cuda.synchronize()
        tag = "descending" if o_arg is not None else "natural"
        close(got_m.cpu().numpy(), want_m, f"operator masked {tag} H={H}")
        close(got_d.cpu().numpy(), want_d, f"operator tile-dense {tag} H={H}")
    torch.library.opcheck(op, (q, k, v, offs, bcol, mask, order, 0.25),
                          test_utils=("test_schema", "test_faketensor"))
    with pytest.raises(RuntimeError, match="forward-only"):
        op(q.clone().requires_grad_(), k, v, offs, bcol, mask, order, 0.25)
    with pytest.raises(ValueError, match="float16"):
        op(q.float(), k, v, offs, bcol, mask, order, 0.25)
    with pytest.raises(ValueError, match="window_offsets"):
        op(q, k, v, offs[:-1], bcol, mask, order, 0.25)
    with pytest.raises(ValueError, match="tile_mask"):
        op(q, k, v, offs, bcol, mask[:-1], order, 0.25)
