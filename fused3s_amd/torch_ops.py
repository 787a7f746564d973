"""PyTorch-ROCm binding of the fused pass, for a graph-transformer layer.

The reference has no framework binding; its natural caller is a graph
attention layer: a QKV projection GEMM, the fused sparse attention over the
graph's edges, and an output projection.  Here torch supplies the device
memory, the GEMMs (hipBLASLt through torch.nn.Linear) and the stream; the
attention itself is the HIP library's planned pass
(f3s_attention_fwd_planned), called on torch's current stream with the
tensors' device pointers.  There is no CPU fallback and no autograd: the
fused pass is forward-only, so calling it on tensors that require grad
raises.

    graph = TorchGraph(row_ptr, col_idx, heads=4)      # convert + plan + compile once
    o = graph.attention(q, k, v)                       # q/k/v [n, H, 64] fp16 -> fp32
    layer = GraphTransformerLayer(in_dim, heads=4).cuda().half()
    y = layer(x, graph)                                # x [n, in_dim] fp16

The drop-in launch is also a registered torch operator, on the block-sparse
form held in torch tensors (no plan, no state between calls):

    offs, bcol, mask = to_block_sparse(row_ptr, col_idx)        # GPU converter
    o = torch.ops.fused3s.attention_fwd(q, k, v, offs, bcol, mask, order, scale)
"""
from __future__ import annotations

import numpy as np
import torch

# torch ships its own HIP runtime (torch/lib/libamdhip64.so, soname
# libamdhip64.so.7).  libf3s_hip.so binds to whichever libamdhip64.so.7 the
# process loaded first, so torch must be imported before the library's first
# GPU call; loaded the other way round, the process holds two HIP runtimes
# and torch sees no device.  Refuse that state with a clear message.


def _hip_runtimes() -> set[str]:
    try:
        with open("/proc/self/maps") as f:
            return {line.split()[-1] for line in f if "libamdhip64" in line}
    except OSError:
        return set()


if len(_hip_runtimes()) > 1:
    raise ImportError("two HIP runtimes are loaded (" + ", ".join(sorted(_hip_runtimes())) +
                      "): import torch before the first fused3s_amd GPU call")

import ctypes as C

from . import _lib
from .attention import Plan
from .device import DeviceArray, Stream, check
from .graph import DeviceBSF, DeviceCSR, convert_device, window_order_device

HEAD_DIM = 64


class _TorchStream(Stream):
    """torch's current HIP stream, viewed as a library Stream (not owned)."""

    def __init__(self, handle: int):   # noqa: D107 -- no stream is created
        self.handle = handle

    def __del__(self):
        pass


def current_stream() -> Stream:
    return _TorchStream(torch.cuda.current_stream().cuda_stream)


class _TensorView(DeviceArray):
    """A torch tensor's device memory passed to the C-ABI (not owned)."""

    def __init__(self, t: torch.Tensor):   # noqa: D107 -- nothing is allocated
        self._ptr = t.data_ptr()
        self.shape = tuple(t.shape)
        self.nbytes = t.numel() * t.element_size()
        self._tensor = t

    def free(self) -> None:
        self._ptr = None   # the memory is torch's


class TorchGraph:
    """A graph prepared once for repeated fused passes: CSR on the device,
    block-sparse form with row masks (GPU converter), descending-workload
    window order, and a compiled plan for `heads` heads of 64 dims."""

    def __init__(self, row_ptr, col_idx, heads: int = 1, masked: bool = True):
        if not torch.cuda.is_available():
            raise RuntimeError("TorchGraph needs a ROCm device (no CPU fallback)")
        rp = np.ascontiguousarray(row_ptr.cpu().numpy() if torch.is_tensor(row_ptr) else row_ptr,
                                  np.int32)
        ci = np.ascontiguousarray(col_idx.cpu().numpy() if torch.is_tensor(col_idx) else col_idx,
                                  np.int32)
        self.n = len(rp) - 1
        self.nnz = len(ci)
        self.heads = heads
        self.masked = masked
        s = current_stream()
        self.csr = DeviceCSR(rp, ci, s)
        self.bsf: DeviceBSF = convert_device(self.csr, masks=True, stream=s)
        self.order = window_order_device(self.bsf, s)
        self.plan = Plan(self.bsf, self.order, H=heads, stream=s)
        if masked:
            self.plan.compile(s)

    def attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  scale: float = 1.0, out: torch.Tensor | None = None) -> torch.Tensor:
        """softmax over each node's neighbours of scale * q.k, weights applied
        to v; [n, H, 64] fp16 contiguous CUDA tensors in, [n, H, 64] fp32 out.
        masked=False gives the reference's tile-dense semantics instead."""
        shape = (self.n, self.heads, HEAD_DIM)
        for name, t in (("q", q), ("k", k), ("v", v)):
            if t.requires_grad:
                raise RuntimeError("the fused pass is forward-only (no autograd)")
            if t.dtype != torch.float16 or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous float16 CUDA tensor")
            if tuple(t.shape) != shape and tuple(t.shape) != (self.n, self.heads * HEAD_DIM):
                raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
        if out is None:
            out = torch.empty(shape, dtype=torch.float32, device=q.device)
        elif (out.dtype != torch.float32 or not out.is_contiguous()
              or out.numel() != self.n * self.heads * HEAD_DIM):
            raise ValueError("out must be a contiguous float32 tensor of n * H * 64 elements")
        self.plan.forward(_TensorView(q), _TensorView(k), _TensorView(v), _TensorView(out),
                          masked=self.masked, d=HEAD_DIM, scale=scale, stream=current_stream())
        return out


class GraphTransformerLayer(torch.nn.Module):
    """x -> [Q K V] = x W_qkv -> fused edge attention per head -> concat ->
    W_o, forward only.  Compute dtype of the projections is the module's
    (fp16 after .half()); attention accumulates and returns fp32, which is
    cast back to the projection dtype before W_o."""

    def __init__(self, in_dim: int, heads: int = 1, out_dim: int | None = None,
                 bias: bool = True):
        super().__init__()
        self.heads = heads
        self.qkv = torch.nn.Linear(in_dim, 3 * heads * HEAD_DIM, bias=bias)
        self.proj = torch.nn.Linear(heads * HEAD_DIM, out_dim or in_dim, bias=bias)
        self.scale = HEAD_DIM ** -0.5

    @torch.no_grad()
    def forward(self, x: torch.Tensor, graph: TorchGraph) -> torch.Tensor:
        if graph.heads != self.heads:
            raise ValueError("graph was planned for a different head count")
        n = x.shape[0]
        qkv = self.qkv(x).to(torch.float16).view(n, 3, self.heads, HEAD_DIM)
        q, k, v = (qkv[:, i].contiguous() for i in range(3))
        o = graph.attention(q, k, v, scale=self.scale)
        return self.proj(o.view(n, self.heads * HEAD_DIM).to(self.proj.weight.dtype))


# ------------------------------------------------------------------ operator

def _cuda_i32(t, what: str) -> torch.Tensor:
    """An int32 CUDA copy (or view) of an integer array; int64 input (the
    usual index type of torch graph code) is narrowed after a range check."""
    t = torch.as_tensor(t)
    if t.dtype == torch.int64:
        if t.numel() and (int(t.min()) < -2**31 or int(t.max()) >= 2**31):
            raise ValueError(f"{what} holds values outside the int32 range")
        t = t.to(torch.int32)
    elif t.dtype != torch.int32:
        raise ValueError(f"{what} must hold int32 (or int64) values")
    if not t.is_cuda:
        t = t.to("cuda")
    return t.contiguous()


def to_block_sparse(row_ptr, col_idx, masks: bool = True):
    """convert_csr_to_block_sparse (src/converter.cu:13-44) on the GPU into
    torch tensors: (window_offsets int32 [W + 1], block_col_indices int32
    [T], tile_mask int16 [T, 16] -- bit c of row r of a tile set iff that
    edge exists -- or None).  Two calls of f3s_convert_csr_to_bsf on torch's
    current stream: the count (one host round trip for T), then the fill."""
    rp = _cuda_i32(row_ptr, "row_ptr")
    ci = _cuda_i32(col_idx, "col_idx")
    n = rp.numel() - 1
    if n < 0:
        raise ValueError("row_ptr must hold n + 1 entries")
    W = (n + 15) // 16
    lib = _lib.hip()
    s = torch.cuda.current_stream().cuda_stream
    offs = torch.empty(W + 1, dtype=torch.int32, device=rp.device)
    T = C.c_int64(0)
    cptr = ci.data_ptr() if ci.numel() else None
    check(lib.f3s_convert_csr_to_bsf(rp.data_ptr(), cptr, n, ci.numel(), offs.data_ptr(), None,
                                     None, C.byref(T), s), "f3s_convert_csr_to_bsf(count)")
    t = int(T.value)
    # at least one element each, so the fill call gets real pointers
    bcol = torch.empty(max(t, 1), dtype=torch.int32, device=rp.device)
    mask = torch.empty((max(t, 1), 16), dtype=torch.int16, device=rp.device) if masks else None
    T2 = C.c_int64(0)
    check(lib.f3s_convert_csr_to_bsf(rp.data_ptr(), cptr, n, ci.numel(), offs.data_ptr(),
                                     bcol.data_ptr(), mask.data_ptr() if masks else None,
                                     C.byref(T2), s), "f3s_convert_csr_to_bsf(fill)")
    return offs, bcol[:t], (mask[:t] if masks else None)


def _check_operands(q, k, v, window_offsets, block_col, tile_mask, window_order):
    if q.dim() != 3 or q.shape[2] != HEAD_DIM:
        raise ValueError(f"q must be [n, H, {HEAD_DIM}]")
    n, H = q.shape[0], q.shape[1]
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.float16 or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float16 CUDA tensor")
        if tuple(t.shape) != (n, H, HEAD_DIM):
            raise ValueError(f"{name} must have shape {(n, H, HEAD_DIM)}, got {tuple(t.shape)}")
    W = (n + 15) // 16
    for name, t, shape in (("window_offsets", window_offsets, (W + 1,)),
                           ("block_col", block_col, None),
                           ("window_order", window_order, (W,))):
        if t is None:
            if name != "window_order":
                raise ValueError(f"{name} is required")
            continue
        if t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous() or t.dim() != 1:
            raise ValueError(f"{name} must be a contiguous 1-d int32 CUDA tensor")
        if shape is not None and tuple(t.shape) != shape:
            raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
    if tile_mask is not None:
        if (tile_mask.dtype not in (torch.int16, torch.uint16) or not tile_mask.is_cuda
                or not tile_mask.is_contiguous()
                or tuple(tile_mask.shape) != (block_col.shape[0], 16)):
            raise ValueError("tile_mask must be a contiguous [T, 16] int16 CUDA tensor")
    return n, H, W


@torch.library.custom_op("fused3s::attention_fwd", mutates_args=())
def attention_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  window_offsets: torch.Tensor, block_col: torch.Tensor,
                  tile_mask: torch.Tensor | None, window_order: torch.Tensor | None,
                  scale: float = 1.0) -> torch.Tensor:
    """f3s_attention_fwd (the reference's launch, tests/test_fused_3s_v2.cu:
    124-131, every window whole) on torch tensors and torch's current
    stream: q/k/v [n, H, 64] float16, the block-sparse form of
    to_block_sparse, window_order int32 [W] or None (natural order); a
    tile_mask gives the masked (edge-exact) semantics, None the reference's
    tile-dense one.  Returns O [n, H, 64] float32."""
    if q.requires_grad or k.requires_grad or v.requires_grad:
        raise RuntimeError("the fused pass is forward-only (no autograd)")
    n, H, W = _check_operands(q, k, v, window_offsets, block_col, tile_mask, window_order)
    out = torch.empty((n, H, HEAD_DIM), dtype=torch.float32, device=q.device)
    if n == 0:
        return out
    s = torch.cuda.current_stream(q.device).cuda_stream
    # an empty block_col tensor may have no storage: the C-ABI wants a pointer
    # whenever W > 0, and with T = 0 no tile is read through it
    bptr = block_col.data_ptr() or window_offsets.data_ptr()
    mptr = None
    if tile_mask is not None:
        mptr = tile_mask.data_ptr() or out.data_ptr()
    check(_lib.hip().f3s_attention_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                       window_offsets.data_ptr(), bptr, mptr,
                                       window_order.data_ptr() if window_order is not None
                                       else None, W, n, HEAD_DIM, H, float(scale), s),
          "f3s_attention_fwd")
    return out


@attention_fwd.register_fake
def _attention_fwd_fake(q, k, v, window_offsets, block_col, tile_mask, window_order, scale=1.0):
    return torch.empty(q.shape, dtype=torch.float32, device=q.device)
