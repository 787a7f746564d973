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

from .attention import Plan
from .device import DeviceArray, Stream
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
