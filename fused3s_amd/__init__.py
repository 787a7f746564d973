"""fused3s_amd -- MI355X (gfx950) fused sparse graph attention.

The hot path of fatalhawk/fused3S -- CSR load, CSR -> 16x16 block-sparse
conversion (with intra-tile masks), descending-workload window order and the
fused SDDMM -> online softmax -> SpMM pass -- behind the reference's host API
(graph.load_csr_graph, graph.convert_csr_to_block_sparse,
graph.generate_balanced_window_order) and the C-ABI of libf3s_hip.so.
Every compute call goes to the HIP library; there is no CPU fallback.
"""
from .device import (DeviceArray, Event, F3SError, Stream, device_count, device_name, init,
                     synchronize)
from .graph import (BlockSparseFormat, DeviceBSF, DeviceCSR, GraphData, bsf_stats,
                    convert_csr_to_block_sparse, convert_device, generate_balanced_window_order,
                    load_csr_graph, load_graph, save_graph, window_order_device)
from .attention import (Plan, attention_fwd, attention_fwd_timed, cast_f32_to_f16,
                        naive_attention_fwd, probe_gather)
from .configs import CONFIGS, Config

__all__ = [
    "DeviceArray", "Event", "F3SError", "Stream", "device_count", "device_name", "init",
    "synchronize",
    "BlockSparseFormat", "DeviceBSF", "DeviceCSR", "GraphData", "bsf_stats",
    "convert_csr_to_block_sparse", "convert_device", "generate_balanced_window_order",
    "load_csr_graph", "load_graph", "save_graph", "window_order_device", "Plan",
    "attention_fwd", "attention_fwd_timed", "cast_f32_to_f16", "naive_attention_fwd",
    "probe_gather",
    "CONFIGS", "Config",
]
