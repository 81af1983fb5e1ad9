"""MI355X (gfx950) implementation of SinkAttention's sparse-attention hot path.

Modules mirror the reference package ``sinkattention``: ``sparse_attention``,
``pooling_kernel`` and ``timing``; ``ops`` exposes the kernels on torch tensors and
``_lib`` is the ctypes binding of libsinkattn.so (include/sinkattn.h).
"""
from sinkattn_amd.sparse_attention import (
    SinkMaskCalibrator,
    SinkRuntimeState,
    SinkSparseConfig,
    iter_seed_list,
    load_sink_mask_package,
    parse_int_list,
    summarize_sink_package,
)

__all__ = [
    "SinkMaskCalibrator",
    "SinkRuntimeState",
    "SinkSparseConfig",
    "iter_seed_list",
    "load_sink_mask_package",
    "parse_int_list",
    "summarize_sink_package",
]
