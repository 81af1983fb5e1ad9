"""Import-compatible alias of the reference package name.

``import sinkattention.sparse_attention`` (and ``pooling_kernel``, ``timing``) resolves to
the corresponding ``sinkattn_amd`` module object, so code written against the reference
runs unchanged on the MI355X kernels.
"""
from sinkattn_amd import (  # noqa: F401
    SinkMaskCalibrator,
    SinkRuntimeState,
    SinkSparseConfig,
    iter_seed_list,
    load_sink_mask_package,
    parse_int_list,
    summarize_sink_package,
)
from sinkattn_amd import __all__  # noqa: F401
