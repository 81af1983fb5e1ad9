"""Max-pool block statistics, drop-in for ``sinkattention.pooling_kernel``.

``attn_with_pooling(q, k, v, causal, sm_scale, block_size) -> (o, Po)`` keeps the
reference's signature and outputs (sinkattention/pooling_kernel.py:194-248): ``o`` is
all zeros in q's dtype (the reference kernel never accumulates into it) and ``Po`` is
the row-normalised max-pool map [B, H, nd, nd] in q's dtype.  ``Po`` comes from the
max_pool HIP kernel, a persistent kernel whose work-groups each keep the per-(row,
key-block) maxima of the one query block in flight in a workspace slot, instead of the
reference's [B, H, N, nd] scratch tensor.
"""
from __future__ import annotations

import torch

from sinkattn_amd import ops


def attn_with_pooling(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
                      sm_scale: float, block_size: int):
    assert block_size in {16, 32, 64, 128}
    assert q.shape[-1] == k.shape[-1] == v.shape[-1]
    assert k.shape[-1] in {16, 32, 64, 128, 256}
    assert k.shape[1] == v.shape[1]
    po = ops.max_pool_scores(q, k, float(sm_scale), block_size=int(block_size), causal=bool(causal))
    o = torch.zeros_like(q)
    return o, po


__all__ = ["attn_with_pooling"]
