"""The launch-order cache of the block-sparse plan (sinkattn_block_sparse_plan_cached).

A plan made with the cache must equal the plan made without it: the same counts and lists
(always built from the mask), and the same launch order, either ranked afresh (a miss, then
stored) or copied from an entry whose tile counts hash alike (a hit).  The order buffer's
chunk table records which: entry [slots + 25] is 1 for a copied order.  The forward over a
cached plan is bit-identical to the forward over the uncached one.  The drop-in
`_block_sparse_attn`, handed a fresh mask tensor per call as the reference's Z-Image
processor does (zimg/runtime/sink_sparse_zimage.py:513-538), runs through the cache.
"""
import math

import pytest
import torch

from sinkattn_amd import ops
from sinkattn_amd import sparse_attention as sa
from sinkattn_amd import zimage_runtime as zr

pytestmark = pytest.mark.gpu

COPIED = 25


def _mask(B, H, nqb, nkb, density, seed, dense_rows=()):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(B, H, nqb, nkb, generator=g) < density
    d = torch.arange(min(nqb, nkb))
    m[:, :, d, d] = True
    for r in dense_rows:
        m[:, :, r] = True
    return m.cuda()


def _meta_start(plan):
    """Index of the chunk table in the order buffer: the launch slots come first (the chunk
    layout of the launch order, as tests/test_gpu_block_sparse.py restates it)."""
    from math import gcd
    B, H, nqb, _ = plan.shape
    nbh = B * H
    Cw = max(1, nqb // 128)
    rem = (nbh * Cw) % 8
    nsplit = 0 if rem == 0 else -(-rem // Cw)
    F = 8 // gcd(nsplit * Cw, 8)
    while F > 1 and Cw * F > nqb:
        F //= 2
    Cs = Cw * F
    nw, ns = (nbh - nsplit) * Cw, nsplit * Cs
    slots = (-(-nw // 8) * -(-nqb // Cw) + -(-ns // 8) * -(-nqb // Cs)) * 8
    assert plan.order.numel() == slots + 32 + 2 * (nw + ns)
    return slots


def _same_plan(a, b):
    assert torch.equal(a.counts, b.counts)
    rows = a.counts.numel()
    nkb = a.shape[3]
    ia, ib = a.idx.view(rows, nkb).cpu(), b.idx.view(rows, nkb).cpu()
    for r, c in enumerate(a.counts.cpu().tolist()):
        assert torch.equal(ia[r, :c], ib[r, :c])
    s = _meta_start(a)
    assert torch.equal(a.order[:s], b.order[:s])


@pytest.mark.parametrize("B,H,nqb,nkb", [(1, 30, 132, 132), (2, 12, 256, 256), (1, 5, 300, 40)])
def test_cache_miss_then_hit_equals_uncached_plan(B, H, nqb, nkb):
    entries = 4
    cache = torch.zeros(ops.order_cache_ints(B, H, nqb, entries), dtype=torch.int32, device="cuda")
    m1 = _mask(B, H, nqb, nkb, 0.2, seed=1, dense_rows=(0, nqb - 1))
    ref = ops.block_sparse_plan(m1)
    p1 = ops.block_sparse_plan(m1, cache, entries)
    torch.cuda.synchronize()
    s = _meta_start(ref)
    assert int(p1.order[s + COPIED]) == 0                 # first time: ranked, then stored
    _same_plan(p1, ref)
    p2 = ops.block_sparse_plan(m1.clone(), cache, entries)
    torch.cuda.synchronize()
    assert int(p2.order[s + COPIED]) == 1                 # a fresh tensor, same counts: copied
    _same_plan(p2, ref)
    # same tile counts, other key blocks: the order is copied, the lists are the new mask's
    m3 = m1.cpu().clone()
    flat = m3.view(-1, nkb)
    for r in range(0, flat.shape[0], 3):
        row = flat[r]
        if 0 < int(row.sum()) < nkb:
            on = torch.nonzero(row).flatten()
            off = torch.nonzero(~row).flatten()
            row[on[0]] = False
            row[off[0]] = True
    m3 = m3.cuda()
    assert not torch.equal(m3, m1)
    ref3 = ops.block_sparse_plan(m3)
    p3 = ops.block_sparse_plan(m3, cache, entries)
    torch.cuda.synchronize()
    assert int(p3.order[s + COPIED]) == 1
    _same_plan(p3, ref3)
    # other counts: a miss, ranked afresh
    m4 = _mask(B, H, nqb, nkb, 0.35, seed=2)
    ref4 = ops.block_sparse_plan(m4)
    p4 = ops.block_sparse_plan(m4, cache, entries)
    torch.cuda.synchronize()
    assert int(p4.order[s + COPIED]) == 0
    _same_plan(p4, ref4)


def test_cache_round_robin_eviction():
    B, H, nqb, nkb, entries = 1, 4, 40, 40, 3
    cache = torch.zeros(ops.order_cache_ints(B, H, nqb, entries), dtype=torch.int32, device="cuda")
    masks = [_mask(B, H, nqb, nkb, 0.1 + 0.1 * i, seed=10 + i) for i in range(4)]
    s = None
    flags = []
    for i in [0, 1, 2, 0, 1, 2, 3, 0, 3]:
        p = ops.block_sparse_plan(masks[i].clone(), cache, entries)
        torch.cuda.synchronize()
        s = _meta_start(p) if s is None else s
        flags.append(int(p.order[s + COPIED]))
        _same_plan(p, ops.block_sparse_plan(masks[i]))
    # 0,1,2 fill the three entries; their repeats hit; 3 evicts 0 (the oldest); 0 then misses
    # and evicts 1; 3 still hits
    assert flags == [0, 0, 0, 1, 1, 1, 0, 0, 1]


def test_forward_over_cached_plan_is_bit_identical():
    B, H, N = 1, 6, 2000
    nb = math.ceil(N / 128)
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(B, H, N, 128, generator=g).to("cuda", torch.bfloat16) for _ in range(3))
    m = _mask(B, H, nb, nb, 0.3, seed=6, dense_rows=(0,))
    cache = torch.zeros(ops.order_cache_ints(B, H, nb, 8), dtype=torch.int32, device="cuda")
    want_o, want_l = ops.block_sparse_attention(q, k, v, ops.block_sparse_plan(m))
    for _ in range(3):
        o, l = ops.block_sparse_attention(q, k, v, ops.block_sparse_plan(m.clone(), cache, 8))
        torch.cuda.synchronize()
        assert torch.equal(o.view(torch.int16), want_o.view(torch.int16))
        assert torch.equal(l, want_l)


def test_drop_in_with_a_fresh_zimage_runtime_mask_per_call():
    # The reference's Z-Image processor slices the layer's package mask and forces the text
    # blocks dense on every call; each call's tensor is new, so the plan is rebuilt, its
    # launch order coming from the cache after the first call.
    B, H, N, text = 1, 4, 2048 + 256, 256
    image_blocks, total_blocks = 16, 18
    g = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(B, H, N, 128, generator=g).to("cuda", torch.bfloat16) for _ in range(3))
    pkg = torch.rand(H, total_blocks, total_blocks, generator=g) < 0.25
    pkg = pkg.cuda()
    ops.PLAN_CACHE.clear()
    outs = []
    for _ in range(3):
        rm = zr._slice_runtime_sink_mask(pkg, image_blocks=image_blocks, current_text_blocks=2,
                                         total_blocks=total_blocks)
        rm = zr._force_text_dense_runtime_mask(rm, image_blocks=image_blocks, current_text_blocks=2).unsqueeze(0)
        o, _ = sa._block_sparse_attn(q, k, v, rm, return_lse=False)
        outs.append(o.clone())
    want, _ = ops.block_sparse_attention(q, k, v, ops.block_sparse_plan(rm), return_lse=False)
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), want.view(torch.int16))


def test_plan_cached_rejects_bad_arguments():
    m = _mask(1, 2, 8, 8, 0.5, seed=9)
    small = torch.zeros(16, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        ops.block_sparse_plan(m, small, 4)
    with pytest.raises(ValueError):
        ops.block_sparse_plan(m, torch.zeros(ops.order_cache_ints(1, 2, 8, 4), dtype=torch.int64, device="cuda"), 4)


def test_cached_plan_over_the_interleaved_fallback():
    # More than 4096 chunks (4100 heads of 20 q-blocks): the plan's interleaved fallback has no
    # chunk table, and the cached plan gives the same lists and slots as the plain one
    B, H, nqb = 1, 4100, 20
    m = _mask(B, H, nqb, nqb, 0.3, seed=70)
    ref = ops.block_sparse_plan(m)
    cache = torch.zeros(ops.order_cache_ints(B, H, nqb, 2), dtype=torch.int32, device="cuda")
    for _ in range(2):
        p = ops.block_sparse_plan(m.clone(), cache, 2)
        torch.cuda.synchronize()
        assert torch.equal(p.counts, ref.counts) and torch.equal(p.order, ref.order)


def test_drop_in_on_a_side_stream_with_new_mask_tensors():
    # the drop-in keeps a launch-order cache per stream; calls on a side stream, each with a new
    # mask tensor, give the outputs of the uncached plan
    B, H, N = 1, 3, 1500
    nb = math.ceil(N / 128)
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(B, H, N, 128, generator=g).to("cuda", torch.bfloat16) for _ in range(3))
    m = _mask(B, H, nb, nb, 0.3, seed=9, dense_rows=(2,))
    want, wl = ops.block_sparse_attention(q, k, v, ops.block_sparse_plan(m))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    outs = []
    with torch.cuda.stream(side):
        for _ in range(3):
            o, l = sa._block_sparse_attn(q, k, v, m.clone())
            outs.append((o, l))
    torch.cuda.synchronize()
    for o, l in outs:
        assert torch.equal(o.view(torch.int16), want.view(torch.int16))
        assert torch.equal(l[..., 0], wl.to(l.dtype))
