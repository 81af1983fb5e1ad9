"""GPU parity of the block-score kernels.

exact mode  vs oracle/torch_ref.exact_block_mass (fp32 restatement of
            sparse_attention.py:145-227): elementwise rtol 1e-5 (atol 1e-8); rows of the
            map sum to 1.
max mode    vs oracle/torch_ref.max_pool_map (the reference's four rounding points in
            q.dtype, pinned bit for bit against the reference kernel's own outputs in
            tests/test_golden_max_pool.py): `parity_bars.max_pool_bar`, i.e. entries within
            the factor 2^ulp(max |R|) plus two ulps of q.dtype, at most 0.2% of the entries
            beyond a 2-ulp ripple and 8% of the rows touched, each such entry explained by
            a row near a rounding boundary (q.k is summed in another order on the matrix
            cores than on the CPU).
mean mode   vs oracle/torch_ref.mean_pool_scores: rtol 1e-5.
"""
import math

import pytest
import torch

from oracle import torch_ref
from parity_bars import max_block_logit, max_pool_bar
from sinkattn_amd import ops
from sinkattn_amd import sparse_attention as sa

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-5, 1e-8


def _qk(B, H, Nq, Nk, dtype, seed, sinks=0, sink_scale=8.0, sink_at_end=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Nq, 128, generator=g)
    k = torch.randn(B, H, Nk, 128, generator=g)
    if sinks:
        if sink_at_end:
            k[:, :, -sinks:] *= sink_scale
        else:
            k[:, :, :sinks] *= sink_scale
    return q.to(dtype), k.to(dtype)


def _max_pool_close(ours, ref, q, k, sm, block=128, causal=False, what=""):
    max_pool_bar(ours, ref, max_block_logit(q, k, sm, block, causal), what, qk=(q, k, sm, block, causal))


def _close(ours, ref):
    ours = ours.cpu().double()
    ref = ref.cpu().double()
    bad = (ours - ref).abs() > ATOL + RTOL * ref.abs()
    assert not bad.any(), f"{bad.sum().item()} elements, max rel {((ours - ref).abs() / ref.abs().clamp_min(1e-30)).max().item():.3g}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("N", [384, 1000])
def test_exact_mass_small(dtype, N):
    q, k = _qk(1, 2, N, N, dtype, seed=N, sinks=4)
    ours = ops.block_mass_scores(q.cuda(), k.cuda())
    ref = torch_ref.exact_block_mass(q, k)
    _close(ours, ref)
    assert torch.allclose(ours.sum(-1).cpu(), torch.ones(1, 2, ours.shape[2]), atol=1e-5)


def test_exact_mass_config1_fp32():
    # [1,12,4096,128] fp32 with 4 sink keys scaled 8x -> [1,12,32,32]
    q, k = _qk(1, 12, 4096, 4096, torch.float32, seed=0, sinks=4)
    cfg = sa.SinkSparseConfig(pooling_mode="exact")
    ours = sa._compute_block_scores(q.cuda(), k.cuda(), k.cuda(), cfg)
    assert ours.shape == (1, 12, 32, 32) and ours.dtype == torch.float32
    ref = torch_ref.exact_block_mass(q, k)
    _close(ours, ref)


def test_exact_mass_rescale_path_sinks_last():
    # the running maximum keeps rising (sinks at the end, growing key norms): exercises
    # the per-row rescaling of earlier key-block sums
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 512, 128, generator=g)
    k = torch.randn(1, 2, 1500, 128, generator=g) * torch.linspace(0.2, 3.0, 1500).view(1, 1, -1, 1)
    for dt in (torch.bfloat16, torch.float32):
        qq, kk = q.to(dt), k.to(dt)
        _close(ops.block_mass_scores(qq.cuda(), kk.cuda()), torch_ref.exact_block_mass(qq, kk))


# The matrix-core exact block-mass kernel at block sizes 16, 32 and 64 (16-bit inputs, head
# dim 128; smaller head dims are zero-padded to 128): q-blocks of KB rows inside 128-row
# items, key blocks of KB keys inside 128-key tiles, ragged ends on both sides, Nq != Nk.
@pytest.mark.parametrize("bs", [16, 32, 64])
@pytest.mark.parametrize("D,Nq,Nk,dtype", [(128, 1000, 1000, torch.bfloat16), (128, 333, 1111, torch.float16),
                                           (64, 520, 260, torch.bfloat16)])
def test_exact_mass_mfma_block_sizes(bs, D, Nq, Nk, dtype):
    q, k = _qkd(2, 3, 3, Nq, Nk, D, dtype, seed=bs + Nq, sinks=3)
    ours = ops.block_mass_scores(q.cuda(), k.cuda(), block_size=bs)
    ref = torch_ref.exact_block_mass(q, k, block_size=bs)
    assert ours.shape == ref.shape == (2, 3, math.ceil(Nq / bs), math.ceil(Nk / bs))
    _close(ours, ref)
    assert torch.allclose(ours.cpu().sum(-1), torch.ones(ref.shape[:-1]), atol=1e-5)


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
def test_exact_mass_mfma_rescale_and_persistent_loop(bs):
    # 96 heads x 9 items of 128 rows: more items than resident work-groups, so slots are
    # reused.  q = 0.5 + 0.1 N(0,1) and the first 128 keys all -10: those scores are about
    # -640, ~80 log2 units below the N(0,1) keys after them, so the first tile's maximum
    # (the rows' reference point) sends every row through the 2^64 rescale of its earlier
    # key-block sums on the second tile (moderate scores elsewhere keep fp32 summation-order
    # differences below the 1e-5 bar)
    g = torch.Generator().manual_seed(bs)
    q = 0.5 + 0.1 * torch.randn(1, 96, 1100, 128, generator=g)
    k = torch.randn(1, 96, 1500, 128, generator=g)
    k[:, :, :128] = -10.0
    qq, kk = q.bfloat16(), k.bfloat16()
    ours = ops.block_mass_scores(qq.cuda(), kk.cuda(), block_size=bs)
    ref = torch_ref.exact_block_mass(qq, kk, block_size=bs)
    _close(ours, ref)
    assert float(ours[..., : 128 // bs].sum(-1).max()) < 1e-20   # the first tile holds no mass


def test_exact_mass_closed_forms():
    # Q = 0: uniform softmax -> mass = |kb| / N (last block 120 of 32760 -> 120/N)
    N = 1016  # 7 full blocks + 120
    q = torch.zeros(1, 1, 256, 128, dtype=torch.bfloat16)
    k = torch.randn(1, 1, N, 128).to(torch.bfloat16)
    m = ops.block_mass_scores(q.cuda(), k.cuda()).cpu()
    want = torch.tensor([128.0] * 7 + [120.0]) / N
    assert torch.allclose(m[0, 0], want.expand(2, -1), rtol=1e-5, atol=0)
    # one dominant key: all the mass in its block
    k2 = torch.zeros(1, 1, N, 128)
    k2[0, 0, 300] = 50.0
    q2 = torch.ones(1, 1, 256, 128)
    m2 = ops.block_mass_scores(q2.cuda().bfloat16(), k2.cuda().bfloat16()).cpu()
    assert torch.allclose(m2[0, 0, :, 2], torch.ones(2), atol=1e-6)


def test_exact_mass_vs_fp64():
    q, k = _qk(2, 2, 700, 900, torch.bfloat16, seed=4, sinks=3)
    ours = ops.block_mass_scores(q.cuda(), k.cuda()).cpu().double()
    ref = torch_ref.exact_block_mass_fp64(q, k)
    assert ((ours - ref).abs() <= 2e-5 * ref.abs() + 1e-9).all()


@pytest.mark.slow
def test_exact_mass_wan_shape_one_head():
    # Wan config 2/3 shape per (b, h): N = 32760 (ragged 120), bf16 -> [256, 256]
    q, k = _qk(1, 1, 32760, 32760, torch.bfloat16, seed=5, sinks=16)
    ours = ops.block_mass_scores(q.cuda(), k.cuda()).cpu()
    assert ours.shape == (1, 1, 256, 256)
    assert torch.allclose(ours.sum(-1), torch.ones(1, 1, 256), atol=2e-5)
    rows = [0, 1, 97, 255]
    ref = torch_ref.exact_block_mass(q[:, :, [r * 128 + i for r in rows for i in range(128 if r < 255 else 120)]], k)
    # ref rows are the selected q-blocks in order
    _close(ours[:, :, rows], ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [False, True])
def test_max_pool_vs_closed_form(dtype, causal):
    q, k = _qk(1, 4, 1024, 1024, dtype, seed=7, sinks=2)
    sm = 1.0 / math.sqrt(128)
    ours = ops.max_pool_scores(q.cuda(), k.cuda(), sm, causal=causal).cpu()
    ref = torch_ref.max_pool_map(q, k, sm, causal=causal)
    assert ours.dtype == dtype
    _max_pool_close(ours, ref, q, k, sm, causal=causal)
    # the unrounded formula agrees up to the reference's own rounding of the log2-domain
    # block maxima to q.dtype (|R| ~ 40 -> bf16 ulp 0.25 -> up to 2^0.125 in the ratio)
    ex = torch_ref.max_pool_map(q, k, sm, causal=causal, exact=True)
    assert torch.allclose(ours.double(), ex, rtol=0.2, atol=1e-3)


def test_max_pool_persistent_loop_ragged():
    # 96 heads x 9 query blocks = 864 items: more than one item per resident work-group,
    # so the workspace slot of a group is reused; N = 1100 leaves a ragged last block.
    q, k = _qk(1, 96, 1100, 1100, torch.bfloat16, seed=12, sinks=3)
    sm = 1.0 / math.sqrt(128)
    for causal in (False, True):
        ours = ops.max_pool_scores(q.cuda(), k.cuda(), sm, causal=causal).cpu()
        ref = torch_ref.max_pool_map(q, k, sm, causal=causal)
        _max_pool_close(ours, ref, q, k, sm, causal=causal, what=f"causal={causal}")


@pytest.mark.parametrize("bs", [16, 32, 64])
def test_max_pool_small_blocks_persistent_loop_ragged(bs):
    # the matrix-core max-pool kernel at blocks 16-64: 96 heads x 9 items of 128 rows (more
    # than one item per resident work-group), N = 1100 (ragged last block), causal and not
    q, k = _qk(1, 96, 1100, 1100, torch.bfloat16, seed=40 + bs, sinks=3)
    sm = 1.0 / math.sqrt(128)
    for causal in (False, True):
        ours = ops.max_pool_scores(q.cuda(), k.cuda(), sm, block_size=bs, causal=causal).cpu()
        ref = torch_ref.max_pool_map(q, k, sm, block_size=bs, causal=causal)
        _max_pool_close(ours, ref, q, k, sm, bs, causal, what=f"bs={bs} causal={causal}")


def test_max_pool_many_key_blocks():
    # N = 40000 -> 313 key blocks per row (ragged 64); three query blocks are checked
    # against the closed form.
    q, k = _qk(1, 1, 40000, 40000, torch.bfloat16, seed=13, sinks=8)
    assert ops.max_pool_scores(q.cuda(), k.cuda(), 0.088).shape == (1, 1, 313, 313)
    sel = [0, 150, 312]
    for causal in (False, True):
        ours = ops.max_pool_scores(q.cuda(), k.cuda(), 0.088, causal=causal).cpu()
        ref = torch_ref.max_pool_map(q, k, 0.088, causal=causal, query_blocks=sel)
        rows = [r * 128 + i for r in sel for i in range(128) if r * 128 + i < 40000]
        max_pool_bar(ours[:, :, sel], ref, max_block_logit(q, k, 0.088, 128, causal, rows=rows),
                     what=f"causal={causal}", qk=(q, k, 0.088, 128, causal, sel))


def test_attn_with_pooling_api_and_gqa():
    from sinkattention.pooling_kernel import attn_with_pooling
    q, _ = _qk(1, 4, 512, 512, torch.bfloat16, seed=8)
    _, k = _qk(1, 2, 512, 512, torch.bfloat16, seed=9)
    o, po = attn_with_pooling(q.cuda(), k.cuda(), k.cuda(), False, 0.088, 128)
    assert o.shape == q.shape and not o.any()
    ref = torch_ref.max_pool_map(q, k, 0.088)
    _max_pool_close(po, ref, q, k, 0.088)


def _qkd(B, H, Hk, Nq, Nk, D, dtype, seed, sinks=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Nq, D, generator=g)
    k = torch.randn(B, Hk, Nk, D, generator=g)
    if sinks:
        k[:, :, :sinks] *= 6.0
    return q.to(dtype), k.to(dtype)


# Shapes off the block-128 / head-dim-128 MFMA kernels run on the generic kernels: block
# sizes that do not divide 128 or exceed it, head dims 16..256, ragged ends, Nq != Nk, fp32
# with more than 256 key blocks.
@pytest.mark.parametrize("D,bs,Nq,Nk,dtype", [
    (64, 64, 300, 300, torch.bfloat16), (128, 32, 260, 500, torch.bfloat16),
    (32, 96, 333, 250, torch.float16), (256, 16, 200, 130, torch.float32),
    (128, 256, 600, 600, torch.bfloat16), (80, 128, 300, 300, torch.bfloat16),
    (128, 128, 200, 33000, torch.float32), (16, 7, 50, 61, torch.bfloat16),
    (20, 64, 300, 280, torch.bfloat16), (20, 50, 300, 280, torch.float32)])
def test_exact_mass_generic_shapes(D, bs, Nq, Nk, dtype):
    q, k = _qkd(1, 2, 2, Nq, Nk, D, dtype, seed=D + bs, sinks=3)
    ours = ops.block_mass_scores(q.cuda(), k.cuda(), block_size=bs)
    ref = torch_ref.exact_block_mass(q, k, block_size=bs)
    assert ours.shape == ref.shape
    _close(ours, ref)
    assert torch.allclose(ours.cpu().sum(-1), torch.ones(ref.shape[:-1]), atol=1e-5)


@pytest.mark.parametrize("D,bs,N,dtype,causal", [
    (64, 64, 500, torch.bfloat16, False), (64, 32, 333, torch.float16, True),
    (256, 16, 200, torch.bfloat16, False), (32, 128, 400, torch.float32, False),
    (128, 64, 1000, torch.bfloat16, True), (16, 16, 100, torch.bfloat16, False)])
def test_max_pool_generic_shapes(D, bs, N, dtype, causal):
    q, k = _qkd(1, 4, 2, N, N, D, dtype, seed=D * 7 + bs, sinks=2)  # GQA: 4 query heads, 2 kv
    sm = 1.0 / math.sqrt(D)
    ours = ops.max_pool_scores(q.cuda(), k.cuda(), sm, block_size=bs, causal=causal).cpu()
    ref = torch_ref.max_pool_map(q, k, sm, block_size=bs, causal=causal)
    assert ours.dtype == dtype and ours.shape == ref.shape
    if dtype == torch.float32:
        assert torch.allclose(ours, ref, rtol=1e-5, atol=1e-12)
    else:
        _max_pool_close(ours, ref, q, k, sm, bs, causal, what=f"D={D} bs={bs}")


def test_attn_with_pooling_block_64_head_dim_64():
    from sinkattention.pooling_kernel import attn_with_pooling
    q, k = _qkd(2, 3, 3, 640, 640, 64, torch.bfloat16, seed=21)
    o, po = attn_with_pooling(q.cuda(), k.cuda(), k.cuda(), False, 0.125, 64)
    assert o.shape == q.shape and not o.any() and po.shape == (2, 3, 10, 10)
    _max_pool_close(po, torch_ref.max_pool_map(q, k, 0.125, block_size=64), q, k, 0.125, 64)


@pytest.mark.parametrize("bs,D", [(64, 64), (200, 128), (16, 32), (64, 20)])
def test_mean_mode_generic_block(bs, D):
    q, k = _qkd(1, 2, 2, 700, 500, D, torch.bfloat16, seed=bs)
    ours = ops.mean_pool_scores(q.cuda(), k.cuda(), block_size=bs).cpu()
    ref = torch_ref.mean_pool_scores(q, k, block_size=bs)
    assert torch.allclose(ours, ref, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mean_mode(dtype):
    q, k = _qk(2, 3, 1000, 700, dtype, seed=10)
    cfg = sa.SinkSparseConfig(pooling_mode="mean")
    ours = sa._compute_block_scores(q.cuda(), k.cuda(), k.cuda(), cfg).cpu()
    ref = torch_ref.mean_pool_scores(q, k)
    assert torch.allclose(ours, ref, rtol=1e-5, atol=1e-7)


def test_pooling_mode_dispatch():
    q, k = _qk(1, 2, 256, 256, torch.bfloat16, seed=11)
    qc, kc = q.cuda(), k.cuda()
    with pytest.raises(ValueError):
        sa._compute_block_scores(qc, kc, kc, sa.SinkSparseConfig(pooling_mode="bogus"))
    t = sa._compute_block_scores(qc, kc, kc, sa.SinkSparseConfig(pooling_mode="triton"))
    assert t.dtype == torch.float32 and t.shape == (1, 2, 2, 2)
