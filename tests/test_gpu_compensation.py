"""Compensation-branch kernels on the GPU: token mean pooling, the LSE mix with the
reference's rounding, and the block-sparse forward fused with the compensation tiles.

Oracles: `torch_ref.mean_pool_tokens` (fp32), `torch_ref.mix` (evaluated in fp32 for the
math and on bf16 GPU tensors for the reference's exact op sequence), and
`torch_ref.dense_masked_attention` for both attention branches.  Tolerances: pooling
within one rounding of the dtype; the mix bit-exact with the reference's op sequence
for bf16/f16 (one-ulp differences allowed on at most 1e-4 of the elements, for `exp`
implementations that differ in the last fp32 bit), within 1e-5 relative for fp32; the fused
attention 2e-2 max-abs / 1e-3 mean-abs against the fp32 union attention, its fp32 lse within
4e-3 + 1e-5|lse| (row sums of the bf16 P values, log(1 + 2^-8) = 3.9e-3 at most); against the reference's unfused sequence (whose LSEs
are rounded to bf16 before the mix) 2e-3 mean-abs and, per element, 2e-2 plus the
largest shift that the reference's bf16 roundings of the LSEs and mix steps can cause."""
import math

import pytest
import torch

from oracle import torch_ref
from sinkattn_amd import ops
from sinkattn_amd import sparse_attention as sa

pytestmark = pytest.mark.gpu
DEV = "cuda"
ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -23}


def _layout(x, bshd):
    """x [B,H,N,D] as-is, or the same values in [B,N,H,D] memory viewed as [B,H,N,D]."""
    return x.transpose(1, 2).contiguous().transpose(1, 2) if bshd else x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("N,gap,prefix,D,bshd", [
    (32760, 30, 0, 128, True),     # Wan config 2: 1092 pooled rows, ragged last group (0 rows short)
    (2000, 30, 0, 128, False),     # 67 groups, the last one 20 rows short
    (1000, 7, 17, 64, True),       # kept prefix
    (300, 30, 300, 128, False),    # prefix covers everything -> copy
    (129, 1, 0, 128, False),       # gap 1 -> copy
])
def test_mean_pool_tokens_vs_oracle(dtype, N, gap, prefix, D, bshd):
    print(f"mean_pool_tokens dtype={dtype} N={N} gap={gap} prefix={prefix} D={D} bshd={bshd}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(N + gap)
    x = _layout(torch.randn(2, 3, N, D, device=DEV, generator=g).to(dtype), bshd)
    got = ops.mean_pool_tokens(x, gap, prefix, like=x)
    want = torch_ref.mean_pool_tokens(x, gap, prefix)
    assert got.shape == want.shape and got.dtype == dtype
    if bshd:
        assert got.stride(2) == x.stride(2)  # like=x keeps the row stride
    err = (got.float().cpu() - want).abs()
    bound = ULP[dtype] * want.abs() + 1e-6
    assert bool((err <= bound).all()), f"max err {err.max().item()}"
    if gap == 1 or prefix >= N:
        assert torch.equal(got.cpu(), x.cpu())
    # the reference's own torch ops on this GPU: equal, or one rounding step apart where the
    # two fp32 sums (different order) straddle a rounding boundary of the dtype
    # (16-bit only: in fp32 a different summation order shows in the last bit)
    ref = sa._pad_to_multiple(x[:, :, prefix:], gap) if gap > 1 and prefix < N and dtype != torch.float32 else None
    if ref is not None:
        b, h, n, d = ref.shape
        ref = torch.cat([x[:, :, :prefix], ref.reshape(b, h, n // gap, gap, d).mean(dim=-2)], 2)
        neq = got != ref
        diff = neq.float().mean().item()
        assert diff <= 1e-2, f"{diff:.2e} of the elements differ from torch's mean"
        if diff:  # and those by one rounding step at most
            step = ULP[dtype] * ref.float().abs()[neq] * 2
            assert bool(((got.float() - ref.float()).abs()[neq] <= step + 1e-6).all())


def test_mean_pool_tokens_errors():
    x = torch.randn(1, 2, 64, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.mean_pool_tokens(x, 0)
    with pytest.raises(RuntimeError):
        ops.mean_pool_tokens(x.cpu(), 30)
    with pytest.raises(ValueError):  # 24-element rows are not a power-of-two number of chunks
        ops.mean_pool_tokens(torch.randn(1, 2, 64, 24, device=DEV, dtype=torch.bfloat16), 4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_lse_mix_matches_reference_ops(dtype):
    print(f"lse_mix dtype={dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(7)
    B, H, N, D = 2, 3, 1000, 128
    so = _layout(torch.randn(B, H, N, D, device=DEV, generator=g).to(dtype), True)
    do = torch.randn(B, H, N, D, device=DEV, generator=g).to(dtype)
    ls = (torch.randn(B, H, N, 1, device=DEV, generator=g) * 3 + 8).to(dtype)
    ld = (torch.randn(B, H, N, 1, device=DEV, generator=g) * 3 + 5).to(dtype)
    for gap in (30, 1, 7):
        cfg = sa.SinkSparseConfig(sample_gap=gap)
        got = sa._mix_attention_outputs(so, ls, do, ld, cfg)
        ref = torch_ref.mix(so, ls, do, ld, gap)  # the reference's ops on dtype tensors
        assert got.dtype == dtype and got.shape == (B, H, N, D)
        if dtype == torch.float32:
            # no rounding to a coarse dtype hides last-bit differences of exp/log between
            # the host (log_gap) and device libraries; such a shift of the mixing weight
            # moves the result by a few fp32 ulps of |sink| + |dyn|
            bound = 1e-5 * (so.abs() + do.abs()) + 1e-7
            assert bool(((got - ref).abs() <= bound).all())
            continue
        neq = got != ref
        frac = neq.float().mean().item()
        assert frac <= 1e-4, f"gap {gap}: {frac:.2e} differ"
        if frac:
            rel = ((got.float() - ref.float()).abs() / ref.float().abs().clamp_min(1e-30))[neq]
            assert rel.max().item() <= 2 * ULP[dtype]
        # and the fp32 math within the dtype's rounding of the inputs and the result
        m32 = torch_ref.mix(so.float(), ls.float(), do.float(), ld.float(), gap)
        bound = 8 * ULP[dtype] * (so.float().abs() + do.float().abs() + 1)
        assert bool(((got.float() - m32).abs() <= bound).all())


def _case(B, H, N, D, density, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q, k, v = (_layout(torch.randn(B, H, N, D, device=DEV, generator=g).to(dtype), True) for _ in range(3))
    k[:, :, :4] *= 6.0
    nb = -(-N // 128)
    m = torch.rand(B, H, nb, nb, generator=torch.Generator().manual_seed(seed)) < density
    m |= torch.eye(nb, dtype=torch.bool)
    return q, k, v, m


def _union_oracle(q, k, v, mask, kd, vd, gap, comp_rows):
    """fp32: sparse attention, attention over the pooled keys, and their exact mix on
    rows < comp_rows (the union attention with the pooled keys counted gap times)."""
    qc, kc, vc = (t.float().cpu() for t in (q, k, v))
    so, sl = torch_ref.dense_masked_attention(qc, kc, vc, mask)
    full = torch.ones(q.size(0), q.size(1), -(-comp_rows // 128), -(-kd.size(2) // 128), dtype=torch.bool)
    do, dl = torch_ref.dense_masked_attention(qc[:, :, :comp_rows], kd.float().cpu(), vd.float().cpu(), full)
    out, lse = so.clone(), sl.clone()
    out[:, :, :comp_rows] = torch_ref.mix(so[:, :, :comp_rows], sl[:, :, :comp_rows, None], do, dl[..., None], gap)
    lse[:, :, :comp_rows] = torch.logaddexp(sl[:, :, :comp_rows], dl + math.log(gap))
    return out, lse


@pytest.mark.parametrize("N,gap,prefix,comp_rows,seed", [
    (2000, 30, 0, None, 1),     # Wan-like, ragged last block and ragged pooled tile
    (2000, 30, 300, None, 2),   # kept text prefix in the pooled keys
    (556, 8, 0, 256, 3),        # Z-Image-like: only the first two q-blocks compensated
    (4096, 30, 0, None, 4),
])
def test_fused_compensation_vs_oracle(N, gap, prefix, comp_rows, seed):
    print(f"fused comp N={N} gap={gap} prefix={prefix} comp_rows={comp_rows}", flush=True)
    B, H, D = 1, 2, 128
    q, k, v, m = _case(B, H, N, D, 0.2, seed)
    kd = ops.mean_pool_tokens(k, gap, prefix, like=k)
    vd = ops.mean_pool_tokens(v, gap, prefix, like=v)
    plan = ops.block_sparse_plan(m.to(DEV))
    out, lse = ops.block_sparse_attention_comp(q, k, v, plan, kd, vd, gap, comp_rows=comp_rows, return_lse=True)
    torch.cuda.synchronize()
    cr = N if comp_rows is None else comp_rows
    want, want_lse = _union_oracle(q, k, v, m, kd, vd, gap, cr)
    err = (out.float().cpu() - want).abs()
    print(f"  vs fp32 union: max {err.max().item():.3e} mean {err.mean().item():.3e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 1e-3
    # the kernel's row sums add the bf16 P values it multiplies V with (each within 2^-8
    # relative of the fp32 value), so the lse is within log(1 + 2^-8) = 3.9e-3 of the fp32 one
    lerr = (lse.cpu() - want_lse).abs()
    assert (lerr <= 4e-3 + 1e-5 * want_lse.abs()).all(), lerr.max().item()
    # against the reference's unfused sequence (bf16 LSEs into the reference-rounded mix)
    so, sl = sa._block_sparse_attn(q, k, v, m.to(DEV), return_lse=True)
    full = torch.ones(B, H, -(-cr // 128), -(-kd.size(2) // 128), dtype=torch.bool, device=DEV)
    do, dl = sa._block_sparse_attn(q[:, :, :cr], kd, vd, full, return_lse=True)
    mixed = sa._mix_attention_outputs(so[:, :, :cr], sl[:, :, :cr], do, dl, sa.SinkSparseConfig(sample_gap=gap))
    ref = so.clone()
    ref[:, :, :cr] = mixed
    err2 = (out.float() - ref.float()).abs()
    print(f"  vs unfused:    max {err2.max().item():.3e} mean {err2.mean().item():.3e}", flush=True)
    assert err2.mean().item() <= 2e-3
    # The reference rounds both LSEs (and every mix step) to bf16: a relative error u =
    # 2^-9 on each LSE moves the weight a by at most a(1-a)(|lse_s| + |lse_d| + ln gap)u
    # <= (|lse_s| + |lse_d| + ln gap)u / 4, and the mix steps add a few u.  Bound the
    # difference per element by that weight shift times |out_s - out_d| plus the
    # roundings of the outputs themselves (and the sparse kernels' own 2e-2 bar).
    u = 2.0 ** -9
    so_c, do_c = so[:, :, :cr].float(), do.float()
    shift = ((sl[:, :, :cr].float().abs() + dl.float().abs() + math.log(gap)) / 4 + 4) * u
    bound = torch.full_like(err2, 2e-2)
    bound[:, :, :cr] += shift * (so_c - do_c).abs() + 8 * u * (so_c.abs() + do_c.abs())
    assert bool((err2 <= bound).all()), f"max excess {(err2 - bound).max().item():.3e}"
    if cr < N:  # rows past comp_rows are the plain sparse result
        assert torch.equal(out[:, :, cr:], so[:, :, cr:])


def test_fused_compensation_argument_checks():
    q, k, v, m = _case(1, 2, 512, 128, 0.5, 9)
    plan = ops.block_sparse_plan(m.to(DEV))
    kd = ops.mean_pool_tokens(k, 30, like=k)
    vd = ops.mean_pool_tokens(v, 30, like=v)
    with pytest.raises(ValueError, match="row strides"):
        ops.block_sparse_attention_comp(q, k, v, plan, kd.contiguous(), vd, 30)
    with pytest.raises(ValueError, match="comp_rows"):
        ops.block_sparse_attention_comp(q, k, v, plan, kd, vd, 30, comp_rows=100)
    with pytest.raises(TypeError):
        ops.block_sparse_attention_comp(q.float(), k.float(), v.float(), plan, kd.float(), vd.float(), 30)
    # gap 1 and comp_rows 0 are ordinary cases: weight 1 / no compensated rows
    o0, _ = ops.block_sparse_attention_comp(q, k, v, plan, kd, vd, 30, comp_rows=0)
    o1, _ = ops.block_sparse_attention(q, k, v, plan, return_lse=False)
    assert torch.equal(o0, o1)
