"""Fused QK-norm + rotary kernel against the fp32 oracle (RMSNorm, pair rotation) with the
reference's rounding points: the norm's output is a tensor of the input dtype (rounded
once), the rotation is computed in fp32 and rounded once.  Bound: one rounding step of
the dtype on each side, i.e. |ours - oracle| <= 2 ulp(|oracle|) (sum-of-squares order
and fused multiply-adds may move a value across a rounding boundary)."""
import pytest
import torch
import torch.nn as nn

from oracle import torch_ref
from sinkattn_amd import ops
from sinkattn_amd import wan_runtime as wr
from sinkattn_amd import zimage_runtime as zr

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -23}


def _expect(x, w, eps, re, im, heads_per_row, D, dtype):
    """(oracle output, per-element scale): the scale is |y0| + |y1| of the element's
    channel pair before the rotation (|y| without a rotation)."""
    y = torch_ref.rms_norm_rows(x, w, eps).to(dtype).float()
    if re is None:
        return y, y.abs()
    shp = y.shape
    yh = y.reshape(*shp[:-1], heads_per_row, D)
    out = torch_ref.rotate_pairs(yh, re, im)
    mag = (yh[..., 0::2].abs() + yh[..., 1::2].abs()).repeat_interleave(2, -1)
    return out.reshape(shp), mag.reshape(shp)


def _check(got, want_and_scale, dtype, what):
    """A normed value may round to the neighbouring dtype value (one ulp of |y|) when the
    two sides' fp32 sums straddle a rounding boundary; the rotation carries that into
    the output scaled by the pair's magnitude, and the output rounds once more."""
    want, scale = want_and_scale
    err = (got.float().cpu() - want).abs()
    bound = 2 * EPS[dtype] * scale + EPS[dtype] * want.abs() + 1e-6
    print(f"{what}: max err {err.max().item():.3e}", flush=True)
    assert bool((err <= bound).all()), what


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_wan_layout_vs_oracle(dtype):
    B, N, H, D = 2, 1000, 12, 128
    C = H * D
    g = torch.Generator(device=DEV).manual_seed(1)
    q = (torch.randn(B, N, C, device=DEV, generator=g) * 3).to(dtype)
    k = torch.randn(B, N, C, device=DEV, generator=g).to(dtype)
    wq, wk = torch.rand(C, device=DEV) + 0.5, torch.rand(C, device=DEV) + 0.5
    ang = torch.randn(N, D // 2, device=DEV)
    re, im = torch.cos(ang), torch.sin(ang)
    qo, ko = ops.qk_norm_rotary(q, k, wq, wk, 1e-6, 1e-5, D, re, im, rows_per_pos=1)
    reb, imb = re.cpu().view(1, N, 1, D // 2), im.cpu().view(1, N, 1, D // 2)
    _check(qo, _expect(q.cpu(), wq.cpu(), 1e-6, reb, imb, H, D, dtype), dtype, f"wan q {dtype}")
    _check(ko, _expect(k.cpu(), wk.cpu(), 1e-5, reb, imb, H, D, dtype), dtype, f"wan k {dtype}")
    # no rotation table: the norm alone
    qn, _ = ops.qk_norm_rotary(q, k, wq, wk, 1e-6, 1e-5, D)
    _check(qn, _expect(q.cpu(), wq.cpu(), 1e-6, None, None, H, D, dtype), dtype, f"norm only {dtype}")


# Rows of one head share their position's table row.  6 heads in bf16 take the row-walk
# kernel; 30 heads (Z-Image's), and fp32 rows of 4 lanes' worth, take the position-major one
# (a position's rows in steps of 64 / lanes-per-row, the table entries loaded once).
@pytest.mark.parametrize("H,dtype", [(6, torch.bfloat16), (30, torch.bfloat16), (30, torch.float16),
                                     (30, torch.float32), (9, torch.float32)])
def test_zimage_layout_per_batch_tables_vs_oracle(H, dtype):
    B, N, D = 2, 700, 128
    g = torch.Generator(device=DEV).manual_seed(2)
    q = torch.randn(B, N, H, D, device=DEV, generator=g).to(dtype)
    k = torch.randn(B, N, H, D, device=DEV, generator=g).to(dtype)
    wq, wk = torch.rand(D, device=DEV) + 0.5, torch.rand(D, device=DEV) + 0.5
    ang = torch.randn(B, N, D // 2, device=DEV)
    f = torch.polar(torch.ones_like(ang), ang)
    qo, ko = ops.qk_norm_rotary(q, k, wq, wk, 1e-5, 1e-5, D, f.real, f.imag, rows_per_pos=H)
    re, im = f.real.cpu()[:, :, None, None, :], f.imag.cpu()[:, :, None, None, :]
    _check(qo, _expect(q.cpu(), wq.cpu(), 1e-5, re, im, 1, D, dtype), dtype, f"zimage q H={H} {dtype}")
    _check(ko, _expect(k.cpu(), wk.cpu(), 1e-5, re, im, 1, D, dtype), dtype, f"zimage k H={H} {dtype}")


def test_errors():
    q = torch.randn(4, 96, device=DEV, dtype=torch.bfloat16)
    w = torch.ones(96, device=DEV)
    with pytest.raises(ValueError):  # head dim 12 is not a multiple of 8 elements
        ops.qk_norm_rotary(q, q, w, w, 1e-6, 1e-6, 12)
    with pytest.raises(ValueError):
        ops.qk_norm_rotary(q, q, torch.ones(95, device=DEV), w, 1e-6, 1e-6, 32)
    with pytest.raises(RuntimeError):
        ops.qk_norm_rotary(q.cpu(), q.cpu(), w, w, 1e-6, 1e-6, 32)


class _WanAttn(nn.Module):
    def __init__(self, C, heads):
        super().__init__()
        self.heads = heads
        self.to_q, self.to_k, self.to_v = nn.Linear(C, C), nn.Linear(C, C), nn.Linear(C, C)
        self.norm_q, self.norm_k = nn.RMSNorm(C, eps=1e-6), nn.RMSNorm(C, eps=1e-6)
        self.add_k_proj = None


@pytest.mark.parametrize("form", ["complex", "tuple"])
def test_wan_prepare_fused_equals_torch_path(form, monkeypatch):
    torch.manual_seed(3)
    H, D, N = 4, 128, 600
    attn = _WanAttn(H * D, H).to(DEV, torch.bfloat16)
    with torch.no_grad():
        attn.norm_q.weight.uniform_(0.5, 1.5)
        attn.norm_k.weight.uniform_(0.5, 1.5)
    x = torch.randn(2, N, H * D, device=DEV, dtype=torch.bfloat16)
    ang = torch.randn(N, D // 2, device=DEV)
    if form == "complex":
        freqs = torch.polar(torch.ones_like(ang), ang).view(1, 1, N, D // 2)
    else:
        freqs = (torch.cos(ang).repeat_interleave(2, -1).view(1, N, 1, D),
                 torch.sin(ang).repeat_interleave(2, -1).view(1, N, 1, D))
    assert wr._fused_qk_prep(attn, attn.to_q(x), attn.to_k(x), freqs) is not None
    qf, kf, vf, _ = wr._prepare_attention_tensors(attn, x, None, freqs)
    monkeypatch.setattr(wr, "FUSE_QK_PREP", False)
    qt, kt, vt, _ = wr._prepare_attention_tensors(attn, x, None, freqs)
    # the torch path rounds the norm's bf16 multiply by the weight differently (the
    # module multiplies in bf16): allow two rounding steps
    for a, b, name in ((qf, qt, "q"), (kf, kt, "k")):
        err = (a.float() - b.float()).abs()
        assert bool((err <= 4 * 2.0 ** -8 * b.float().abs() + 1e-3).all()), name
    assert torch.equal(vf, vt)
    assert qf.shape == (2, H, N, D) and qf.stride(2) == H * D  # [B, N, H, D] memory, no copy


def test_zimage_prepare_fused_equals_torch_path(monkeypatch):
    torch.manual_seed(4)
    H, D, N = 4, 128, 300

    class A(nn.Module):
        def __init__(self):
            super().__init__()
            self.heads = H
            self.to_q, self.to_k, self.to_v = (nn.Linear(H * D, H * D) for _ in range(3))
            self.norm_q, self.norm_k = nn.RMSNorm(D, eps=1e-5), nn.RMSNorm(D, eps=1e-5)

    attn = A().to(DEV, torch.bfloat16)
    x = torch.randn(2, N, H * D, device=DEV, dtype=torch.bfloat16)
    ang = torch.randn(2, N, D // 2, device=DEV)
    f = torch.polar(torch.ones_like(ang), ang)
    qf, kf, vf = zr.prepare_zimage_attention_tensors(attn, x, freqs_cis=f)
    monkeypatch.setattr(zr, "FUSE_QK_PREP", False)
    qt, kt, vt = zr.prepare_zimage_attention_tensors(attn, x, freqs_cis=f)
    for a, b in ((qf, qt), (kf, kt)):
        err = (a.float() - b.float()).abs()
        assert bool((err <= 4 * 2.0 ** -8 * b.float().abs() + 1e-3).all())
    assert torch.equal(vf, vt)
