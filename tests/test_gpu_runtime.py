"""Wan and Z-Image runtimes end to end on the GPU kernels, against the fp32 oracle.

The oracle side follows the reference's precision where it rounds on purpose: the
pooled K/V of the compensation branch are bf16 tensors there and both LSEs are cast to
q.dtype (sparse_attention.py:776) before the mix, so the oracle rounds the same values
to bf16 at the same points and computes everything else in fp32.  Tolerances: the
attention output 2e-2 max-abs / 1e-3 mean-abs (the attention bar), also for the installed
processors' outputs, with and without the output projection; the unfused reference sequence
(and the fused kernel compared with it) within `_check_rounded_mix`'s bound, because a bf16 LSE
that rounds to the neighbouring value on one side shifts the mixing weight on that row."""
import math

import pytest
import torch
import torch.nn as nn

from oracle import torch_ref
from sinkattn_amd import wan_runtime as wr
from sinkattn_amd import zimage_runtime as zr
from sinkattn_amd.sparse_attention import SinkRuntimeState, SinkSparseConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16(x):
    return x.to(torch.bfloat16).float()


def _expected_wan(q, k, v, mask, cfg, round_lse=True, parts=False):
    """Oracle output of the Wan inner attention.  round_lse: the reference's sequence
    (branch outputs and LSEs rounded to bf16 before the mix); else the exact fp32 mix,
    which is what the fused kernel computes.  parts: also return the branch outputs
    and LSEs (for the rounding bound)."""
    sink_o, sink_l = torch_ref.dense_masked_attention(q, k, v, mask)
    if cfg.dynamic_mode == "none":
        return sink_o
    gap = max(int(cfg.sample_gap), 1)
    kd = _bf16(torch_ref.mean_pool_tokens(k, gap, max(int(cfg.text_length), 0)))
    vd = _bf16(torch_ref.mean_pool_tokens(v, gap, max(int(cfg.text_length), 0)))
    full = torch.ones(q.size(0), q.size(1), mask.size(2), -(-kd.size(2) // 128), dtype=torch.bool)
    dyn_o, dyn_l = torch_ref.dense_masked_attention(q, kd, vd, full)
    r = _bf16 if round_lse else (lambda x: x)
    out = torch_ref.mix(r(sink_o), r(sink_l).unsqueeze(-1), r(dyn_o), r(dyn_l).unsqueeze(-1), gap)
    return (out, sink_o, sink_l, dyn_o, dyn_l, gap) if parts else out


def _check(out, want, max_abs, mean_abs, what):
    err = (out.float().cpu() - want).abs()
    print(f"{what}: max {err.max().item():.3e} mean {err.mean().item():.3e}", flush=True)
    assert err.max().item() <= max_abs and err.mean().item() <= mean_abs, what


def _check_rounded_mix(out, want, so, sl, do, dl, gap, what):
    """Reference sequence vs the same sequence on the kernels: the two sides' LSEs differ
    slightly before they are rounded to bf16 (the kernel's row sums add the bf16 P
    values) and can round to neighbouring bf16 values, one ulp <= 2^-7 |lse| apart; that
    moves the mix weight a = sigmoid(lse_s - lse_d - ln gap) by at most a quarter of the
    difference.  Bound each element by 2e-2 plus that shift (with margin, and a few
    roundings of the mix steps) times |out_s - out_d|; mean-abs 2e-3."""
    err = (out.float().cpu() - want).abs()
    print(f"{what}: max {err.max().item():.3e} mean {err.mean().item():.3e}", flush=True)
    shift = (sl.abs() + dl.abs() + math.log(gap)) * 2.0 ** -8 + 4 * 2.0 ** -9
    # plus the bf16 roundings of both branch outputs and of the mix's products and sum
    # (a few ulps of |out_s| + |out_d|)
    bound = 2e-2 + shift.unsqueeze(-1) * (so - do).abs() + 4 * 2.0 ** -8 * (so.abs() + do.abs())
    assert err.mean().item() <= 2e-3 and bool((err <= bound).all()), what


@pytest.mark.parametrize("mode,text,band,fuse", [("none", 0, 0, True), ("pooled_kv", 0, 1, True),
                                                 ("pooled_kv", 300, 0, True), ("pooled_kv", 0, 1, False),
                                                 ("pooled_kv", 300, 0, False)])
def test_wan_inner_attention_vs_oracle(mode, text, band, fuse, monkeypatch):
    monkeypatch.setattr(wr, "FUSE_COMPENSATION", fuse)
    B, H, N, D = 1, 2, 2000, 128  # 16 blocks, last one 80 rows
    g = torch.Generator(device=DEV).manual_seed(11)
    q, k, v = (torch.randn(B, H, N, D, device=DEV, dtype=torch.bfloat16, generator=g) for _ in range(3))
    k[:, :, :4] *= 6.0
    sink = torch.rand(H, 16, 16, generator=torch.Generator().manual_seed(12)) < 0.25
    cfg = SinkSparseConfig(dynamic_mode=mode, text_length=text, force_text_global_attention=text > 0,
                           runtime_diagonal_band_width=band)
    state = SinkRuntimeState()
    inner = wr.WanSinkSparseInnerAttention(0, sink, cfg, runtime_state=state)
    out = inner(q, k, v)
    torch.cuda.synchronize()
    mask = inner._get_runtime_mask(inner.sink_mask, "__base__", B, H, N, N, q.device).cpu()
    qc, kc, vc = q.float().cpu(), k.float().cpu(), v.float().cpu()
    assert out.shape == (B, H, N, D) and out.dtype == torch.bfloat16
    if mode == "none":
        _check(out, _expected_wan(qc, kc, vc, mask, cfg), 2e-2, 1e-3, f"wan sparse {mode}")
    elif fuse:  # one kernel: the exact fp32 mix of the two branches
        _check(out, _expected_wan(qc, kc, vc, mask, cfg, round_lse=False), 2e-2, 1e-3,
               f"wan fused text={text} band={band}")
        # and against the reference's own sequence (both LSEs rounded to bf16 before the mix):
        # the fused kernel departs from it only by those roundings
        want, so, sl, do, dl, gap = _expected_wan(qc, kc, vc, mask, cfg, parts=True)
        _check_rounded_mix(out, want, so, sl, do, dl, gap, f"wan fused vs reference-rounded text={text}")
    else:
        want, so, sl, do, dl, gap = _expected_wan(qc, kc, vc, mask, cfg, parts=True)
        _check_rounded_mix(out, want, so, sl, do, dl, gap, f"wan unfused text={text} band={band}")
    ev = state.sparsity_events[-1]
    assert ev["dynamic_mode"] == mode and abs(ev["base_density"] - mask.float().mean().item()) < 1e-6
    # a second call reuses the cached kernel mask (same tensor -> cached plan)
    m1 = inner._get_runtime_mask(inner.sink_mask, "__base__", B, H, N, N, q.device)
    inner(q, k, v)
    assert inner._get_runtime_mask(inner.sink_mask, "__base__", B, H, N, N, q.device) is m1


class _WanAttn(nn.Module):
    def __init__(self, C, heads):
        super().__init__()
        self.heads = heads
        self.to_q, self.to_k, self.to_v = nn.Linear(C, C), nn.Linear(C, C), nn.Linear(C, C)
        self.norm_q, self.norm_k = nn.RMSNorm(C, eps=1e-6), nn.RMSNorm(C, eps=1e-6)
        self.add_k_proj = self.add_v_proj = self.norm_added_k = None
        self.to_out = nn.ModuleList([nn.Linear(C, C), nn.Dropout(0.0)])
        self.processor = None

    def get_processor(self):
        return self.processor

    def set_processor(self, p):
        self.processor = p

    def forward(self, hidden_states, rotary_emb=None):
        return self.processor(self, hidden_states, rotary_emb=rotary_emb)


def test_wan_processor_installed_model(tmp_path):
    torch.manual_seed(0)
    H, D, N = 2, 128, 1500
    model = nn.Module()
    model.blocks = nn.ModuleList([nn.Module() for _ in range(2)])
    for blk in model.blocks:
        blk.attn1 = _WanAttn(H * D, H)
    model = model.to(DEV, torch.bfloat16)
    nb = -(-N // 128)
    masks = {str(i): torch.rand(H, nb, nb, generator=torch.Generator().manual_seed(i)) < 0.3 for i in range(2)}
    path = tmp_path / "wan.pt"
    torch.save({"version": 3, "config": {"dynamic_mode": "pooled_kv", "sample_gap": 30},
                "sink_masks": masks, "mean_scores": {}, "std_scores": {}, "counts": {"0": 1, "1": 1}}, path)
    info = wr.set_sink_sparse_attn_wanx(model, str(path))
    assert info["num_layers"] == 2
    x = torch.randn(1, N, H * D, device=DEV, dtype=torch.bfloat16)
    ang = torch.randn(N, D // 2, device=DEV)
    freqs = torch.polar(torch.ones_like(ang), ang)
    for i, blk in enumerate(model.blocks):
        out = blk.attn1(x, rotary_emb=freqs)
        torch.cuda.synchronize()
        q, k, v, _ = wr._prepare_attention_tensors(blk.attn1, x, None, freqs)
        inner = blk.attn1.inner_attention
        mask = inner._get_runtime_mask(inner.sink_mask, "__base__", 1, H, N, N, q.device).cpu()
        o = _expected_wan(q.float().cpu(), k.float().cpu(), v.float().cpu(), mask, inner.config, round_lse=False)
        o_rows = o.transpose(1, 2).flatten(2, 3)
        want = blk.attn1.to_out[0](o_rows.to(DEV, torch.bfloat16)).float().cpu()
        # after the output projection
        _check(out, want, 2e-2, 1e-3, f"wan processor layer {i}")
        # the attention output itself, with the projection taken out: the attention bar
        proj = blk.attn1.to_out[0]
        blk.attn1.to_out[0] = nn.Identity()
        try:
            att = blk.attn1(x, rotary_emb=freqs)
            torch.cuda.synchronize()
        finally:
            blk.attn1.to_out[0] = proj
        _check(att, o_rows, 2e-2, 1e-3, f"wan processor layer {i} attention output")
    # layer 0 ran twice (with and without the projection): two steps, four events
    assert model._sink_runtime_state.current_step == 1 and len(model._sink_runtime_state.sparsity_events) == 4


class _ZAttn(nn.Module):
    def __init__(self, C, heads):
        super().__init__()
        self.heads = heads
        self.to_q, self.to_k, self.to_v = nn.Linear(C, C), nn.Linear(C, C), nn.Linear(C, C)
        self.norm_q, self.norm_k = nn.RMSNorm(C // heads, eps=1e-6), nn.RMSNorm(C // heads, eps=1e-6)
        self.to_out = nn.ModuleList([nn.Linear(C, C)])


def _zimage_expected(q, k, v, mask, cfg, image_tokens, n):
    """One sample's `[1, H, n, d]` output: sparse attention over the sliced, text-forced
    mask, then for pooled_kv the compensation on the image rows."""
    o, l = torch_ref.dense_masked_attention(q, k, v, mask)
    if cfg.dynamic_mode != "pooled_kv":
        return o
    gap = max(int(cfg.sample_gap), 1)
    il = image_tokens
    kd = torch.cat([_bf16(torch_ref.mean_pool_tokens(k[:, :, :il], gap)), k[:, :, il:n]], 2)
    vd = torch.cat([_bf16(torch_ref.mean_pool_tokens(v[:, :, :il], gap)), v[:, :, il:n]], 2)
    full = torch.ones(1, q.size(1), -(-il // 128), -(-kd.size(2) // 128), dtype=torch.bool)
    do, dl = torch_ref.dense_masked_attention(q[:, :, :il], kd, vd, full)
    out = o.clone()  # the processor runs the fused kernel: the exact fp32 mix
    out[:, :, :il] = torch_ref.mix(o[:, :, :il], l[:, :, :il].unsqueeze(-1), do, dl.unsqueeze(-1), gap)
    return out


@pytest.mark.parametrize("mode", ["none", "pooled_kv"])
def test_zimage_static_processor_vs_oracle(mode):
    torch.manual_seed(1)
    H, D = 2, 128
    # the image prefix is a whole number of 128-token blocks, as at every Z-Image resolution
    # the layout supports (the text suffix then starts on a block boundary)
    cfg = zr.build_zimg_sink_config(package_config={"token_width": 16, "token_height": 16, "text_length": 300,
                                                    "dynamic_mode": mode, "sample_gap": 8})
    image_tokens, ib, T = zr._fixed_block_shape(cfg)
    assert (image_tokens, ib, T) == (256, 2, 5)
    sink = torch.rand(H, T, T, generator=torch.Generator().manual_seed(2)) < 0.3
    # calibrated masks always hold the diagonal (no empty rows: an empty row has lse = +inf
    # and the LSE mix of the reference is NaN there, on both sides of this comparison)
    sink |= torch.eye(T, dtype=torch.bool)
    state = SinkRuntimeState()
    proc = zr.ZImageStaticSinkProcessor(layer_idx=0, total_layers=1, sink_mask=sink, config=cfg, runtime_state=state)
    attn = _ZAttn(H * D, H).to(DEV, torch.bfloat16)
    lens = [image_tokens + 300, image_tokens + 90, image_tokens]
    Nmax = max(lens)
    x = torch.randn(3, Nmax, H * D, device=DEV, dtype=torch.bfloat16)
    amask = torch.zeros(3, Nmax, dtype=torch.bool, device=DEV)
    for b, n in enumerate(lens):
        amask[b, :n] = True
    out = proc(attn, x, attention_mask=amask)
    torch.cuda.synchronize()
    # the attention output itself: the same call with the output projection taken out
    proj = attn.to_out[0]
    attn.to_out[0] = nn.Identity()
    att = proc(attn, x, attention_mask=amask)
    torch.cuda.synchronize()
    attn.to_out[0] = proj
    q, k, v = zr.prepare_zimage_attention_tensors(attn, x)
    for b, n in enumerate(lens):
        tb = -(-(n - image_tokens) // 128)
        m = zr._force_text_dense_runtime_mask(
            zr._slice_runtime_sink_mask(sink, image_blocks=ib, current_text_blocks=tb, total_blocks=T),
            image_blocks=ib, current_text_blocks=tb).unsqueeze(0)
        qs, ks, vs = (t[b:b + 1, :n].permute(0, 2, 1, 3).float().cpu() for t in (q, k, v))
        o = _zimage_expected(qs, ks, vs, m, cfg, image_tokens, n)
        o_rows = o.transpose(1, 2).flatten(2, 3)[0]
        want_rows = attn.to_out[0](o_rows.to(DEV, torch.bfloat16)).float().cpu()
        # after the output projection
        _check(out[b, :n], want_rows, 2e-2, 1e-3, f"zimage {mode} sample {b} len {n}")
        _check(att[b, :n], o_rows, 2e-2, 1e-3, f"zimage {mode} sample {b} attention output")
        pad = attn.to_out[0](torch.zeros(1, H * D, device=DEV, dtype=torch.bfloat16)).float().cpu()
        if n < Nmax:
            assert torch.allclose(out[b, n:].float().cpu(), pad.expand(Nmax - n, -1), atol=1e-2)
    assert len(state.sparsity_events) == 6
    # masks are cached per text-block count: 3 distinct lengths -> 3 entries
    assert len(proc._runtime_mask_cache) == 3


def test_zimage_calibrator_vs_oracle():
    torch.manual_seed(2)
    H, D = 2, 128
    cfg = SinkSparseConfig(token_width=16, token_height=16, token_depth=1, text_length=256, pooling_mode="exact",
                           offline_direct_coverage=0.85)
    cal = zr.ZImageSinkMaskCalibrator(cfg)
    cal_host = zr.ZImageSinkMaskCalibrator(cfg)
    cal_host.accumulate_on_host = True  # the reference's placement of the sums
    it, ib, T = cal.image_token_count, cal.image_blocks, cal.total_blocks
    assert (it, ib, T) == (256, 2, 4)
    samples = []
    for text in (256, 100, 0):
        n = it + text
        q, k = (torch.randn(1, H, n, D, device=DEV, dtype=torch.bfloat16) for _ in range(2))
        k[:, :, :3] *= 5.0
        cal.record(0, q, k, k, text_token_count=text)
        cal_host.record(0, q, k, k, text_token_count=text)
        samples.append((q, k, text))
    assert cal.score_sums[0].is_cuda and cal_host.score_sums[0].device.type == "cpu"
    pkg = cal.build_package()
    pkg_host = cal_host.build_package()
    for part in ("mean_scores", "std_scores", "sink_masks"):
        assert torch.equal(pkg[part]["0"].cpu(), pkg_host[part]["0"].cpu()), part
    # oracle: exact mass per sample, aligned by explicit block copies, mean over presence
    sums = torch.zeros(H, T, T)
    pres = torch.zeros(H, T, T)
    for q, k, text in samples:
        s = torch_ref.exact_block_mass(q.float().cpu(), k.float().cpu())[0]
        tb = -(-text // 128)
        idx = list(range(ib)) + list(range(T - tb, T))
        for a, ia in enumerate(idx):
            for c, ic in enumerate(idx):
                sums[:, ia, ic] += s[:, a, c]
                pres[:, ia, ic] += 1
    mean = sums / pres.clamp_min(1.0)
    got = pkg["mean_scores"]["0"]
    assert got.device.type == "cpu" and got.shape == (H, T, T)
    assert torch.allclose(got, mean, rtol=1e-5, atol=1e-7)
    assert pkg["counts"]["0"] == 3 and pkg["meta"]["total_blocks"] == T
    # the mask is the coverage builder applied to the package's own mean (bit-exact)
    want_mask = torch_ref.coverage_mask(got, coverage=0.85, keep_diagonal=True, block_size=128, text_length=256,
                                        force_text=True)
    assert torch.equal(pkg["sink_masks"]["0"].cpu(), want_mask)
