"""Host logic of the Wan and Z-Image runtimes (CPU only): mask composition and caching,
the Z-Image block layout (suffix alignment, presence, slicing, forced-dense text),
config building, rotary arithmetic, installers; plus the oracle pins of the
compensation-branch helpers (K/V mean pooling, LSE mixing)."""
import math

import pytest
import torch
import torch.nn as nn

from oracle import torch_ref
from sinkattn_amd import wan_runtime as wr
from sinkattn_amd import zimage_runtime as zr
from sinkattn_amd.sparse_attention import SinkRuntimeState, SinkSparseConfig


# --- oracle pins: compensation helpers ------------------------------------------------------
def test_mean_pool_tokens_closed_forms():
    # a ramp 0..n-1 pooled by g has group means (g0 + g1) / 2; the ragged group repeats n-1
    n, g = 67, 10
    x = torch.arange(n, dtype=torch.float32).view(1, 1, n, 1)
    got = torch_ref.mean_pool_tokens(x, g)[0, 0, :, 0]
    want = [sum(range(s, s + g)) / g for s in range(0, 60, g)] + [(60 + 61 + 62 + 63 + 64 + 65 + 66 + 66 * 3) / g]
    assert torch.allclose(got, torch.tensor(want))
    # a constant sequence pools to itself; the prefix rows are untouched
    c = torch.full((2, 3, 95, 4), 1.5)
    c[:, :, :7] = torch.arange(7.0).view(1, 1, 7, 1)
    p = torch_ref.mean_pool_tokens(c, 30, prefix=7)
    assert p.shape == (2, 3, 7 + 3, 4)
    assert torch.equal(p[:, :, :7], c[:, :, :7]) and torch.allclose(p[:, :, 7:], torch.tensor(1.5))
    # gap 1 and a prefix covering everything are identities
    assert torch.equal(torch_ref.mean_pool_tokens(c, 1), c)
    assert torch.equal(torch_ref.mean_pool_tokens(c, 30, prefix=500), c)


def test_mix_equals_attention_over_union_with_multiplicity():
    """mix(attn over A, attn over D, gap) == attention over A plus every key of D counted
    `gap` times: the identity the adaptive mixing is built on."""
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 2, 9, 16, generator=g, dtype=torch.float64)
    ka, va = torch.randn(1, 2, 20, 16, generator=g, dtype=torch.float64), torch.randn(1, 2, 20, 16, generator=g, dtype=torch.float64)
    kd, vd = torch.randn(1, 2, 5, 16, generator=g, dtype=torch.float64), torch.randn(1, 2, 5, 16, generator=g, dtype=torch.float64)
    gap = 7

    def attn(k, v):
        s = q @ k.transpose(-1, -2) / 4.0
        return torch.softmax(s, -1) @ v, torch.logsumexp(s, -1, keepdim=True)

    oa, la = attn(ka, va)
    od, ld = attn(kd, vd)
    got = torch_ref.mix(oa, la, od, ld, gap)
    ou, _ = attn(torch.cat([ka] + [kd] * gap, 2), torch.cat([va] + [vd] * gap, 2))
    assert torch.allclose(got, ou, atol=1e-12)
    # gap 1, equal LSEs -> plain average
    assert torch.allclose(torch_ref.mix(oa, la, od, la, 1), (oa + od) / 2)


def test_host_pooling_helper_matches_oracle():
    from sinkattn_amd import sparse_attention as sa
    x = torch.randn(1, 2, 1000, 8)
    for gap, pre in [(30, 0), (30, 512), (4, 999), (30, 1000)]:
        a = sa._mean_pool_sequence_preserve_prefix(x, gap, prefix_tokens=pre)
        b = torch_ref.mean_pool_tokens(x, gap, pre)
        assert a.shape == b.shape and torch.allclose(a, b, atol=1e-6)


# --- Wan runtime -------------------------------------------------------------------------------
def _band(nq, nk, w):
    return torch.tensor([[abs(i - j) <= w for j in range(nk)] for i in range(nq)])


@pytest.mark.parametrize("band,text", [(0, 0), (1, 0), (2, 300)])
def test_wan_runtime_mask_composition(band, text):
    H, N = 3, 1000  # 8 blocks, ragged last block
    g = torch.Generator().manual_seed(band + text)
    sink = torch.rand(H, 8, 8, generator=g) < 0.2
    cfg = SinkSparseConfig(runtime_diagonal_band_width=band, text_length=text,
                           force_text_global_attention=text > 0)
    inner = wr.WanSinkSparseInnerAttention(0, sink, cfg)
    m = inner._get_runtime_mask(inner.sink_mask, "__base__", 2, H, N, N, torch.device("cpu"))
    want = sink.clone()
    req = torch_ref.required_mask(8, 8, 128, text, text > 0)
    if req is not None:
        want |= req
    if band:
        want |= _band(8, 8, band)
    assert m.shape == (2, H, 8, 8) and m.dtype == torch.bool
    assert torch.equal(m, want.unsqueeze(0).expand(2, -1, -1, -1))
    # cached: the same tensor object comes back (so the kernel plan is reused)
    assert inner._get_runtime_mask(inner.sink_mask, "__base__", 2, H, N, N, torch.device("cpu")) is m


def test_wan_runtime_mask_errors_and_plan():
    inner = wr.WanSinkSparseInnerAttention(0, torch.ones(2, 4, 4, dtype=torch.bool), SinkSparseConfig())
    with pytest.raises(ValueError, match="Re-calibrate"):
        inner._get_runtime_mask(inner.sink_mask, "__base__", 1, 2, 600, 512, torch.device("cpu"))
    assert inner._resolve_dynamic_plan() == ("pooled_kv", 30)
    inner.config = SinkSparseConfig(dynamic_mode="none", sample_gap=0)
    assert inner._resolve_dynamic_plan() == ("none", 1)
    inner.config = SinkSparseConfig(dynamic_mode="topk")
    with pytest.raises(ValueError, match="pooled_kv"):
        inner._resolve_dynamic_plan()
    full = inner._get_dynamic_mask(1, 2, 600, 40, torch.device("cpu"))
    assert full.shape == (1, 2, 5, 1) and bool(full.all())


def test_wan_rotary_forms_agree_with_complex_multiply():
    g = torch.Generator().manual_seed(3)
    B, H, N, D = 1, 2, 6, 8
    x = torch.randn(B, H, N, D, generator=g)
    ang = torch.randn(N, D // 2, generator=g, dtype=torch.float64)
    freqs = torch.polar(torch.ones_like(ang), ang)                  # [N, D/2] complex128
    want = torch.view_as_real(torch.view_as_complex(x.double().unflatten(-1, (-1, 2))) * freqs).flatten(-2)
    q, k = wr.apply_rotary_qk(x, x.clone(), freqs)
    assert torch.allclose(q.double(), want, atol=1e-6) and torch.equal(q, k)
    # Wan's tuple form: per-channel cos/sin tables [1, N, 1, D] with each angle repeated
    cos = torch.cos(ang).float().repeat_interleave(2, -1).view(1, N, 1, D)
    sin = torch.sin(ang).float().repeat_interleave(2, -1).view(1, N, 1, D)
    q2, _ = wr.apply_rotary_qk(x, x, (cos, sin))
    assert torch.allclose(q2.double(), want, atol=1e-6)
    with pytest.raises(TypeError):
        wr.apply_rotary_qk(x, x, torch.randn(N, D))
    assert wr.apply_rotary_qk(x, x, None)[0] is x


class _Proc:
    pass


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.processor = _Proc()

    def get_processor(self):
        return self.processor

    def set_processor(self, p):
        self.processor = p


def _package(tmp_path, layers, shape):
    pkg = {"version": 3, "config": {"dynamic_mode": "none", "block_size": 128},
           "sink_masks": {str(i): torch.ones(shape, dtype=torch.bool) for i in range(layers)},
           "mean_scores": {}, "std_scores": {}, "counts": {str(i): 1 for i in range(layers)}}
    path = tmp_path / "pkg.pt"
    torch.save(pkg, path)
    return str(path)


def test_wan_installers(tmp_path):
    model = nn.Module()
    model.blocks = nn.ModuleList([nn.Module() for _ in range(3)])
    for b in model.blocks:
        b.attn1 = _Attn()
    originals = [b.attn1.processor for b in model.blocks]
    info = wr.set_sink_sparse_attn_wanx(model, _package(tmp_path, 3, (2, 4, 4)), {"sample_gap": 10})
    assert info["num_layers"] == 3 and info["config"].sample_gap == 10 and info["config"].dynamic_mode == "none"
    for i, b in enumerate(model.blocks):
        assert isinstance(b.attn1.processor, wr.WanSinkSparseAttnProcessor2_0)
        assert isinstance(b.attn1.inner_attention, wr.WanSinkSparseInnerAttention)
        assert b.attn1.inner_attention.runtime_state is model._sink_runtime_state
        assert b.attn1.origin_processor is originals[i]
    model.blocks.append(nn.Module())
    model.blocks[3].attn1 = _Attn()
    with pytest.raises(KeyError):
        wr.set_sink_sparse_attn_wanx(model, _package(tmp_path, 3, (2, 4, 4)))
    cal = object()
    assert wr.set_sink_calibration_attn_wanx(model, cal) is cal
    assert all(isinstance(b.attn1.processor, wr.WanSinkCalibrationProcessor2_0) for b in model.blocks)
    assert model.blocks[0].attn1.origin_processor is originals[0]


# --- Z-Image layout ----------------------------------------------------------------------------
def _explicit_align(scores, ib, tb, T):
    """Four block copies, written out."""
    H = scores.size(0)
    out = torch.zeros(H, T, T)
    out[:, :ib, :ib] = scores[:, :ib, :ib]
    if tb:
        s = T - tb
        out[:, :ib, s:] = scores[:, :ib, ib:]
        out[:, s:, :ib] = scores[:, ib:, :ib]
        out[:, s:, s:] = scores[:, ib:, ib:]
    return out


@pytest.mark.parametrize("tb", [0, 1, 2, 4])
def test_zimage_alignment_and_presence(tb):
    ib, T, H = 5, 9, 3
    n = ib + tb
    scores = torch.rand(H, n, n)
    got = zr._align_scores_image_text_suffix(scores, image_blocks=ib, current_text_blocks=tb, total_blocks=T)
    assert torch.equal(got, _explicit_align(scores, ib, tb, T))
    pres = zr._alignment_presence_mask(num_heads=H, image_blocks=ib, current_text_blocks=tb, total_blocks=T,
                                       device=torch.device("cpu"))
    assert torch.equal(pres, _explicit_align(torch.ones(H, n, n), ib, tb, T))
    # slicing the aligned layout gives the call's map back
    sl = zr._slice_runtime_sink_mask(got > 0.5, image_blocks=ib, current_text_blocks=tb, total_blocks=T)
    assert torch.equal(sl, scores > 0.5)
    with pytest.raises(ValueError):
        zr._align_scores_image_text_suffix(torch.rand(H, n + 1, n + 1), image_blocks=ib, current_text_blocks=tb,
                                           total_blocks=T)
    with pytest.raises(ValueError):
        zr._slice_runtime_sink_mask(torch.zeros(H, T, T + 1, dtype=torch.bool), image_blocks=ib,
                                    current_text_blocks=tb, total_blocks=T)


def test_zimage_force_text_dense():
    m = torch.zeros(1, 2, 7, 7, dtype=torch.bool)
    f = zr._force_text_dense_runtime_mask(m, image_blocks=5, current_text_blocks=2)
    assert f is not m and not bool(m.any())
    assert bool(f[..., 5:, :].all()) and bool(f[..., :, 5:].all()) and not bool(f[..., :5, :5].any())
    assert zr._force_text_dense_runtime_mask(m, image_blocks=5, current_text_blocks=0) is m


def test_zimage_config_and_layout():
    cfg = zr.build_zimg_sink_config()
    assert (cfg.token_depth, cfg.dynamic_mode, cfg.runtime_diagonal_band_width) == (1, "none", 0)
    assert cfg.force_text_global_attention and cfg.text_length == 512 and cfg.dynamic_kernel == "auto"
    # package config over defaults, overrides over package; None never overrides
    cfg = zr.build_zimg_sink_config(package_config={"token_width": 128, "token_height": 128, "sample_gap": 8,
                                                    "force_text_global_attention": False},
                                    config_overrides={"sample_gap": None, "dynamic_mode": "pooled_kv",
                                                      "dynamic_kernel": " Dense "})
    assert cfg.sample_gap == 8 and cfg.dynamic_mode == "pooled_kv" and cfg.dynamic_kernel == "dense"
    assert cfg.force_text_global_attention
    # config 4: 128x128 tokens + 512 text -> 128 + 4 = 132 blocks
    assert zr._fixed_block_shape(cfg) == (16384, 128, 132)
    assert zr._fixed_block_shape(SinkSparseConfig(token_width=10, token_height=7, token_depth=1,
                                                  text_length=100)) == (96, 1, 2)
    with pytest.raises(ValueError):
        zr.build_zimg_sink_config(config_overrides={"dynamic_mode": "topk"})
    with pytest.raises(ValueError):
        zr.build_zimg_sink_config(config_overrides={"mixing_mode": "fixed"})
    assert zr.infer_zimg_token_layout(height=1024, width=768) == (48, 64, 1)
    assert zr.infer_zimg_token_layout(height=8, width=8) == (1, 1, 1)


def test_zimage_forced_dense_lists():
    cfg = SinkSparseConfig(force_dense_steps=[0, -1, -9], force_dense_layers=[2, -1])
    st = SinkRuntimeState()
    assert zr._resolve_forced_dense_step_list(cfg, None) == {0}
    st.reset_generation(total_steps=8)
    assert zr._resolve_forced_dense_step_list(cfg, st) == {0, 7}
    assert zr._resolve_forced_dense_layer_list(cfg) == {2}
    assert zr._resolve_forced_dense_layer_list(cfg, total_layers=30) == {2, 29}
    p = zr.ZImageStaticSinkProcessor(layer_idx=29, total_layers=30, sink_mask=torch.ones(2, 2, 2, dtype=torch.bool),
                                     config=SinkSparseConfig(token_width=8, token_height=8, token_depth=1,
                                                             text_length=64, force_dense_layers=[-1],
                                                             force_dense_steps=[1]),
                                     runtime_state=st)
    assert p._should_force_dense_current_layer()
    assert not p._should_force_dense_current_step()  # step -1 before the first layer-0 call
    st.enter_layer(0)
    st.enter_layer(0)
    assert p._should_force_dense_current_step()


def test_zimage_rotary_matches_complex_multiply():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 5, 3, 8, generator=g)
    f = torch.polar(torch.ones(2, 5, 4, dtype=torch.float64), torch.randn(2, 5, 4, generator=g, dtype=torch.float64))
    got = zr.apply_zimage_rotary_emb(x, f.to(torch.complex64))
    want = torch.view_as_real(torch.view_as_complex(x.double().unflatten(-1, (-1, 2))) * f.unsqueeze(2)).flatten(-2)
    assert torch.allclose(got.double(), want, atol=1e-6)


def test_zimage_installers(tmp_path):
    model = nn.Module()
    model.layers = nn.ModuleList([nn.Module() for _ in range(2)])
    for b in model.layers:
        b.attention = _Attn()
    path = _package(tmp_path, 2, (2, 132, 132))
    info = zr.set_sink_sparse_attn_zimage(model, path, {"token_width": 128, "token_height": 128})
    assert info["route"] == "zimg_static_only" and info["num_layers"] == 2
    p = model.layers[1].attention.processor
    assert isinstance(p, zr.ZImageStaticSinkProcessor) and p.total_blocks == 132 and p.total_layers == 2
    zr.reset_sink_runtime_state_zimage(model, num_inference_steps=9)
    assert model._sink_runtime_state.total_steps == 9
    # the calibrator takes every field of the config it is given (token_depth included)
    cal = zr.ZImageSinkMaskCalibrator(SinkSparseConfig(token_width=128, token_height=128, token_depth=1,
                                                       text_length=512))
    assert (cal.image_token_count, cal.image_blocks, cal.total_blocks, cal.max_text_tokens) == (16384, 128, 132, 512)
    zr.set_sink_calibration_attn_zimage(model, cal)
    assert isinstance(model.layers[0].attention.processor, zr.ZImageSinkCalibrationProcessor)
    assert model.layers[1].attention.processor.origin_processor is p


def test_zimage_calibrator_accumulation_math():
    """mean = sum/presence (presence clamped to 1), std from the second moment; checked
    on hand-built aligned maps without the GPU score kernel."""
    cal = zr.ZImageSinkMaskCalibrator(SinkSparseConfig(token_width=8, token_height=8, token_depth=1,
                                                       text_length=256))
    ib, T = cal.image_blocks, cal.total_blocks
    assert (ib, T) == (1, 3)
    a = torch.rand(2, 3, 3)
    b = torch.rand(2, 2, 2)
    for sc, tb in ((a, 2), (b, 1)):
        al = zr._align_scores_image_text_suffix(sc, image_blocks=ib, current_text_blocks=tb, total_blocks=T)
        pr = zr._alignment_presence_mask(num_heads=2, image_blocks=ib, current_text_blocks=tb, total_blocks=T,
                                         device=torch.device("cpu"))
        cal._accumulate(layer_idx=0, scores=al, presence=pr)
    pres = cal.score_presence_sums[0].clone()
    mean = cal.score_sums[0] / pres.clamp_min(1.0)
    # cell (0,0) seen twice, the text corner (2,2) twice, cell (1,1) only by the first call
    assert torch.equal(pres[0], torch.tensor([[2.0, 1, 2], [1, 1, 1], [2, 1, 2]]))
    assert torch.allclose(mean[:, 0, 0], (a[:, 0, 0] + b[:, 0, 0]) / 2)
    assert torch.allclose(mean[:, 1, 1], a[:, 1, 1])
    assert torch.allclose(mean[:, 2, 2], (a[:, 2, 2] + b[:, 1, 1]) / 2)
    assert cal.score_counts[0] == 2


# --- QK-norm / rotary: oracle pins and host-side dispatch ---------------------------------------
def test_rms_norm_and_rotation_oracle_pins():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(7, 64, generator=g)
    w = torch.rand(64, generator=g) + 0.5
    y = torch_ref.rms_norm_rows(x, w, 1e-6)
    # unit RMS after dividing out w; invariant to a positive scale of x (eps aside)
    assert torch.allclose(((y / w) ** 2).mean(-1), torch.ones(7), atol=1e-5)
    assert torch.allclose(torch_ref.rms_norm_rows(3.5 * x, w, 0.0), torch_ref.rms_norm_rows(x, w, 0.0), atol=1e-6)
    # constant row c: y = w * c / sqrt(c^2 + eps)
    c = torch.full((1, 64), 0.25)
    assert torch.allclose(torch_ref.rms_norm_rows(c, w, 1e-2), w * 0.25 / math.sqrt(0.0625 + 1e-2), atol=1e-7)
    # rotation: identity at angle 0, (a, b) -> (-b, a) at pi/2, pair norms kept, = complex product
    z = torch.randn(3, 5, 16, generator=g, dtype=torch.float64)
    assert torch.equal(torch_ref.rotate_pairs(z, torch.ones(8, dtype=torch.float64), torch.zeros(8, dtype=torch.float64)), z)
    r90 = torch_ref.rotate_pairs(z, torch.zeros(8, dtype=torch.float64), torch.ones(8, dtype=torch.float64))
    assert torch.equal(r90[..., 0::2], -z[..., 1::2]) and torch.equal(r90[..., 1::2], z[..., 0::2])
    ang = torch.randn(5, 8, generator=g, dtype=torch.float64)
    rot = torch_ref.rotate_pairs(z, torch.cos(ang), torch.sin(ang))
    norms = lambda t: t[..., 0::2] ** 2 + t[..., 1::2] ** 2
    assert torch.allclose(norms(rot), norms(z))
    cz = torch.view_as_complex(z.reshape(3, 5, 8, 2).contiguous()) * torch.polar(torch.ones_like(ang), ang)
    assert torch.allclose(rot, torch.view_as_real(cz).reshape(3, 5, 16))


def test_qk_prep_dispatch_helpers():
    n = nn.RMSNorm(128, eps=1e-6)
    w, eps = wr.rms_norm_params(n)
    assert w is n.weight and eps == 1e-6
    assert wr.rms_norm_params(nn.RMSNorm(128)) is None          # eps None: module path
    assert wr.rms_norm_params(nn.LayerNorm(128)) is None        # has a bias / is a LayerNorm
    assert wr.rms_norm_params(nn.RMSNorm(128, eps=1e-6, elementwise_affine=False)) is None
    assert wr.rms_norm_params(None) is None
    N, D = 6, 8
    ang = torch.randn(N, D // 2, dtype=torch.float64)
    c = torch.polar(torch.ones_like(ang), ang).to(torch.complex64)
    re, im = wr.rotary_tables_2d(c.view(1, 1, N, D // 2), N, D)
    assert torch.equal(re, c.real) and torch.equal(im, c.imag)
    cos = torch.cos(ang).float().repeat_interleave(2, -1).view(1, N, 1, D)
    sin = torch.sin(ang).float().repeat_interleave(2, -1).view(1, N, 1, D)
    re2, im2 = wr.rotary_tables_2d((cos, sin), N, D)
    assert torch.allclose(re2, c.real) and torch.allclose(im2, c.imag)
    assert wr.rotary_tables_2d(torch.randn(N, D), N, D) is None
