"""Host-side behaviour of the drop-in module (no GPU): config semantics, package I/O and
its error conventions, mask re-tiling, required masks, the compensation-branch torch
helpers, runtime statistics, and the rule that the kernel paths never fall back to CPU.
Expected values come from the oracle restatements or from closed forms."""
import math
import os

import pytest
import torch

from oracle import torch_ref
import sinkattention
from sinkattention import sparse_attention as sa


def test_alias_package_is_the_same_module():
    import sinkattn_amd.sparse_attention as impl
    assert sa is impl
    assert sinkattention.SinkSparseConfig is impl.SinkSparseConfig
    for name in ("_BLOCK_SPARSE_KERNEL_BLOCK_SIZE", "_adapt_block_mask_for_kernel", "_block_sparse_attn",
                 "_build_offline_required_mask", "_ceil_div", "_dense_short_attention",
                 "_dense_short_attention_with_lse", "_device_cache_key", "_make_full_block_mask",
                 "_mean_pool_sequence_preserve_prefix", "_mix_attention_outputs", "load_sink_mask_package",
                 "_build_direct_mean_coverage_mask", "_compute_block_scores", "_mean_pool_sequence",
                 "_compute_exact_block_mass_scores", "_get_block_sparse_runtime_tensors"):
        assert hasattr(sa, name), name
    from sinkattention.pooling_kernel import attn_with_pooling  # noqa: F401
    from sinkattention.timing import AttentionTimingCollector  # noqa: F401


def test_config_from_dict_and_merged():
    c = sa.SinkSparseConfig.from_dict({"block_size": 64, "bogus": 1, "text_length": 512})
    assert c.block_size == 64 and c.text_length == 512 and c.pooling_mode == "triton"
    assert sa.SinkSparseConfig.from_dict(None) == sa.SinkSparseConfig()
    m = c.merged({"block_size": None, "sample_gap": 7})
    assert m.block_size == 64 and m.sample_gap == 7 and c.sample_gap == 30
    assert c.merged(None) == c and c.merged(None) is not c
    assert sa.SinkSparseConfig().offline_direct_coverage == 0.85


def test_parse_helpers():
    assert sa.parse_int_list(None) is None and sa.parse_int_list("") is None
    assert sa.parse_int_list("1, 2,,3") == [1, 2, 3]
    assert sa.iter_seed_list((8888, "9999")) == [8888, 9999]
    assert sa._ceil_div(32760, 128) == 256
    assert sa._device_cache_key(torch.device("cpu")) == ("cpu", -1)


def _pkg(tmp_path, obj, name="p.pt"):
    p = tmp_path / name
    torch.save(obj, p)
    return str(p)


def test_load_sink_mask_package_errors(tmp_path):
    with pytest.raises(FileNotFoundError):
        sa.load_sink_mask_package(str(tmp_path / "missing.pt"))
    lfs = tmp_path / "lfs.pt"
    lfs.write_bytes(b"version https://git-lfs.github.com/spec/v1\noid sha256:abc\nsize 10\n")
    with pytest.raises(RuntimeError, match="LFS pointer"):
        sa.load_sink_mask_package(str(lfs))
    junk = tmp_path / "junk.pt"
    junk.write_bytes(b"not a pickle")
    with pytest.raises(RuntimeError, match="Failed to load"):
        sa.load_sink_mask_package(str(junk))
    with pytest.raises(TypeError):
        sa.load_sink_mask_package(_pkg(tmp_path, [1, 2]))
    with pytest.raises(ValueError, match="usable sink_masks"):
        sa.load_sink_mask_package(_pkg(tmp_path, {"sink_masks": {}}))
    with pytest.raises(TypeError):
        sa.load_sink_mask_package(_pkg(tmp_path, {"sink_masks": {"0": torch.ones(1)}, "config": [1]}))
    m = {"0": torch.ones(2, 3, 3, dtype=torch.bool)}
    for bad in ({"config": {"use_rearrange": True}}, {"step_groups": [1]}, {"step_group_sink_masks": {"a": 1}},
                {"config": {"use_step_mask_bank": True}}, {"config": {"step_group_names": ["a"]}}):
        obj = {"sink_masks": m, **bad}
        with pytest.raises(ValueError, match="Incompatible"):
            sa.load_sink_mask_package(_pkg(tmp_path, obj))
    good = sa.load_sink_mask_package(_pkg(tmp_path, {"sink_masks": m, "config": {"step_group_names": []},
                                                     "counts": {"0": 4}, "version": 3}))
    assert torch.equal(good["sink_masks"]["0"], m["0"])
    s = sa.summarize_sink_package({**good, "config": {"offline_direct_coverage": 0.85}})
    assert s == "sink_masks=1, mask_strategy=direct_mean_coverage, coverage=0.850, aggregated_calls=4, mean_density=1.0000"


def test_required_mask_matches_oracle():
    for tl, force in ((512, True), (300, True), (0, True), (512, False)):
        cfg = sa.SinkSparseConfig(text_length=tl, force_text_global_attention=force)
        got = sa._build_offline_required_mask(num_query_blocks=132, num_key_blocks=120, config=cfg,
                                              device=torch.device("cpu"))
        ref = torch_ref.required_mask(132, 120, 128, tl, force)
        assert (got is None) == (ref is None)
        if ref is not None:
            assert torch.equal(got, ref)


def test_adapt_block_mask_for_kernel():
    g = torch.Generator().manual_seed(0)
    m = torch.rand(2, 3, 9, 7, generator=g) < 0.4
    # identity with shape check
    assert torch.equal(sa._adapt_block_mask_for_kernel(m, source_block_size=128, seq_len_q=9 * 128 - 5,
                                                      seq_len_k=7 * 128), m)
    with pytest.raises(ValueError, match="wrong shape"):
        sa._adapt_block_mask_for_kernel(m, source_block_size=128, seq_len_q=100, seq_len_k=100)
    # finer source (64): OR over 2x2 groups
    fine = torch.rand(1, 1, 10, 9, generator=g) < 0.3
    out = sa._adapt_block_mask_for_kernel(fine, source_block_size=64, seq_len_q=640, seq_len_k=576)
    assert out.shape == (1, 1, 5, 5)
    for i in range(5):
        for j in range(5):
            assert bool(out[0, 0, i, j]) == bool(fine[0, 0, 2 * i:2 * i + 2, 2 * j:2 * j + 2].any())
    # coarser source (256): repeat, then crop
    coarse = torch.rand(1, 1, 3, 2, generator=g) < 0.5
    out = sa._adapt_block_mask_for_kernel(coarse, source_block_size=256, seq_len_q=600, seq_len_k=500)
    assert out.shape == (1, 1, 5, 4)
    assert torch.equal(out, coarse.repeat_interleave(2, -2).repeat_interleave(2, -1)[..., :5, :4])
    for bad in ((96, 128), (0, 128)):
        with pytest.raises(ValueError):
            sa._adapt_block_mask_for_kernel(m, source_block_size=bad[0], seq_len_q=128, seq_len_k=128,
                                            kernel_block_size=bad[1])
    assert sa._make_full_block_mask(2, 3, 300, 129, 128, torch.device("cpu")).shape == (2, 3, 3, 2)


def test_mean_pool_sequence_helpers():
    x = torch.arange(2 * 7 * 3, dtype=torch.float32).view(1, 2, 7, 3)
    p = sa._mean_pool_sequence(x, 3)
    padded = torch.cat([x, x[:, :, -1:].expand(1, 2, 2, 3)], dim=2)
    assert torch.equal(p, padded.view(1, 2, 3, 3, 3).mean(-2))
    assert sa._mean_pool_sequence(x, 1) is x
    q = sa._mean_pool_sequence_preserve_prefix(x, 3, prefix_tokens=2)
    assert torch.equal(q[:, :, :2], x[:, :, :2]) and q.shape[2] == 2 + 2
    assert sa._mean_pool_sequence_preserve_prefix(x, 3, prefix_tokens=99) is x
    assert torch.equal(sa._mean_pool_sequence_preserve_prefix(x, 3, prefix_tokens=0), p)


def test_dense_short_attention_with_lse_chunked(monkeypatch):
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 2, 37, 16, generator=g) for _ in range(3))
    out, lse = sa._dense_short_attention_with_lse(q, k, v)
    s = (q @ k.transpose(-1, -2)) / 4.0
    assert torch.allclose(lse[..., 0], torch.logsumexp(s, -1), atol=1e-5)
    assert torch.allclose(out, torch.softmax(s, -1) @ v, atol=1e-5)
    monkeypatch.setenv("SINK_DENSE_LSE_MAX_SCORE_ELEMENTS", "300")
    out2, lse2 = sa._dense_short_attention_with_lse(q, k, v)
    assert torch.allclose(out, out2, atol=1e-6) and torch.allclose(lse, lse2, atol=1e-6)


def test_mix_attention_outputs_matches_oracle_and_sigmoid():
    g = torch.Generator().manual_seed(2)
    so, do = torch.randn(1, 2, 5, 4, generator=g), torch.randn(1, 2, 5, 4, generator=g)
    sl, dl = torch.randn(1, 2, 5, 1, generator=g), torch.randn(1, 2, 5, 1, generator=g)
    cfg = sa.SinkSparseConfig()
    got = sa._mix_attention_outputs(so, sl, do, dl, cfg, dynamic_sample_gap=30)
    assert torch.allclose(got, torch_ref.mix(so, sl, do, dl, 30))
    alpha = torch.sigmoid(sl - dl - math.log(30))
    assert torch.allclose(got, so * alpha + do * (1 - alpha), atol=1e-6)
    with pytest.raises(ValueError):
        sa._mix_attention_outputs(so, None, do, dl, cfg)
    with pytest.raises(ValueError):
        sa._mix_attention_outputs(so, sl, do, dl, sa.SinkSparseConfig(mixing_mode="fixed"))


def test_runtime_state_statistics():
    st = sa.SinkRuntimeState()
    st.reset_generation(total_steps=2)
    for step in range(2):
        for layer in range(2):
            st.enter_layer(layer)
            m = torch.zeros(1, 2, 4, 4, dtype=torch.bool)
            m[..., : layer + 1] = True
            st.record_mask_stats(layer_idx=layer, sink_mask_tag="__base__", dynamic_mode="pooled_kv",
                                 dynamic_sample_gap=30, base_runtime_mask=m, dynamic_seq_len_k=10,
                                 total_seq_len_k=100)
    summ = st.summarize_sparsity()
    assert summ["num_events"] == 4 and summ["steps_recorded"] == [0, 1] and summ["layers_recorded"] == [0, 1]
    assert summ["by_layer"]["0"]["base_density_mean"] == pytest.approx(0.25)
    assert summ["overall"]["dense_equivalent_density_mean"] == pytest.approx(0.375 + 0.1)
    assert sa.SinkRuntimeState().summarize_sparsity()["num_events"] == 0
    assert st.summarize_timing()["enabled"] in (False, True)


def test_kernel_paths_do_not_fall_back_to_cpu():
    if torch.cuda.is_available():
        pytest.skip("checks the CPU-only behaviour")
    q = torch.randn(1, 1, 128, 128)
    with pytest.raises(RuntimeError, match="GPU"):
        sa._block_sparse_attn(q, q, q, torch.ones(1, 1, 1, 1, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="GPU"):
        sa._compute_block_scores(q, q, q, sa.SinkSparseConfig(pooling_mode="exact"))
    with pytest.raises(RuntimeError, match="GPU"):
        sa._build_direct_mean_coverage_mask(torch.rand(1, 2, 2), sa.SinkSparseConfig())
    with pytest.raises(ValueError, match="pooling_mode"):
        sa._compute_block_scores(q, q, q, sa.SinkSparseConfig(pooling_mode="nope"))
    with pytest.raises(ValueError, match="blocks_q"):
        sa._build_direct_mean_coverage_mask(torch.rand(2, 2), sa.SinkSparseConfig())


def test_calibrator_accumulation_math(monkeypatch):
    # record() with the score extraction stubbed: checks the batch mean, sums, std, counts
    seq = [torch.rand(2, 3, 4, 4) for _ in range(3)]
    it = iter(seq)
    monkeypatch.setattr(sa, "_compute_block_scores", lambda q, k, v, c: next(it))
    captured = {}
    monkeypatch.setattr(sa, "_build_direct_mean_coverage_masks",
                        lambda means, cfg: [captured.setdefault("m", torch_ref.coverage_mask(m)) for m in means])
    cal = sa.SinkMaskCalibrator(sa.SinkSparseConfig())
    for _ in range(3):
        cal.record(0, None, None, None)
    pkg = cal.build_package()
    means = torch.stack([x.mean(0) for x in seq])
    assert torch.allclose(pkg["mean_scores"]["0"], means.sum(0) / 3)
    assert torch.allclose(pkg["std_scores"]["0"], means.std(0, unbiased=False), atol=1e-5)
    assert pkg["counts"] == {"0": 3} and pkg["meta"] == {"route": "wanx_direct_coverage"}
    assert cal.current_step == 2  # every layer-0 record starts a step
    pkg2 = cal.build_package(include_scores=False)
    assert pkg2["mean_scores"] == {} and "0" in pkg2["sink_masks"]


def test_runtime_stats_density_is_cached_per_mask():
    st = sa.SinkRuntimeState()
    m = torch.zeros(1, 2, 4, 4, dtype=torch.bool)
    m[..., 0] = True
    calls = []
    real = sa.SinkRuntimeState._mask_density
    st._mask_density = lambda mask: calls.append(1) or real(mask)
    for _ in range(3):
        st.record_mask_stats(layer_idx=0, sink_mask_tag="t", dynamic_mode="none", dynamic_sample_gap=1,
                             base_runtime_mask=m)
    assert len(calls) == 1 and st.sparsity_events[-1]["base_density"] == 0.25
    m[..., 1] = True  # in-place change bumps the version: recomputed
    st.record_mask_stats(layer_idx=0, sink_mask_tag="t", dynamic_mode="none", dynamic_sample_gap=1,
                         base_runtime_mask=m)
    assert len(calls) == 2 and st.sparsity_events[-1]["combined_density"] == 0.5


def test_bench_refuses_more_than_one_gpu():
    # one GPU only: --gpus N > 1 exits with status 2 and a JSON error line (before any GPU
    # or torch work)
    import json
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "4"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"] and "--gpus 4" in msg["error"]
