"""GPU coverage-mask kernel: bit-exact against the reference semantics on CPU torch
(oracle/torch_ref.coverage_mask, the same torch calls as sparse_attention.py:268-376,
run on this machine's CPU) and against the C restatement (oracle/coverage_ref.c).
The per-row index lists and counts must describe the same mask.
"""
import zlib

import numpy as np
import pytest
import torch

from oracle import torch_ref
from sinkattn_amd import ops
from sinkattn_amd import sparse_attention as sa

pytestmark = pytest.mark.gpu


def _scores(H, nq, nk, kind, seed):
    rng = np.random.default_rng(seed)
    if kind == "dirichlet":
        x = rng.gamma(0.3, size=(H * nq, nk))
    elif kind == "ties":
        x = rng.integers(0, 5, size=(H * nq, nk)) / 7.0
    elif kind == "sinky":  # exact-mass-like rows: a few large blocks, long small tail
        x = rng.gamma(0.05, size=(H * nq, nk)) + 1e-4 * rng.random((H * nq, nk))
        x[:, 0] += 2.0
    elif kind == "uniform":
        x = np.ones((H * nq, nk))
    else:
        raise ValueError(kind)
    s = torch.from_numpy(x.astype(np.float32)).view(H, nq, nk)
    return s / s.sum(-1, keepdim=True).clamp_min(1e-30)


def _check_lists(mask, counts, idx):
    m = mask.cpu()
    c = counts.cpu()
    i = idx.cpu()
    assert torch.equal(c, m.sum(-1).to(torch.int32))
    H, nq, nk = m.shape
    for h in range(H):
        for q in range(0, nq, max(1, nq // 16)):
            want = torch.nonzero(m[h, q]).flatten().to(torch.int32)
            assert torch.equal(i[h, q, : want.numel()], want)


CONFIGS = [
    ("c1", (12, 32, 32), {}),
    ("c2", (12, 256, 256), {}),
    ("c4", (30, 132, 132), dict(text_length=512, force_text=True)),
    ("c4_video", (30, 132, 132), dict(text_length=512, force_text=True, mode="video_residual")),
    ("nodiag", (4, 40, 17), dict(keep_diagonal=False)),
    ("wide_rows", (2, 8, 600), {}),
    ("short_rows", (3, 9, 5), dict(coverage=0.5)),
    ("mid_rows", (2, 7, 300), {}),  # one kernel instance per power-of-two row capacity
    ("rows_1024", (1, 4, 1024), {}),
    ("video_long", (2, 10, 700), dict(text_length=512, force_text=True, mode="video_residual")),
    ("long_rows", (2, 6, 2000), {}),
    ("max_rows", (1, 3, 4096), {}),
]


@pytest.mark.parametrize("name,shape,kw", CONFIGS, ids=[c[0] for c in CONFIGS])
@pytest.mark.parametrize("kind", ["dirichlet", "ties", "sinky", "uniform"])
def test_mask_bit_exact(oracle_lib, name, shape, kw, kind):
    s = _scores(*shape, kind, seed=zlib.crc32(f"{name}/{kind}".encode()) % 1000)
    ref = torch_ref.coverage_mask(s, **kw)
    cfg = sa.SinkSparseConfig(
        offline_direct_coverage=kw.get("coverage", 0.85),
        keep_diagonal=kw.get("keep_diagonal", True),
        text_length=kw.get("text_length", 0),
        force_text_global_attention=kw.get("force_text", False),
        offline_text_video_coverage_mode=kw.get("mode", "joint"),
    )
    ours_cpu_in = sa._build_direct_mean_coverage_mask(s, cfg)  # CPU tensor in, like the reference
    assert ours_cpu_in.device.type == "cpu" and ours_cpu_in.dtype == torch.bool
    assert torch.equal(ours_cpu_in, ref)
    # direct kernel call with lists
    rq = rk = 0
    if kw.get("force_text"):
        tb = -(-kw["text_length"] // 128)
        rq, rk = min(tb, shape[1]), min(tb, shape[2])
    vt = min(-(-kw["text_length"] // 128), shape[1], shape[2]) if kw.get("mode") == "video_residual" else None
    mask, counts, idx = ops.coverage_mask(s.cuda(), kw.get("coverage", 0.85), kw.get("keep_diagonal", True),
                                          rq, rk, vt, want_lists=True)
    assert torch.equal(mask.cpu(), ref)
    _check_lists(mask, counts, idx)


def test_empty_row_fallback_quirk_on_gpu(oracle_lib):
    # an all-zero row without diagonal empties -> every row's top-1 bit is overwritten
    nk = 16
    rows = np.zeros((3, nk), np.float32)
    rows[0, 5] = 0.9
    rows[0, :5] = 0.02
    rows[1, :] = 1.0 / nk  # tie at the top: top-1 comes from the exact std::sort order
    s = torch.from_numpy(rows).view(1, 3, nk)
    ref = torch_ref.coverage_mask(s, keep_diagonal=False)
    cfg = sa.SinkSparseConfig(keep_diagonal=False)
    assert torch.equal(sa._build_direct_mean_coverage_mask(s.cuda(), cfg).cpu(), ref)
    assert torch.equal(torch.from_numpy(oracle_lib.coverage_mask(s.numpy(), 0.85, False)), ref)


@pytest.mark.parametrize("nk,force_text", [(300, False), (700, True)])
def test_empty_row_fallback_many_rows(oracle_lib, nk, force_text):
    # zero rows without the diagonal come out empty, so every row's top-1 bit is rewritten:
    # unique maxima, ties at the top, and required text blocks (-inf candidates) included
    rng = np.random.default_rng(nk)
    x = rng.gamma(0.3, size=(2 * 24, nk)).astype(np.float32)
    x[5] = 0.0
    x[30] = 0.0
    x[7, :3] = x[7].max() + 1.0  # tie at the top
    s = torch.from_numpy(x).view(2, 24, nk)
    kw = dict(keep_diagonal=False, text_length=256 if force_text else 0, force_text=force_text)
    ref = torch_ref.coverage_mask(s, **kw)
    rq = rk = 2 if force_text else 0
    got, counts, idx = ops.coverage_mask(s.cuda(), 0.85, False, rq, rk, None, want_lists=True)
    assert torch.equal(got.cpu(), ref)
    _check_lists(got, counts, idx)
    if not force_text:
        assert np.array_equal(oracle_lib.coverage_mask(s.numpy(), 0.85, False), ref.numpy())


def test_many_tie_rows_exact_permutation(oracle_lib):
    # small-integer scores: ties straddle the cut in most rows
    rng = np.random.default_rng(0)
    for nk in (32, 132, 256):
        x = rng.integers(1, 4, size=(8 * 64, nk)).astype(np.float32)
        s = torch.from_numpy(x).view(8, 64, nk)
        ref = torch_ref.coverage_mask(s)
        got = ops.coverage_mask(s.cuda(), 0.85, True).cpu()
        assert torch.equal(got, ref), nk
        assert np.array_equal(oracle_lib.coverage_mask(s.numpy()), ref.numpy())


def test_calibrator_end_to_end_matches_reference_math():
    # record() twice on small Wan-like layers, then build the package
    torch.manual_seed(0)
    cfg = sa.SinkSparseConfig(pooling_mode="exact")
    cal = sa.SinkMaskCalibrator(cfg)
    for step in range(2):
        for layer in range(2):
            q = torch.randn(2, 3, 640, 128, device="cuda", dtype=torch.bfloat16)
            k = torch.randn(2, 3, 640, 128, device="cuda", dtype=torch.bfloat16)
            cal.record(layer, q, k, k)
    pkg = cal.build_package()
    assert pkg["version"] == 3 and set(pkg["sink_masks"]) == {"0", "1"}
    for key, mean in pkg["mean_scores"].items():
        assert mean.device.type == "cpu"
        assert torch.equal(pkg["sink_masks"][key], torch_ref.coverage_mask(mean))
        assert pkg["counts"][key] == 2


def test_calibrator_device_accumulation_is_bit_identical():
    """Sums stay on the GPU (no per-call host copy) and give the same bits as the
    reference's host accumulation of the same per-call batch means."""
    torch.manual_seed(1)
    cfg = sa.SinkSparseConfig(pooling_mode="exact")
    cal = sa.SinkMaskCalibrator(cfg)
    cal_host = sa.SinkMaskCalibrator(cfg)
    cal_host.accumulate_on_host = True  # the reference's placement of the sums
    host_sum, host_sq = None, None
    for step in range(3):
        q = torch.randn(2, 2, 700, 128, device="cuda", dtype=torch.bfloat16)
        k = torch.randn(2, 2, 700, 128, device="cuda", dtype=torch.bfloat16)
        cal.record(0, q, k, k)
        cal_host.record(0, q, k, k)
        m = sa._compute_block_scores(q, k, k, cfg).float().mean(dim=0).cpu()
        host_sum = m.clone() if host_sum is None else host_sum + m
        host_sq = m.square() if host_sq is None else host_sq + m.square()
    assert cal.score_sums[0].is_cuda and cal_host.score_sums[0].device.type == "cpu"
    pkg = cal.build_package()
    pkg_host = cal_host.build_package()
    for part in ("mean_scores", "std_scores", "sink_masks"):
        assert torch.equal(pkg[part]["0"], pkg_host[part]["0"]), part
    mean = host_sum / 3
    std = torch.sqrt((host_sq / 3 - mean.square()).clamp_min_(0.0))
    assert torch.equal(pkg["mean_scores"]["0"], mean)
    assert torch.equal(pkg["std_scores"]["0"], std)
    assert torch.equal(pkg["sink_masks"]["0"], torch_ref.coverage_mask(mean))


def test_calibrator_block_64_head_dim_64():
    # block_size 64 and head dim 64 run the generic pooling kernel; the package's masks
    # are the reference's mask of the package's own mean scores, and those means match the
    # oracle's exact block mass of the recorded layers.
    torch.manual_seed(2)
    cfg = sa.SinkSparseConfig(pooling_mode="exact", block_size=64)
    cal = sa.SinkMaskCalibrator(cfg)
    qs, ks = [], []
    for step in range(2):
        q = torch.randn(2, 3, 700, 64, device="cuda", dtype=torch.bfloat16)
        k = torch.randn(2, 3, 700, 64, device="cuda", dtype=torch.bfloat16)
        cal.record(0, q, k, k)
        qs.append(q.cpu())
        ks.append(k.cpu())
    pkg = cal.build_package()
    mean = pkg["mean_scores"]["0"]
    assert mean.shape == (3, 11, 11)
    assert torch.equal(pkg["sink_masks"]["0"], torch_ref.coverage_mask(mean, block_size=64))
    want = sum(torch_ref.exact_block_mass(q, k, block_size=64).mean(dim=0) for q, k in zip(qs, ks)) / 2
    assert torch.allclose(mean, want, rtol=1e-5, atol=1e-8)


@pytest.mark.slow
def test_calibrator_full_wan_layers():
    # BASELINE config 3 at full size: SinkMaskCalibrator.record on two Wan2.1-1.3B layers
    # (B2 H12 N32760 d128 bf16, per-head sink keys at frame-0 positions) x two calls, then
    # build_package (sparse_attention.py:537-608).  The package's masks must be the
    # reference's coverage mask of the package's own means, bit for bit; the means must
    # match the oracle's fp32 exact block mass (the mean over calls of the batch means) on
    # sampled q-blocks, the ragged last one (120 rows) among them, within 1e-5 relative.
    cfg = sa.SinkSparseConfig(pooling_mode="exact")
    cal = sa.SinkMaskCalibrator(cfg)
    B, H, N, D = 2, 12, 32760, 128
    samples = [(0, 0), (3, 17), (7, 128), (11, 255), (5, 254)]   # (head, q-block)
    rows_of = {}
    for call in range(2):
        for layer in range(2):
            seed = 100 * layer + call
            g = torch.Generator(device="cuda").manual_seed(seed)
            q = torch.randn(B, H, N, D, device="cuda", dtype=torch.bfloat16, generator=g)
            k = torch.randn(B, H, N, D, device="cuda", dtype=torch.bfloat16, generator=g)
            gc = torch.Generator().manual_seed(seed)
            for h in range(H):
                k[:, h, torch.randint(0, 30 * 52, (4,), generator=gc).to("cuda")] *= 6.0
            print(f"calibrator full size: layer {layer} call {call}", flush=True)
            cal.record(layer, q, k, k)
            for h, qb in samples:
                r0, r1 = qb * 128, min((qb + 1) * 128, N)
                rows_of[(layer, call, h, qb)] = (q[:, h:h + 1, r0:r1].cpu(), k[:, h:h + 1].cpu())
            del q, k
    pkg = cal.build_package(include_scores=True)
    assert set(pkg["sink_masks"]) == {"0", "1"} and pkg["counts"] == {"0": 2, "1": 2}
    for layer in range(2):
        mean = pkg["mean_scores"][str(layer)]
        assert mean.shape == (H, 256, 256) and mean.device.type == "cpu"
        assert torch.equal(pkg["sink_masks"][str(layer)], torch_ref.coverage_mask(mean))
        assert bool((pkg["std_scores"][str(layer)] >= 0).all())
        for h, qb in samples:
            per_call = []
            for call in range(2):
                qr, kr = rows_of[(layer, call, h, qb)]
                per_call.append(torch_ref.exact_block_mass(qr, kr).mean(dim=0)[0, 0])   # batch mean
            want = (per_call[0] + per_call[1]) / 2
            got = mean[h, qb]
            assert torch.allclose(got, want, rtol=1e-5, atol=1e-8), (layer, h, qb, (got - want).abs().max().item())
            assert abs(float(got.double().sum()) - 1.0) < 1e-4


def _serial_walk_rows(s, coverage):
    """Rows whose coverage cut lies past the range where fp64 prefix sums are exact in any
    order (the kernel scans that range across the wave and walks the rest serially):
    restated from the bound the kernel documents, to show these inputs reach the walk."""
    x = np.sort(s.reshape(-1, s.shape[-1]).astype(np.float32), axis=-1)[:, ::-1]
    count = 0
    for row in x:
        tot = max(np.float32(row.sum(dtype=np.float32)), np.float32(1e-6))
        cum = np.cumsum(row.astype(np.float64)).astype(np.float32)
        hit = np.nonzero(cum >= np.float32(coverage) * tot)[0]
        cut = hit[0] if hit.size else len(row)
        ab = np.abs(row.astype(np.float64))
        mant, ex = np.frexp(np.where(ab > 0, ab, 1.0))  # v = mant * 2^ex, mant in [0.5, 1)
        sig = (mant * 2.0 ** 24).astype(np.int64)  # 24-bit significand as an integer
        tz = np.log2(sig & -sig).astype(np.int64)
        lsb = np.where(ab > 0, ex - 24 + tz, 1 << 20)
        top = np.where(ab > 0, ex - 1, -(1 << 20))  # floor(log2 |x|)
        lsb_min = np.minimum.accumulate(lsb)
        e_max = np.maximum.accumulate(top)
        j = np.arange(len(row))
        cl = np.ceil(np.log2(j + 1)).astype(np.int64)
        bad = np.nonzero((e_max > -(1 << 20)) & (cl + e_max + 1 > lsb_min + 52))[0]
        if bad.size and bad[0] <= cut:
            count += 1
    return count


@pytest.mark.parametrize("coverage,alpha", [(1.0, 0.02), (0.9999999, 0.02)])
def test_prefix_walk_past_exact_range(oracle_lib, coverage, alpha):
    # Wide dynamic range (gamma draws down to denormals) with the cut in the tail: the
    # prefix sums leave the exact range before the cut, so the serial walk finishes them.
    rng = np.random.default_rng(11)
    x = rng.gamma(alpha, size=(3 * 40, 300)).astype(np.float32)
    x[:, 7] += 0.5
    s = torch.from_numpy(x).view(3, 40, 300)
    s = s / s.sum(-1, keepdim=True)
    assert _serial_walk_rows(s.numpy(), coverage) > 10
    ref = torch_ref.coverage_mask(s, coverage=coverage)
    got, counts, idx = ops.coverage_mask(s.cuda(), coverage, True, want_lists=True)
    assert torch.equal(got.cpu(), ref)
    _check_lists(got, counts, idx)
    assert np.array_equal(oracle_lib.coverage_mask(s.numpy(), coverage), ref.numpy())


@pytest.mark.parametrize("mode", ["joint", "video_residual"])
def test_non_finite_scores(mode):
    # inf and NaN entries: NaN sorts first, non-finite values count as 0 in the joint
    # prefix sums, and the video branch's sums and argmax carry them as CPU torch does.
    rng = np.random.default_rng(5)
    x = rng.gamma(0.3, size=(2 * 20, 40)).astype(np.float32)
    x[3, 5] = np.inf
    x[4, 6] = np.nan
    x[5, :] = np.nan
    x[6, 9] = -np.inf
    x[7, 2] = np.nan
    x[7, 30] = np.inf
    x[25, 11] = np.inf
    x[26, 12] = np.nan
    s = torch.from_numpy(x).view(2, 20, 40)
    kw = dict(text_length=256, force_text=True, mode=mode)
    ref = torch_ref.coverage_mask(s, **kw)
    tb = 2
    vt = tb if mode == "video_residual" else None
    got = ops.coverage_mask(s.cuda(), 0.85, True, tb, tb, vt)
    assert torch.equal(got.cpu(), ref)


def test_wan_pooled_map_bit_exact():
    # A full Wan-size pooled map (B2 H12 N32760, frame-0 keys as sinks) averaged over the
    # batch as the calibrator does: near-uniform rows, deep cuts and, for this seed, rows
    # whose cut splits equal values (the tie-exact path on realistic data).
    torch.manual_seed(0)
    q = torch.randn(2, 12, 32760, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(2, 12, 32760, 128, device="cuda", dtype=torch.bfloat16)
    k[:, :, :1560] *= 3.0
    cfg = sa.SinkSparseConfig(pooling_mode="exact")
    s = sa._compute_block_scores(q, k, k, cfg).float().mean(dim=0).contiguous()
    del q, k
    ref = torch_ref.coverage_mask(s.cpu())
    got, counts, idx = ops.coverage_mask(s, 0.85, True, want_lists=True)
    assert torch.equal(got.cpu(), ref)
    _check_lists(got, counts, idx)
    # the drop-in entry point with the reference's CPU tensors
    assert torch.equal(sa._build_direct_mean_coverage_mask(s.cpu(), cfg), ref)


def test_zimage_pooled_map_bit_exact():
    # A Z-Image-shaped pooled map (H30, 16384 image + 512 text tokens, text keys x4 as
    # sinks) through the drop-in with the required text rows and columns.
    torch.manual_seed(1)
    n_img, n_txt = 16384, 512
    q = torch.randn(1, 30, n_img + n_txt, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(1, 30, n_img + n_txt, 128, device="cuda", dtype=torch.bfloat16)
    k[:, :, :n_txt] *= 4.0
    cfg = sa.SinkSparseConfig(pooling_mode="exact", text_length=n_txt, force_text_global_attention=True)
    s = sa._compute_block_scores(q, k, k, cfg).float().mean(dim=0).contiguous()
    del q, k
    assert s.shape == (30, 132, 132)
    ref = torch_ref.coverage_mask(s.cpu(), text_length=n_txt, force_text=True)
    assert torch.equal(sa._build_direct_mean_coverage_mask(s.cpu(), cfg), ref)
    got = ops.coverage_mask(s, 0.85, True, 4, 4)
    assert torch.equal(got.cpu(), ref)
