"""Pin the coverage-mask oracles (CPU only).

oracle/torch_ref.coverage_mask restates sinkattention/sparse_attention.py:268-376 with
the same torch calls; oracle/coverage_ref.c restates it in plain C together with the
CPU torch arithmetic it depends on.  These tests tie the C model to this machine's torch
(sum order, cumsum rounding, sort permutation incl. ties), the sort emulation to the
real libstdc++ std::sort, and both builders to definitions that do not reuse their code:
a float64 brute-force minimal cover, invariants and special cases.
"""
import numpy as np
import pytest
import torch

from oracle import torch_ref


def _rows(rng, n_rows, n, kind):
    if kind == "dirichlet":
        x = rng.gamma(0.3, size=(n_rows, n)).astype(np.float32)
    elif kind == "ties":
        x = rng.integers(0, 5, size=(n_rows, n)).astype(np.float32) / 7.0
    elif kind == "wide":
        x = (rng.random((n_rows, n)) * 10.0 ** rng.uniform(-30, 3, size=(n_rows, n))).astype(np.float32)
    else:
        raise ValueError(kind)
    return x


@pytest.mark.parametrize("n", [1, 3, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 100, 127, 128, 132,
                               255, 256, 257, 511, 512, 513, 1000, 1024])
def test_aten_row_sum_model_matches_torch(oracle_lib, n):
    rng = np.random.default_rng(n)
    for kind in ("dirichlet", "wide"):
        x = _rows(rng, 64, n, kind)
        ours = np.array([oracle_lib.aten_row_sum(r) for r in x], dtype=np.float32)
        ref = torch.from_numpy(x).sum(dim=-1).numpy()
        assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32)), (n, kind)


def test_aten_row_sum_model_on_strided_slice(oracle_lib):
    # the video_residual branch sums a [H, nq-tb, nk-tb] slice of a contiguous tensor
    rng = np.random.default_rng(7)
    full = torch.from_numpy(_rows(rng, 12 * 132, 132, "dirichlet")).view(12, 132, 132)
    sl = full[:, 4:, 4:]
    ref = sl.sum(dim=-1).numpy()
    ours = np.array([[oracle_lib.aten_row_sum(np.ascontiguousarray(sl[h, r].numpy()))
                      for r in range(sl.shape[1])] for h in range(12)], dtype=np.float32)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_cumsum_model_matches_torch(oracle_lib):
    rng = np.random.default_rng(1)
    for n in (17, 256, 1024):
        x = _rows(rng, 1, n, "wide")[0]
        assert np.array_equal(oracle_lib.cumsum_f32(x), torch.cumsum(torch.from_numpy(x), 0).numpy())


@pytest.mark.parametrize("n", [2, 5, 16, 17, 32, 33, 100, 132, 256, 600, 1024])
def test_sort_emulation_matches_libstdcxx_and_torch(oracle_lib, n):
    rng = np.random.default_rng(100 + n)
    for trial in range(60):
        v = rng.integers(0, 4, size=n).astype(np.float32)
        v[rng.random(n) < 0.15] = -np.inf
        if trial % 5 == 0:
            v[:] = 0.0  # all ties
        if trial % 7 == 1:
            v = np.sort(v)  # ascending input drives introsort deep
        if trial % 11 == 2:
            v[rng.random(n) < 0.1] = np.nan
        ve, ie = oracle_lib.std_sort_desc(v)
        vr, ir = oracle_lib.std_sort_desc(v, emulated=False)
        _, it = torch.sort(torch.from_numpy(v).view(1, -1), dim=-1, descending=True)
        assert np.array_equal(ie, ir), (n, trial)
        assert np.array_equal(ir, it.numpy()[0]), (n, trial)


def test_torch_sort_is_not_stable_on_ties():
    # the permutation matters: a stable sort would give a different tie order
    v = torch.zeros(1, 64)
    a = torch.sort(v, dim=-1, descending=True)[1]
    b = torch.sort(v, dim=-1, descending=True, stable=True)[1]
    assert not torch.equal(a, b)


CASES = [
    dict(shape=(12, 32, 32)),
    dict(shape=(12, 256, 256)),
    dict(shape=(30, 132, 132), text_length=512, force_text=True),
    dict(shape=(30, 132, 132), text_length=512, force_text=True, mode="video_residual"),
    dict(shape=(4, 40, 17), keep_diagonal=False),
    dict(shape=(4, 17, 40), text_length=300, force_text=True),
    dict(shape=(3, 9, 7), coverage=0.5),
    dict(shape=(3, 64, 600)),
]


def _c_call(oracle_lib, s, *, coverage=0.85, keep_diagonal=True, block_size=128, text_length=0,
            force_text=False, mode="joint"):
    H, nq, nk = s.shape
    rq = rk = 0
    if force_text and text_length > 0:
        tb = -(-text_length // block_size)
        rq, rk = min(tb, nq), min(tb, nk)
    vt = None
    if mode == "video_residual" and force_text and text_length > 0:
        vt = min(-(-text_length // block_size), nq, nk)
    return oracle_lib.coverage_mask(s.numpy(), coverage, keep_diagonal, rq, rk, vt)


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("kind", ["dirichlet", "ties", "wide"])
def test_c_builder_matches_torch_builder(oracle_lib, case, kind):
    c = dict(CASES[case])
    shape = c.pop("shape")
    rng = np.random.default_rng(case * 10 + len(kind))
    s = torch.from_numpy(_rows(rng, shape[0] * shape[1], shape[2], kind)).view(*shape)
    s = s / s.sum(-1, keepdim=True).clamp_min(1e-30)
    ref = torch_ref.coverage_mask(s, **c).numpy()
    ours = _c_call(oracle_lib, s, **c)
    assert np.array_equal(ours, ref)


def test_builder_special_rows(oracle_lib):
    nk = 32
    rows = []
    r = np.full(nk, 0.1 / (nk - 1), np.float32); r[5] = 0.9; rows.append(r)      # dominant block
    rows.append(np.full(nk, 1.0 / nk, np.float32))                              # uniform
    r = np.zeros(nk, np.float32); r[20] = 0.7; r[[10, 12, 14]] = 0.1; rows.append(r)  # tie at the cut
    s = torch.from_numpy(np.stack(rows)).view(1, len(rows), nk)
    for keep in (True, False):
        ref = torch_ref.coverage_mask(s, keep_diagonal=keep).numpy()[0]
        ours = _c_call(oracle_lib, s, keep_diagonal=keep)[0]
        assert np.array_equal(ours, ref)
        # dominant block: {5} plus the diagonal (row 0)
        assert set(np.nonzero(ref[0])[0]) == ({5, 0} if keep else {5})
        # a tie straddling the cut: 0.7 + two of the three tied 0.1 blocks reach 0.85
        assert ref[2][20] and ref[2][[10, 12, 14]].sum() == 2
    # uniform row: the smallest k whose fp32 prefix reaches 0.85 of the fp32 total
    tot = oracle_lib.aten_row_sum(rows[1])
    cum = oracle_lib.cumsum_f32(rows[1])
    k = int(np.argmax(cum >= np.float32(0.85) * tot)) + 1
    assert _c_call(oracle_lib, s, keep_diagonal=False)[0][1].sum() == k


def test_builder_empty_row_fallback_quirk(oracle_lib):
    """The reference's fallback `mask.scatter_(-1, top1, empty_rows)` writes the empty
    flag at every row's top-1 position: the empty row gains its top-1 block, and every
    non-empty row LOSES its top-1 block (sparse_attention.py:371-374)."""
    nk = 16
    a = np.full(nk, 0.1 / (nk - 1), np.float32); a[5] = 0.9
    z = np.zeros(nk, np.float32)
    s = torch.from_numpy(np.stack([a, z])).view(1, 2, nk)
    ref = torch_ref.coverage_mask(s, keep_diagonal=False).numpy()[0]
    assert np.array_equal(_c_call(oracle_lib, s, keep_diagonal=False)[0], ref)
    assert not ref[0].any()          # lost block 5 (its only block)
    assert ref[1].sum() == 1         # the all-zero row got its first sorted index
    # without an empty row nothing is cleared
    s2 = torch.from_numpy(np.stack([a, a])).view(1, 2, nk)
    assert torch_ref.coverage_mask(s2, keep_diagonal=False).numpy()[0][:, 5].all()


def test_builder_matches_float64_minimal_cover(oracle_lib):
    """Definition check: kept candidates are the smallest prefix of the descending order
    whose mass reaches coverage*total - required mass (float64), away from rounding ties."""
    rng = np.random.default_rng(5)
    H, nq, nk = 6, 24, 24
    s = torch.from_numpy(rng.gamma(0.5, size=(H * nq, nk)).astype(np.float32)).view(H, nq, nk)
    s = s / s.sum(-1, keepdim=True)
    for force_text in (False, True):
        m = _c_call(oracle_lib, s, keep_diagonal=False, text_length=200 if force_text else 0,
                    force_text=force_text, block_size=128)
        rq = rk = (2 if force_text else 0)
        checked = 0
        for h in range(H):
            for q in range(nq):
                x = s[h, q].double().numpy()
                req = np.zeros(nk, bool)
                req[:rk] = True
                if q < rq:
                    req[:] = True
                tot = x.sum()
                res = max(0.85 * tot - x[req].sum(), 0.0)
                cand = np.where(req, -np.inf, x)
                order = np.argsort(-cand, kind="stable")
                cum = np.cumsum(np.where(np.isfinite(cand[order]), cand[order], 0.0))
                if res <= 1e-6:
                    k = 0
                else:
                    hit = np.nonzero(cum >= res)[0]
                    k = hit[0] + 1 if hit.size else int((~req).sum())
                    near = np.abs(cum - res) < 1e-5 * max(res, 1e-12)
                    if near.any():
                        continue
                want = req.copy()
                want[order[:k]] = True
                if not want.any():
                    continue
                assert np.array_equal(m[h, q], want), (h, q)
                checked += 1
        assert checked > H * nq // 2


def test_builder_invariants(oracle_lib):
    rng = np.random.default_rng(9)
    s = torch.from_numpy(rng.gamma(0.4, size=(8 * 64, 64)).astype(np.float32)).view(8, 64, 64)
    s = s / s.sum(-1, keepdim=True)
    m = _c_call(oracle_lib, s, keep_diagonal=False)
    md = _c_call(oracle_lib, s, keep_diagonal=True)
    sd = s.double().numpy()
    assert md.any(-1).all()
    assert all(md[h, q, q] for h in range(8) for q in range(64))
    assert np.array_equal(md | m, md)
    for h in range(8):
        for q in range(64):
            x = sd[h, q]
            sel = m[h, q]
            covered = x[sel].sum()
            assert covered >= 0.85 * x.sum() - 1e-6
            # minimality: removing the smallest kept block falls below the target
            smallest = x[sel].min()
            assert covered - smallest < 0.85 * x.sum() + 1e-6


def test_required_prefix_zimage():
    m = torch_ref.required_mask(132, 132, 128, 512, True)
    assert m[:4].all() and m[:, :4].all() and not m[4:, 4:].any()
    assert torch_ref.required_mask(132, 132, 128, 512, False) is None
    assert torch_ref.required_mask(132, 132, 128, 0, True) is None
