"""Max-pool map (`attn_with_pooling`, sinkattention/pooling_kernel.py:11-248) against the
reference kernel's own outputs.

tests/golden/max_pool.npz holds Po from the reference's Triton kernel run by Triton's CPU
interpreter (tests/golden/make_max_pool_golden.py), float16, 12 cases: blocks 16-128, head
dims 32-256, causal and not, GQA, "exact" inputs (every q.k exact in fp32) and N(0,1)
inputs.  Inputs are regenerated from their seeds (tests/golden/max_pool_cases.py) and checked
against the fixture's checksum.

CPU:  the oracle reproduces every "exact" fixture bit for bit, and leaving out any one of its
      four rounding points to q.dtype (R, Po, the row sum, the division) breaks some of them.
GPU:  the drop-in `attn_with_pooling` reproduces the "exact" fixtures bit for bit.
N(0,1) inputs, both: the fp32 sums q.k are rounded in another order (numpy's BLAS in the
      fixture, this host's BLAS in the oracle, the matrix cores on the GPU), which moves a
      block maximum R across a q.dtype rounding boundary now and then; the bar there is
      `parity_bars.max_pool_bar` (entries within the factor 2^ulp(max |R|) plus two ulps,
      at most 0.2% of the entries beyond a 2-ulp ripple, 8% of the rows touched, and every
      entry beyond the ripple explained by a deciding row whose block maximum lies within
      the fp32 dot-product error of a rounding boundary).
bf16: the interpreter cannot run the kernel in bf16 (see the fixture script), so bf16 rests
      on the same oracle code, whose bf16 conversion is checked here to round to nearest
      even, and on the GPU-vs-oracle test with the same bar.
"""
import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import torch_ref

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
from max_pool_cases import CASES, DTYPE, digest, make_inputs  # noqa: E402

sys.path.pop(0)
from parity_bars import flips_near_rounding_boundary, max_block_logit, max_pool_bar  # noqa: E402
FIX = np.load(GOLD / "max_pool.npz")
CASE_BY_NAME = {c[0]: c for c in CASES}


def _case(name):
    _, B, H, Hk, N, D, block, causal, kind, seed = CASE_BY_NAME[name]
    q, k, v = make_inputs(B, H, Hk, N, D, kind, seed)
    assert digest(q, k) == str(FIX[f"{name}__inputs_sha256"]), "inputs no longer match the fixture"
    po = torch.from_numpy(FIX[f"{name}__po"].copy()).view(DTYPE)
    return q, k, v, po, block, bool(causal), 1.0 / math.sqrt(D), kind


def _ulps(a, b):
    """Distance in units in the last place of two same-sign finite 16-bit float tensors."""
    return (a.view(torch.int16).int() - b.view(torch.int16).int()).abs()


def test_fixture_lists_every_case():
    assert sorted(str(n) for n in FIX["cases"]) == sorted(CASE_BY_NAME)


def _randn_bar(got, po, q, k, sm, block, causal, what):
    max_pool_bar(got, po, max_block_logit(q, k, sm, block, causal), what, qk=(q, k, sm, block, causal))


@pytest.mark.parametrize("name", sorted(CASE_BY_NAME))
def test_oracle_reproduces_reference_fixture(name):
    q, k, _, po, block, causal, sm, kind = _case(name)
    ours = torch_ref.max_pool_map(q, k, sm, block, causal=causal)
    assert ours.dtype == DTYPE
    d = _ulps(ours, po)
    if kind == "exact":
        assert int(d.max()) == 0, int(d.gt(0).sum())
    else:
        _randn_bar(ours, po, q, k, sm, block, causal, name)


def test_bar_rejects_a_planted_error_away_from_rounding_boundaries():
    # A mistake planted in the oracle's map: one entry of an N(0,1) case scaled by 1.008,
    # inside the 2^ulp(max|R|) - 1 = 1.09% growth the bar allows for boundary flips but far
    # beyond its 2-ulp ripple.  Its q-block has no row near a rounding boundary, so the
    # cause check must fail it.
    q, k, _, po, block, causal, sm, kind = _case("randn_b128_d128")
    ours = torch_ref.max_pool_map(q, k, sm, block, causal=causal)
    cand = [(0, h, qb, kb) for h in range(ours.size(1)) for qb in range(ours.size(2)) for kb in range(ours.size(3))]
    ent = torch.tensor(cand)
    near = flips_near_rounding_boundary(q, k, sm, block, causal, ent, DTYPE)
    assert bool(near.any()) and not bool(near.all())   # the check separates entries
    b, h, qb, kb = cand[int((~near).nonzero()[0])]
    bad = ours.clone()
    bad[b, h, qb, kb] = (bad[b, h, qb, kb].double() * 1.008).to(DTYPE)
    _randn_bar(ours, po, q, k, sm, block, causal, "unplanted")
    with pytest.raises(AssertionError, match="no row near a rounding boundary"):
        _randn_bar(bad, po, q, k, sm, block, causal, "planted")


@pytest.mark.parametrize("point", ["R", "Po", "sum", "div"])
def test_fixtures_detect_each_dropped_rounding_point(point):
    broken = 0
    for name in sorted(n for n, *rest in CASES if rest[-2] == "exact"):
        q, k, _, po, block, causal, sm, _ = _case(name)
        wrong = torch_ref.max_pool_map(q, k, sm, block, causal=causal, skip_rounding=(point,))
        broken += int((wrong.double() != po.double()).sum())
    assert broken > 0


def test_bf16_conversion_rounds_to_nearest_even():
    # known answers for fp32 -> bf16 (8 significant bits): ties go to the even neighbour
    x = torch.tensor([1 + 2 ** -8, 1 + 3 * 2 ** -8, 1 + 2 ** -8 + 2 ** -20, 1 + 2 ** -9,
                      -(1 + 3 * 2 ** -8), 255.5, 256.5, 257.0], dtype=torch.float32)
    want = torch.tensor([1.0, 1 + 2 ** -6, 1 + 2 ** -7, 1.0, -(1 + 2 ** -6), 256.0, 256.0, 256.0])
    assert torch.equal(x.to(torch.bfloat16).float(), want)


def test_bf16_rounding_points_are_all_active():
    # in bf16 too, each rounding point changes the oracle's result on a realistic input
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 2, 1024, 128, generator=g).bfloat16()
    k = torch.randn(1, 2, 1024, 128, generator=g)
    k[:, :, :4] *= 4
    k = k.bfloat16()
    sm = 1.0 / math.sqrt(128)
    full = torch_ref.max_pool_map(q, k, sm, 128)
    for point in ("R", "Po", "sum", "div"):
        wrong = torch_ref.max_pool_map(q, k, sm, 128, skip_rounding=(point,))
        assert (wrong.double() != full.double()).any(), point


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASE_BY_NAME))
def test_kernel_matches_reference_fixtures(name):
    """Bar: "exact" inputs bit for bit; N(0,1) inputs `_randn_bar`."""
    from sinkattention.pooling_kernel import attn_with_pooling
    q, k, v, po, block, causal, sm, kind = _case(name)
    o, got = attn_with_pooling(q.cuda(), k.cuda(), v.cuda(), causal, sm, block)
    torch.cuda.synchronize()
    got = got.cpu()
    assert got.dtype == DTYPE and got.shape == po.shape
    assert bool((o == 0).all())
    d = _ulps(got, po)
    print(f"{name}: {int(d.gt(0).sum())} of {d.numel()} entries differ, max {int(d.max())} ulp")
    if kind == "exact":
        assert int(d.max()) == 0
    else:
        _randn_bar(got, po, q, k, sm, block, causal, name)
