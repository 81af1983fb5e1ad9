"""Pin the pooling and attention oracles (CPU only) against float64 brute force, closed
forms and torch's own SDPA, so that the GPU parity tests compare against something
that is itself checked."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import torch_ref


def _qk(B, H, Nq, Nk, D, seed, sinks=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, Nq, D, generator=g)
    k = torch.randn(B, H, Nk, D, generator=g)
    if sinks:
        k[:, :, :sinks] *= 8.0
    return q, k


@pytest.mark.parametrize("Nq,Nk", [(256, 256), (300, 1000), (129, 2200)])
def test_exact_mass_restatement_vs_fp64(Nq, Nk):
    q, k = _qk(1, 2, Nq, Nk, 128, seed=Nq + Nk, sinks=4)
    ours = torch_ref.exact_block_mass(q, k).double()
    ref = torch_ref.exact_block_mass_fp64(q, k)
    assert ((ours - ref).abs() <= 1e-5 * ref.abs() + 1e-12).all()
    assert torch.allclose(ours.sum(-1), torch.ones_like(ours.sum(-1)), atol=1e-5)


def test_exact_mass_closed_forms():
    # Q = 0 -> uniform softmax -> |kb| / Nk, ragged last block included
    Nk = 1016
    q = torch.zeros(1, 1, 200, 64)
    k = torch.randn(1, 1, Nk, 64)
    m = torch_ref.exact_block_mass(q, k)
    want = torch.tensor([128.0] * 7 + [120.0]) / Nk
    assert torch.allclose(m[0, 0], want.expand(2, -1), rtol=1e-6)
    # one dominant key -> its block holds all the mass
    k2 = torch.zeros(1, 1, Nk, 64)
    k2[0, 0, 700] = 60.0
    m2 = torch_ref.exact_block_mass(torch.ones(1, 1, 130, 64), k2)
    assert torch.allclose(m2[0, 0, :, 5], torch.ones(2), atol=1e-6)
    # a single key block: every row's mass is 1
    assert torch.allclose(torch_ref.exact_block_mass(*_qk(1, 1, 70, 100, 32, 3)), torch.ones(1, 1, 1, 1))


def test_exact_mass_chunking_is_irrelevant():
    q, k = _qk(1, 1, 256, 2600, 64, seed=9)
    a = torch_ref.exact_block_mass(q, k, key_chunk_blocks=16)
    b = torch_ref.exact_block_mass(q, k, key_chunk_blocks=3)
    assert torch.allclose(a, b, rtol=1e-6, atol=1e-9)


def test_max_pool_restatement_vs_formula():
    q, k = _qk(1, 2, 512, 512, 128, seed=4)
    qb, kb = q.bfloat16(), k.bfloat16()
    sm = 1 / math.sqrt(128)
    got = torch_ref.max_pool_map(qb, kb, sm)
    assert got.dtype == torch.bfloat16
    # formula evaluated independently in float64 from the definition
    s = (qb.double() @ kb.double().transpose(-1, -2)) * sm * 1.44269504
    bm = s.view(1, 2, 512, 4, 128).amax(-1)  # [B,H,N,nb]
    e = torch.exp2(bm - bm.amax(-1, keepdim=True))
    po = e.view(1, 2, 4, 128, 4).amax(3)
    po = po / po.sum(-1, keepdim=True)
    assert torch.allclose(got.double(), po, rtol=0.25, atol=1e-3)
    # row normalisation (up to bf16 rounding of each entry)
    assert torch.allclose(got.float().sum(-1), torch.ones(1, 2, 4), atol=3e-2)
    # causal: entries above the diagonal are zero, first row is [1, 0, ...]
    c = torch_ref.max_pool_map(qb, kb, sm, causal=True).float()
    assert torch.equal(c[0, 0, 0], torch.tensor([1.0, 0, 0, 0]))
    assert (torch.triu(c[0, 0], diagonal=1) == 0).all()
    # causal against the definition with keys after the row removed: the reference's
    # additive -1e6 on the diagonal tile drops them from every block maximum here
    sc = s.masked_fill(torch.ones(512, 512, dtype=torch.bool).triu(1), float("-inf"))
    bmc = sc.view(1, 2, 512, 4, 128).amax(-1)
    ec = torch.exp2(bmc - bmc.amax(-1, keepdim=True)).view(1, 2, 4, 128, 4).amax(3)
    assert torch.allclose(c.double(), ec / ec.sum(-1, keepdim=True), rtol=0.25, atol=1e-3)


def test_max_pool_query_block_subset_matches_full_map():
    q, k = _qk(1, 2, 700, 700, 128, seed=14)
    qb, kb = q.bfloat16(), k.bfloat16()
    for causal in (False, True):
        full = torch_ref.max_pool_map(qb, kb, 0.09, causal=causal)
        sub = torch_ref.max_pool_map(qb, kb, 0.09, causal=causal, query_blocks=[5, 0, 3])
        assert torch.equal(sub, full[:, :, [5, 0, 3]])


def test_mean_pool_closed_form():
    q, k = _qk(1, 1, 300, 260, 16, seed=5)
    s = torch_ref.mean_pool_scores(q, k)
    # manual: replicate the last row to a multiple of 128, average, softmax
    def pool(x):
        n = x.shape[2]
        pad = (-n) % 128
        x = torch.cat([x, x[:, :, -1:].expand(-1, -1, pad, -1)], dim=2)
        return x.view(1, 1, -1, 128, x.shape[-1]).mean(3)
    want = torch.softmax(pool(q) @ pool(k).transpose(-1, -2) / 4.0, dim=-1)
    assert torch.allclose(s, want, atol=1e-6)


def test_dense_masked_attention_oracle():
    g = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(1, 2, 300, 32, generator=g) for _ in range(3))
    full = torch.ones(1, 2, 3, 3, dtype=torch.bool)
    o, l = torch_ref.dense_masked_attention(q, k, v, full)
    assert torch.allclose(o, F.scaled_dot_product_attention(q, k, v), atol=1e-5)
    s = q @ k.transpose(-1, -2) / math.sqrt(32)
    assert torch.allclose(l, torch.logsumexp(s, -1), atol=1e-5)
    diag = torch.eye(3, dtype=torch.bool).expand(1, 2, 3, 3)
    o2, _ = torch_ref.dense_masked_attention(q, k, v, diag)
    for b in range(3):
        sl = slice(b * 128, min((b + 1) * 128, 300))
        ref = F.scaled_dot_product_attention(q[:, :, sl], k[:, :, sl], v[:, :, sl])
        assert torch.allclose(o2[:, :, sl], ref, atol=1e-5)
    empty = torch.zeros(1, 2, 3, 3, dtype=torch.bool)
    o3, l3 = torch_ref.dense_masked_attention(q, k, v, empty)
    assert (o3 == 0).all() and torch.isinf(l3).all()
    rows = torch.tensor([0, 5, 299])
    o4, l4 = torch_ref.dense_masked_attention(q, k, v, full, rows=rows)
    assert torch.allclose(o4, o[:, :, rows]) and torch.allclose(l4, l[:, :, rows])
