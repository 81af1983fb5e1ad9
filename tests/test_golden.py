"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the
pinned CPU oracle): the oracle must still reproduce them exactly, and the GPU kernels
must match them to the parity bar (bit-exact masks, 1e-5 relative block mass,
2e-2 / 1e-3 attention)."""
import ast
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import torch_ref

GOLD = Path(__file__).resolve().parent / "golden"


def _bf16(a):
    return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)


def _mask_cases():
    z = np.load(GOLD / "coverage_masks.npz")
    names = sorted({k.split("/")[0] for k in z.files})
    for n in names:
        shape = tuple(z[f"{n}/shape"])
        m = np.unpackbits(z[f"{n}/mask_bits"], axis=-1)[..., : shape[-1]].astype(bool)
        yield n, torch.from_numpy(z[f"{n}/scores"]), torch.from_numpy(m), ast.literal_eval(str(z[f"{n}/kw"]))


def test_oracle_reproduces_mask_fixtures():
    for name, s, m, kw in _mask_cases():
        assert torch.equal(torch_ref.coverage_mask(s, **kw), m), name


def test_oracle_reproduces_mass_and_attention_fixtures():
    z = np.load(GOLD / "exact_mass.npz")
    q, k = _bf16(z["q_bf16"]), _bf16(z["k_bf16"])
    assert np.allclose(torch_ref.exact_block_mass(q, k).double().numpy(), z["mass_fp64"], rtol=1e-5, atol=1e-12)
    a = np.load(GOLD / "attention.npz")
    o, l = torch_ref.dense_masked_attention(_bf16(a["q_bf16"]), _bf16(a["k_bf16"]), _bf16(a["v_bf16"]),
                                            torch.from_numpy(a["mask"]))
    assert np.allclose(o.numpy(), a["out_f16"].astype(np.float32), atol=1e-3)
    assert np.array_equal(np.isinf(l.numpy()), np.isinf(a["lse"]))


@pytest.mark.gpu
def test_kernels_match_fixtures():
    from sinkattn_amd import ops
    from sinkattn_amd import sparse_attention as sa
    for name, s, m, kw in _mask_cases():
        cfg = sa.SinkSparseConfig(keep_diagonal=kw.get("keep_diagonal", True), text_length=kw.get("text_length", 0),
                                  force_text_global_attention=kw.get("force_text", False),
                                  offline_text_video_coverage_mode=kw.get("mode", "joint"))
        assert torch.equal(sa._build_direct_mean_coverage_mask(s.cuda(), cfg).cpu(), m), name
    z = np.load(GOLD / "exact_mass.npz")
    got = ops.block_mass_scores(_bf16(z["q_bf16"]).cuda(), _bf16(z["k_bf16"]).cuda()).cpu().double().numpy()
    assert np.all(np.abs(got - z["mass_fp64"]) <= 1e-5 * np.abs(z["mass_fp64"]) + 1e-9)
    a = np.load(GOLD / "attention.npz")
    q, k, v = (_bf16(a[f"{t}_bf16"]).cuda() for t in "qkv")
    out, lse = ops.block_sparse_attention(q, k, v, ops.block_sparse_plan(torch.from_numpy(a["mask"]).cuda()))
    err = np.abs(out.float().cpu().numpy() - a["out_f16"].astype(np.float32))
    assert err.max() <= 2e-2 and err.mean() <= 1e-3
    fin = np.isfinite(a["lse"])
    lse = lse.cpu().numpy()
    assert np.array_equal(np.isfinite(lse), fin) and np.abs(lse[fin] - a["lse"][fin]).max() <= 2e-2
