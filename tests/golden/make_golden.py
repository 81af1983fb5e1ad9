"""Regenerate the golden fixtures in this directory (run from the repository root):

    python tests/golden/make_golden.py

The reference ships no test vectors, so the fixtures come from the CPU oracle
(oracle/torch_ref.py, itself pinned by tests/test_oracle_*.py) on seeded inputs.  They
freeze small cases of each hot-path function so that a change to either the oracle or
the kernels shows up as a fixture mismatch.  Inputs of 16-bit kernels are stored as raw
bf16 bit patterns (uint16); masks are bit-packed.
"""
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import torch_ref  # noqa: E402

OUT = Path(__file__).resolve().parent


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def scores(H, nq, nk, seed, kind):
    rng = np.random.default_rng(seed)
    if kind == "ties":
        x = rng.integers(0, 5, size=(H * nq, nk)) / 7.0
    else:
        x = rng.gamma(0.3, size=(H * nq, nk))
    s = torch.from_numpy(x.astype(np.float32)).view(H, nq, nk)
    return s / s.sum(-1, keepdim=True).clamp_min(1e-30)


def make_masks():
    cases = {
        "c1_joint": (scores(12, 32, 32, 1, "gamma"), dict()),
        "c1_ties": (scores(12, 32, 32, 2, "ties"), dict()),
        "zimg_required": (scores(4, 132, 132, 3, "gamma"), dict(text_length=512, force_text=True)),
        "zimg_video": (scores(4, 132, 132, 4, "ties"), dict(text_length=512, force_text=True, mode="video_residual")),
        "nodiag": (scores(3, 40, 17, 5, "gamma"), dict(keep_diagonal=False)),
    }
    arrays = {}
    for name, (s, kw) in cases.items():
        m = torch_ref.coverage_mask(s, **kw).numpy()
        arrays[f"{name}/scores"] = s.numpy()
        arrays[f"{name}/mask_bits"] = np.packbits(m, axis=-1)
        arrays[f"{name}/shape"] = np.array(m.shape)
        arrays[f"{name}/kw"] = np.array(repr(kw))
    np.savez_compressed(OUT / "coverage_masks.npz", **arrays)


def make_exact_mass():
    g = torch.Generator().manual_seed(10)
    q = torch.randn(1, 2, 256, 128, generator=g).bfloat16()
    k = torch.randn(1, 2, 300, 128, generator=g)
    k[:, :, :3] *= 8.0
    k = k.bfloat16()
    ref = torch_ref.exact_block_mass_fp64(q, k)
    np.savez_compressed(OUT / "exact_mass.npz", q_bf16=bf16_bits(q), k_bf16=bf16_bits(k), mass_fp64=ref.numpy())


def make_attention():
    g = torch.Generator().manual_seed(11)
    q = torch.randn(1, 2, 300, 128, generator=g).bfloat16()
    k = torch.randn(1, 2, 300, 128, generator=g).bfloat16()
    v = torch.randn(1, 2, 300, 128, generator=g).bfloat16()
    m = torch.rand(1, 2, 3, 3, generator=g) < 0.5
    m[0, 0, 1] = False  # one row with no listed block
    m[0, 1, :, 0] = True
    o, l = torch_ref.dense_masked_attention(q, k, v, m)
    np.savez_compressed(OUT / "attention.npz", q_bf16=bf16_bits(q), k_bf16=bf16_bits(k), v_bf16=bf16_bits(v),
                        mask=m.numpy(), out_f16=o.half().numpy(), lse=l.numpy())


if __name__ == "__main__":
    make_masks()
    make_exact_mass()
    make_attention()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
