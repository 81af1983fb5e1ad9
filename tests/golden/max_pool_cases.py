"""Cases and seeded inputs of the max-pool golden fixture (tests/golden/max_pool.npz).

Shared by the script that writes the fixture from the reference's kernel
(make_max_pool_golden.py) and by the tests that read it, so inputs are regenerated from
their seeds instead of being stored; the fixture keeps a checksum of them.
"""
from __future__ import annotations

import hashlib

import torch

DTYPE = torch.float16

# name, B, H, Hk, N, D, block, causal, inputs, seed
CASES = [
    ("exact_b128_d128", 1, 2, 2, 2048, 128, 128, False, "exact", 11),
    ("exact_b128_d128_causal", 1, 2, 2, 2048, 128, 128, True, "exact", 12),
    ("exact_b64_d64", 1, 2, 2, 2048, 64, 64, False, "exact", 13),
    ("exact_b64_d128_causal", 1, 2, 2, 1536, 128, 64, True, "exact", 14),
    ("exact_b32_d64", 1, 2, 2, 1024, 64, 32, False, "exact", 15),
    ("exact_b64_d64_gqa", 1, 4, 2, 1024, 64, 64, False, "exact", 16),
    ("randn_b128_d128", 1, 2, 2, 2048, 128, 128, False, "randn", 21),
    ("randn_b128_d128_causal", 1, 2, 2, 2048, 128, 128, True, "randn", 22),
    ("randn_b64_d64", 1, 2, 2, 2048, 64, 64, False, "randn", 23),
    ("randn_b64_d128_gqa", 2, 2, 1, 1024, 128, 64, False, "randn", 24),
    ("randn_b16_d256", 1, 1, 1, 512, 256, 16, False, "randn", 25),
    ("randn_b32_d32_causal", 1, 2, 2, 1024, 32, 32, True, "randn", 26),
]


def make_inputs(B, H, Hk, N, D, kind, seed, dtype=DTYPE):
    """Q [B,H,N,D], K/V [B,Hk,N,D] on the CPU; keys 0..3 of every head are sinks (x4).

    kind "exact": Q/K entries rounded to multiples of 1/8 in [-3, 3] (x4 for the sinks), so
    every q.k dot product is exact in fp32.  kind "randn": N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, N, D, generator=g)
    k = torch.randn(B, Hk, N, D, generator=g)
    v = torch.randn(B, Hk, N, D, generator=g)
    if kind == "exact":
        q = (q * 8).round().clamp(-24, 24) / 8
        k = (k * 8).round().clamp(-24, 24) / 8
    k[:, :, 0:4] *= 4
    return q.to(dtype), k.to(dtype), v.to(dtype)


def digest(*tensors) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().view(torch.int16).numpy().tobytes())
    return h.hexdigest()
