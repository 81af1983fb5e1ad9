"""Write tests/golden/max_pool.npz: outputs of the reference's own `attn_with_pooling`
(sinkattention/pooling_kernel.py:194-248, kernel :11-192) run by Triton's CPU interpreter.

The max-pool map is the one function of the path that no closed form or brute force pins at
the bit level: its value depends on four rounding points in q.dtype (the per-block row
maximum R, the pooled value Po, the row sum, the division).  So this script runs the
reference's source file itself, in this container only, under `TRITON_INTERPRET=1` (Triton
3.6.0 is installed here; no GPU is used), and stores inputs and outputs as a fixture.  The
reference file is loaded from its path with `importlib`; nothing of it is copied, and no
bytecode is written.

Only float16 runs here.  Triton 3.6.0's interpreter stores bfloat16 as raw uint16: its
`tl.dot` hands those bit patterns to `np.matmul` as integers (it converts only fp8 operands),
and its fp32 -> bf16 `fptrunc` drops mantissa bits (round toward zero) where the hardware
conversion rounds to nearest even.  So it cannot stand for the reference kernel in bf16.
float16 is a native numpy type there: loads, `tl.dot` (fp32 accumulation), `.to(float16)`
(round to nearest even) and the wrapper's torch sum / division all behave as on the GPU.  The
four rounding points are the same code for both 16-bit types (`.to(q.dtype)`), so the f16
fixtures pin them; the bf16 rounding itself is torch's / the hardware's round-to-nearest-even.

Cases (tests/golden/max_pool_cases.py; N a multiple of the block, where the reference is
defined; inputs regenerated from their seeds, the fixture keeps their checksum):
* "exact" inputs: Q/K entries are multiples of 1/8 (sink keys x4 stay multiples of 1/8), so
  every q.k dot product is exact in fp32 whatever the summation order.  The only steps whose
  last fp32 bit may then depend on the implementation are exp2 and the fp32 row sum;
* "randn" inputs, N(0,1) (the realistic case): the fp32 accumulation order of q.k differs
  between implementations as well.
Blocks 128, 64, 32 and 16, head dims 32, 64, 128 and 256, causal off and on, GQA (n_rep 2).
Every exp2 argument stays above -126 (checked), so denormal flushing cannot matter.

Usage:  python tests/golden/make_max_pool_golden.py [/root/reference]
"""
from __future__ import annotations

import importlib.util
import math
import os
import sys
from pathlib import Path

os.environ["TRITON_INTERPRET"] = "1"
sys.dont_write_bytecode = True

import numpy as np  # noqa: E402
import torch  # noqa: E402

sys.path.insert(0, str(Path(__file__).resolve().parent))
from max_pool_cases import CASES, DTYPE, digest, make_inputs  # noqa: E402

HERE = Path(__file__).resolve().parent
OUT = HERE / "max_pool.npz"

def load_reference(root: Path):
    path = root / "sinkattention" / "pooling_kernel.py"
    spec = importlib.util.spec_from_file_location("reference_pooling_kernel", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    # The wrapper asks the active GPU driver whether it runs on HIP (pooling_kernel.py:8-9,
    # 217-219); the interpreter has no driver.  Answer as the MI355X does.  The launch options
    # that answer selects (waves_per_eu, allow_flush_denorm) change no arithmetic here except
    # the flushing of denormal results, which these inputs never produce (checked below).
    mod.is_hip = lambda: True
    return mod


def min_exp2_argument(q, k, sm_scale, block, causal):
    """Smallest R - m over all rows and key blocks, in float64 (no denormal check needed
    above -126)."""
    qd, kd = q.double(), k.double()
    if kd.size(1) != qd.size(1):
        kd = kd.repeat_interleave(qd.size(1) // kd.size(1), dim=1)
    s = qd @ kd.transpose(-1, -2) * sm_scale * 1.44269504
    B, H, N, _ = s.shape
    nd = N // block
    if causal:
        s = s.masked_fill(torch.ones(N, N, dtype=torch.bool).triu(1), float("-inf"))
    bmax = s.view(B, H, N, nd, block).amax(-1)
    m = bmax.amax(-1, keepdim=True)
    diff = bmax - m
    return float(diff[torch.isfinite(diff)].min())


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    ref = load_reference(root)
    arrays = {}
    names = []
    for name, B, H, Hk, N, D, block, causal, kind, seed in CASES:
        q, k, v = make_inputs(B, H, Hk, N, D, kind, seed)
        sm_scale = 1.0 / math.sqrt(D)
        lowest = min_exp2_argument(q, k, sm_scale, block, causal)
        assert lowest > -120.0, (name, lowest)
        o, po = ref.attn_with_pooling(q, k, v, causal, sm_scale, block)
        assert po.dtype == DTYPE and tuple(po.shape) == (B, H, N // block, N // block)
        assert bool((o == 0).all())          # l_i = 1 and acc = 0 throughout (:161-167)
        arrays[f"{name}__inputs_sha256"] = np.array(digest(q, k))
        arrays[f"{name}__po"] = po.view(torch.int16).numpy()
        arrays[f"{name}__meta"] = np.array([B, H, Hk, N, D, block, int(causal), seed], dtype=np.int64)
        arrays[f"{name}__sm_scale"] = np.array(sm_scale, dtype=np.float64)
        names.append(name)
        print(f"{name}: Po {tuple(po.shape)}, lowest exp2 argument {lowest:.1f}", flush=True)
    arrays["cases"] = np.array(names)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
