"""Parity bars shared by several test files (not a test module itself)."""
import math

import torch


def dtype_ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Unit in the last place of `dtype` at |x| (float64; normal range)."""
    mant = {torch.float16: 10, torch.bfloat16: 7}[dtype]
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -14)))
    return torch.pow(2.0, e - mant)


def max_block_logit(q: torch.Tensor, k: torch.Tensor, sm_scale: float, block: int, causal: bool,
                    rows=None) -> float:
    """max |R| over the map: R = (block maximum of q.k) * sm_scale * log2(e), in float64.
    `rows` (optional) limits it to those query rows."""
    qd = q.detach().cpu().double()
    kd = k.detach().cpu().double()
    if kd.size(1) != qd.size(1):
        kd = kd.repeat_interleave(qd.size(1) // kd.size(1), dim=1)
    Nk = kd.size(2)
    ridx = torch.arange(qd.size(2)) if rows is None else torch.as_tensor(rows)
    s = qd[:, :, ridx] @ kd.transpose(-1, -2) * (sm_scale * 1.44269504)
    if causal:
        s = s.masked_fill(torch.arange(Nk).view(1, -1) > ridx.view(-1, 1), float("-inf"))
    nd = math.ceil(Nk / block)
    s = torch.nn.functional.pad(s, (0, nd * block - Nk), value=float("-inf"))
    bmax = s.view(*s.shape[:-1], nd, block).amax(-1)
    return float(bmax[torch.isfinite(bmax)].abs().max())


def max_pool_bar(got: torch.Tensor, ref: torch.Tensor, r_max: float, what: str = "",
                 max_row_frac: float = 0.10, max_flip_frac: float = 0.01) -> None:
    """Bar for the max-pool map where q.k is summed in another order than in `ref`.

    Cause: the last fp32 bits of q.k change; when that moves R = q.dtype(max * scale) across
    a rounding boundary, exp2(R - m) of that block changes by the factor 2^ulp(R), so Po
    changes by at most that factor plus its own rounding, and the row total moves by at
    most one ulp, which moves every entry of the row by one more ulp after the division.
    So: |got - ref| <= ref * (2^ulp(r_max) - 1) + 2 ulp(ref) everywhere, and flips are rare
    (one needs a q.k within a few fp32 ulps of a boundary): at most `max_flip_frac` of the
    entries differ by more than the 2-ulp ripple of a row total, and at most `max_row_frac`
    of the rows differ at all.
    """
    dt = ref.dtype
    got = got.detach().cpu()
    ref = ref.detach().cpu()
    assert got.dtype == dt and got.shape == ref.shape, what
    g, r = got.double(), ref.double()
    growth = 2.0 ** float(dtype_ulp(torch.tensor(r_max, dtype=torch.float64), dt)) - 1.0
    bound = r.abs() * growth + 2 * dtype_ulp(r, dt)
    diff = (g - r).abs()
    worst = float((diff - bound).max())
    assert worst <= 0.0, (what, worst, float(diff.max()))
    flips = (diff > 2 * dtype_ulp(r, dt)).float().mean().item()
    assert flips <= max_flip_frac, (what, flips)
    rows = (got.view(torch.int16) != ref.view(torch.int16)).any(-1).float().mean().item()
    assert rows <= max_row_frac, (what, rows)
