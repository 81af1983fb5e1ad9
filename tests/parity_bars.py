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


LOG2E = 1.44269504


def flips_near_rounding_boundary(q: torch.Tensor, k: torch.Tensor, sm_scale: float, block: int, causal: bool,
                                 entries: torch.Tensor, dtype: torch.dtype, query_blocks=None) -> torch.Tensor:
    """For each map entry (b, h, qb, kb) in `entries` ([n, 4] int64), whether a rounding
    flip can explain a change of it.  The entry is max over the rows r of q-block qb of
    exp2(R[r, kb] - m_r), R = dtype(x), x = max_{j in kb}(q_r.k_j) * sm_scale * log2(e),
    m_r = the row's largest x.  Only rows whose term is within a factor 2^(2 ulp(R)) of the
    entry's largest term (fp64) can decide it, and such a row explains the change only if
    its x can fall on either side of a `dtype` rounding boundary: x rounds to two different
    `dtype` values at the two ends of the interval the fp32 error of the dot products
    allows, |q.k - fl32(q.k)| <= D * 2^-24 * sum_i |q_i k_i| for any summation order
    (recursive-summation bound), plus two fp32 ulps for the scaling.  `query_blocks`: the
    map's rows are these q-blocks."""
    qd = q.detach().cpu().double()
    kd = k.detach().cpu().double()
    H, Hk = qd.size(1), kd.size(1)
    N, Nk, D = qd.size(2), kd.size(2), qd.size(3)
    nkb = math.ceil(Nk / block)
    gamma = D * 2.0 ** -24
    c = sm_scale * LOG2E
    out = torch.zeros(entries.size(0), dtype=torch.bool)
    groups = {}
    for i, (b, h, qb, kb) in enumerate(entries.tolist()):
        groups.setdefault((b, h, qb), []).append((i, kb))
    for (b, h, qb), items in groups.items():
        qb_abs = query_blocks[qb] if query_blocks is not None else qb
        r0, r1 = qb_abs * block, min((qb_abs + 1) * block, N)
        qr = qd[b, h, r0:r1]
        kh = kd[b, h // (H // Hk)]
        s = qr @ kh.T
        if causal:
            s = s.masked_fill(torch.arange(Nk).view(1, -1) > torch.arange(r0, r1).view(-1, 1), float("-inf"))
        sp = torch.nn.functional.pad(s, (0, nkb * block - Nk), value=float("-inf"))
        x = sp.view(s.size(0), nkb, block).amax(-1) * c            # [rows, nkb], log2 units
        m = x.amax(-1)
        for i, kb in items:
            xk = x[:, kb]
            fin = torch.isfinite(xk)
            if not bool(fin.any()):
                continue
            v = (xk - m).masked_fill(~fin, float("-inf"))
            ulp = dtype_ulp(xk.masked_fill(~fin, 0.0), dtype)
            cand = fin & (v >= v.max() - 2 * ulp.max())
            k0, k1 = kb * block, min((kb + 1) * block, Nk)
            kt = kh[k0:k1]
            err = ((qr.abs() @ kt.abs().T) * gamma).amax(-1) * c
            lo, hi = xk - err, xk + err
            lo = lo - lo.abs() * 2.0 ** -22
            hi = hi + hi.abs() * 2.0 ** -22
            flip = lo.float().to(dtype) != hi.float().to(dtype)
            out[i] = bool((flip & cand).any())
    return out


def max_pool_bar(got: torch.Tensor, ref: torch.Tensor, r_max: float, what: str = "",
                 max_row_frac: float = 0.08, max_flip_frac: float = 2e-3, qk=None,
                 max_checked: int = 400) -> None:
    """Bar for the max-pool map where q.k is summed in another order than in `ref`.

    Cause: the last fp32 bits of q.k change; when that moves R = q.dtype(max * scale) across
    a rounding boundary, exp2(R - m) of that block changes by the factor 2^ulp(R), so Po
    changes by at most that factor plus its own rounding, and the row total moves by at
    most one ulp, which moves every entry of the row by one more ulp after the division.
    So: |got - ref| <= ref * (2^ulp(r_max) - 1) + 2 ulp(ref) everywhere, and flips are rare
    (one needs a q.k within a few fp32 ulps of a boundary): at most `max_flip_frac` of the
    entries differ by more than the 2-ulp ripple of a row total, and at most `max_row_frac`
    of the rows differ at all.

    The defaults sit just above what the kernels show against the reference's fixtures and
    the oracle (at most 1 entry of 1024 beyond the ripple and 2 rows of 32 touched, on 16-
    to 32-block maps).

    `qk` = (q, k, sm_scale, block, causal[, query_blocks]): then every entry beyond the 2-ulp
    ripple (up to `max_checked` of them, a seeded sample) must also have the cause above, a
    row whose block maximum lies within the fp32 error of a rounding boundary
    (`flips_near_rounding_boundary`); an error of the kernel confined to a few entries fails
    that check.
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
    beyond = diff > 2 * dtype_ulp(r, dt)
    flips = beyond.float().mean().item()
    assert flips <= max_flip_frac, (what, flips)
    if qk is not None and bool(beyond.any()):
        ent = beyond.nonzero()
        if ent.size(0) > max_checked:
            pick = torch.randperm(ent.size(0), generator=torch.Generator().manual_seed(0))[:max_checked]
            ent = ent[pick]
        q, k, sm_scale, block, causal = qk[:5]
        qbs = qk[5] if len(qk) > 5 else None
        ok = flips_near_rounding_boundary(q, k, sm_scale, block, causal, ent, dt, qbs)
        assert bool(ok.all()), (what, "entries off by more than 2 ulps with no row near a rounding boundary",
                                ent[~ok][:8].tolist())
    rows = (got.view(torch.int16) != ref.view(torch.int16)).any(-1).float().mean().item()
    print(f"max_pool_bar {what}: {flips:.3e} of the entries beyond 2 ulps, {rows:.3e} of the rows differ",
          flush=True)
    assert rows <= max_row_frac, (what, rows)
