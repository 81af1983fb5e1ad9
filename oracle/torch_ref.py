"""TEST INFRASTRUCTURE ONLY: CPU torch restatements of the reference hot path.

Each function names the reference lines it follows (paths relative to the reference
repository root).  Everything runs on CPU tensors; inputs are moved there.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


# ---------------------------------------------------------------------------------------
# sinkattention/sparse_attention.py:145-227  (_compute_exact_block_mass_scores)
# ---------------------------------------------------------------------------------------
def exact_block_mass(q: torch.Tensor, k: torch.Tensor, block_size: int = 128,
                     key_chunk_blocks: int = 16) -> torch.Tensor:
    q = q.detach().cpu().float()
    k = k.detach().cpu().float()
    B, H, Nq, D = q.shape
    Nk = k.size(2)
    nqb, nkb = _cdiv(Nq, block_size), _cdiv(Nk, block_size)
    chunk = max(1, min(key_chunk_blocks, nkb))
    scale = 1.0 / math.sqrt(D)
    out = torch.empty(B, H, nqb, nkb, dtype=torch.float32)
    for qbi in range(nqb):
        q0, q1 = qbi * block_size, min((qbi + 1) * block_size, Nq)
        qb = q[:, :, q0:q1, :]
        nt = qb.size(2)
        row_max = torch.full((B, H, nt), float("-inf"))
        for kb0 in range(0, nkb, chunk):
            cb = min(chunk, nkb - kb0)
            kc = k[:, :, kb0 * block_size:min((kb0 + cb) * block_size, Nk), :]
            logits = torch.matmul(qb, kc.transpose(-1, -2)) * scale
            row_max = torch.maximum(row_max, logits.amax(dim=-1))
        row_sum = torch.zeros_like(row_max)
        mass = torch.empty(B, H, nt, nkb)
        for kb0 in range(0, nkb, chunk):
            cb = min(chunk, nkb - kb0)
            kc = k[:, :, kb0 * block_size:min((kb0 + cb) * block_size, Nk), :]
            logits = torch.matmul(qb, kc.transpose(-1, -2)) * scale
            p = torch.exp(logits - row_max.unsqueeze(-1))
            row_sum += p.sum(dim=-1)
            pad = cb * block_size - kc.size(2)
            if pad:
                p = F.pad(p, (0, pad), value=0.0)
            mass[:, :, :, kb0:kb0 + cb] = p.view(B, H, nt, cb, block_size).sum(dim=-1)
        mass = mass / row_sum.clamp_min_(1e-6).unsqueeze(-1)
        out[:, :, qbi, :] = mass.mean(dim=2)
    return out


def exact_block_mass_fp64(q: torch.Tensor, k: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """Brute force in float64: full softmax, block sums, mean over the existing rows."""
    q = q.detach().cpu().double()
    k = k.detach().cpu().double()
    B, H, Nq, D = q.shape
    Nk = k.size(2)
    nqb, nkb = _cdiv(Nq, block_size), _cdiv(Nk, block_size)
    p = torch.softmax(torch.matmul(q, k.transpose(-1, -2)) / math.sqrt(D), dim=-1)
    p = F.pad(p, (0, nkb * block_size - Nk))
    blk = p.view(B, H, Nq, nkb, block_size).sum(-1)
    out = torch.empty(B, H, nqb, nkb, dtype=torch.float64)
    for qbi in range(nqb):
        out[:, :, qbi] = blk[:, :, qbi * block_size:min((qbi + 1) * block_size, Nq)].mean(dim=2)
    return out


# ---------------------------------------------------------------------------------------
# sinkattention/pooling_kernel.py:11-248  (attn_with_pooling, non-causal and causal)
# Closed form with the reference's rounding points: R in q.dtype, Po in q.dtype, the
# row sum rounded to q.dtype, the division rounded to q.dtype.
# ---------------------------------------------------------------------------------------
def max_pool_map(q: torch.Tensor, k: torch.Tensor, sm_scale: float, block_size: int = 128,
                 causal: bool = False, exact: bool = False, query_blocks=None,
                 skip_rounding=()) -> torch.Tensor:
    """exact=True evaluates the formula in float64 without any rounding.

    query_blocks (optional): the query-block indices to evaluate, in order; the result
    then holds those rows of the map only.  Each query block is computed on its own
    (rows of the map are independent), so long sequences fit in memory.

    skip_rounding (tests only): names among "R", "Po", "sum", "div" whose rounding to
    q.dtype is left out, so a test can show that the golden fixtures detect each one.
    """
    dt = q.dtype
    work = torch.float64 if exact else torch.float32
    q = q.detach().cpu().to(work)
    k = k.detach().cpu().to(work)
    B, H, N, D = q.shape
    Hk = k.size(1)
    if Hk != H:
        k = k.repeat_interleave(H // Hk, dim=1)
    kt = k.transpose(-1, -2)
    nd = _cdiv(N, block_size)
    qk_scale = torch.tensor(sm_scale, dtype=torch.float32) * torch.tensor(1.44269504, dtype=torch.float32)
    qk_scale = float(qk_scale) if not exact else float(sm_scale) * 1.44269504
    qbs = list(range(nd)) if query_blocks is None else [int(x) for x in query_blocks]
    po = torch.zeros(B, H, len(qbs), nd, dtype=work)
    cols = torch.arange(N)
    for i, qbi in enumerate(qbs):
        r0, r1 = qbi * block_size, min((qbi + 1) * block_size, N)
        s = torch.matmul(q[:, :, r0:r1], kt)  # raw qk, [B,H,rows,N]
        if causal:
            # only the diagonal tile gets the additive -1e6; tiles right of it are never
            # visited
            rows = torch.arange(r0, r1).view(-1, 1)
            above = (cols.view(1, -1) > rows) & (cols.view(1, -1) // block_size == qbi)
            s = s + torch.where(above, torch.tensor(-1.0e6, dtype=work), torch.tensor(0.0, dtype=work))
        s = F.pad(s, (0, nd * block_size - N), value=float("-inf"))
        bmax = s.view(B, H, r1 - r0, nd, block_size).amax(-1) * qk_scale  # [B,H,rows,nd]
        if causal:
            bmax[..., qbi + 1:] = float("-inf")
        m = bmax.amax(-1, keepdim=True)
        r = bmax if exact or "R" in skip_rounding else bmax.to(dt).to(work)
        po[:, :, i] = torch.exp2(r - m).amax(dim=2)
        if causal:
            po[:, :, i, qbi + 1:] = 0.0
    if exact:
        return po / po.sum(-1, keepdim=True)
    po = po.float() if "Po" in skip_rounding else po.to(dt).float()
    tot = po.sum(-1, keepdim=True)
    if "sum" not in skip_rounding:
        tot = tot.to(dt).float()
    out = po / tot
    return out if "div" in skip_rounding else out.to(dt)


# ---------------------------------------------------------------------------------------
# sinkattention/sparse_attention.py:79-94, 138-142  (mean pooling mode)
# ---------------------------------------------------------------------------------------
def mean_pool_scores(q: torch.Tensor, k: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    def pool(x: torch.Tensor) -> torch.Tensor:
        rem = x.size(2) % block_size
        if rem:
            x = F.pad(x, (0, 0, 0, block_size - rem), mode="replicate")
        b, h, n, d = x.shape
        return x.view(b, h, n // block_size, block_size, d).mean(dim=-2)

    qp = pool(q.detach().cpu().float())
    kp = pool(k.detach().cpu().float())
    s = torch.matmul(qp, kp.transpose(-1, -2)) * (1.0 / math.sqrt(q.size(-1)))
    return torch.softmax(s, dim=-1)


# ---------------------------------------------------------------------------------------
# sinkattention/sparse_attention.py:241-265  (_build_offline_required_mask)
# ---------------------------------------------------------------------------------------
def required_mask(nq: int, nk: int, block_size: int, text_length: int,
                  force_text: bool) -> Optional[torch.Tensor]:
    if not (force_text and text_length > 0):
        return None
    tb = _cdiv(text_length, block_size)
    rq, rk = min(tb, nq), min(tb, nk)
    if rq <= 0 or rk <= 0:
        return None
    req = torch.zeros(nq, nk, dtype=torch.bool)
    req[:, :rk] = True
    req[:rq, :] = True
    return req


# ---------------------------------------------------------------------------------------
# sinkattention/sparse_attention.py:268-376  (_build_direct_mean_coverage_mask), CPU
# ---------------------------------------------------------------------------------------
def coverage_mask(mean_scores: torch.Tensor, *, coverage: float = 0.85, keep_diagonal: bool = True,
                  block_size: int = 128, text_length: int = 0, force_text: bool = False,
                  mode: str = "joint") -> torch.Tensor:
    mean_scores = mean_scores.detach().cpu()
    H, nq, nk = mean_scores.shape
    coverage = min(max(float(coverage), 0.0), 1.0)
    req = required_mask(nq, nk, block_size, text_length, force_text)
    scores = mean_scores.float()
    if mode in {"video_residual", "video_residual_only", "residual_video"} and force_text and text_length > 0:
        tb = min(_cdiv(text_length, block_size), nq, nk)
        if tb > 0:
            mask = torch.zeros_like(mean_scores, dtype=torch.bool)
            if req is not None:
                mask |= req.unsqueeze(0).expand(H, -1, -1)
            vq, vk = max(nq - tb, 0), max(nk - tb, 0)
            if vq > 0 and vk > 0:
                vs = scores[:, tb:, tb:]
                tot = vs.sum(dim=-1).clamp_min_(1e-6)
                tgt = coverage * tot
                ss, si = torch.sort(vs, dim=-1, descending=True)
                cum = torch.cumsum(ss, dim=-1)
                reached = cum >= tgt.unsqueeze(-1)
                kk = torch.where(
                    tgt > 1e-6,
                    torch.where(reached.any(dim=-1), reached.float().argmax(dim=-1) + 1,
                                torch.full((H, vq), vk, dtype=torch.int64)),
                    torch.zeros((H, vq), dtype=torch.int64),
                ).clamp(min=0, max=vk)
                keep = torch.arange(vk).view(1, 1, -1) < kk.unsqueeze(-1)
                vm = torch.zeros_like(vs, dtype=torch.bool)
                vm.scatter_(-1, si, keep)
                mask[:, tb:, tb:] |= vm
            empty = ~mask.any(dim=-1)
            if empty.any():
                mask.scatter_(-1, scores.argmax(dim=-1, keepdim=True), empty.unsqueeze(-1))
            return mask

    total = scores.sum(dim=-1).clamp_min_(1e-6)
    mask = torch.zeros_like(mean_scores, dtype=torch.bool)
    if req is not None:
        mask |= req.unsqueeze(0).expand(H, -1, -1)
    selected = (scores * mask.float()).sum(dim=-1)
    target = coverage * total
    residual = (target - selected).clamp_min_(0.0)
    cand = scores.masked_fill(mask, float("-inf"))
    ss, si = torch.sort(cand, dim=-1, descending=True)
    ss = torch.where(torch.isfinite(ss), ss, torch.zeros_like(ss))
    cum = torch.cumsum(ss, dim=-1)
    reached = cum >= residual.unsqueeze(-1)
    ncand = (~mask).sum(dim=-1).to(dtype=torch.int64)
    kk = torch.where(
        residual > 1e-6,
        torch.where(reached.any(dim=-1), reached.float().argmax(dim=-1) + 1, ncand),
        torch.zeros_like(ncand),
    ).clamp(min=0, max=nk)
    keep = torch.arange(nk).view(1, 1, -1) < kk.unsqueeze(-1)
    extra = torch.zeros_like(mean_scores, dtype=torch.bool)
    extra.scatter_(-1, si, keep)
    mask |= extra
    if keep_diagonal:
        dl = min(nq, nk)
        d = torch.arange(dl)
        mask[:, d, d] = True
    empty = ~mask.any(dim=-1)
    if empty.any():
        mask.scatter_(-1, si[..., :1], empty.unsqueeze(-1))
    return mask


# ---------------------------------------------------------------------------------------
# Semantics of block_sparse_attn_func at sinkattention/sparse_attention.py:710-776:
# dense masked softmax in fp32 (keys >= Nk masked), natural-log LSE.  Rows with no listed
# key block: out = 0, lse = +inf.
# ---------------------------------------------------------------------------------------
def dense_masked_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           block_mask: torch.Tensor, scale: Optional[float] = None,
                           rows: Optional[torch.Tensor] = None,
                           block_size: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 reference on CPU.  ``rows`` optionally selects a subset of query rows (the
    same subset for every (b, h)); outputs are then [B, H, len(rows), D] / [B, H, len(rows)]."""
    q = q.detach().cpu().float()
    k = k.detach().cpu().float()
    v = v.detach().cpu().float()
    m = block_mask.detach().cpu().bool()
    B, H, Nq, D = q.shape
    Nk = k.size(2)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if rows is None:
        rows = torch.arange(Nq)
    rows = rows.cpu().long()
    kb_of_key = torch.arange(Nk) // block_size
    qb_of_row = rows // block_size
    out = torch.zeros(B, H, rows.numel(), D)
    lse = torch.full((B, H, rows.numel()), float("inf"))
    for b in range(B):
        for h in range(H):
            allowed = m[b, h][qb_of_row][:, kb_of_key]  # [R, Nk]
            s = torch.matmul(q[b, h, rows], k[b, h].transpose(0, 1)) * scale
            s = s.masked_fill(~allowed, float("-inf"))
            has = allowed.any(dim=-1)
            if has.any():
                sm = s[has]
                p = torch.softmax(sm, dim=-1)
                out[b, h, has] = torch.matmul(p, v[b, h])
                lse[b, h, has] = torch.logsumexp(sm, dim=-1)
    return out, lse


# ---------------------------------------------------------------------------------------
# sinkattention/sparse_attention.py:898-919  (_mix_attention_outputs)
# ---------------------------------------------------------------------------------------
def mix(sink_out, sink_lse, dyn_out, dyn_lse, sample_gap: int):
    log_gap = sink_lse.new_tensor(float(max(1, int(sample_gap)))).log()
    ws, wd = sink_lse, dyn_lse + log_gap
    mx = torch.maximum(ws, wd)
    es, ed = torch.exp(ws - mx), torch.exp(wd - mx)
    a = es / (es + ed)
    return sink_out * a + dyn_out * (1.0 - a)


# ---------------------------------------------------------------------------------------
# sinkattention/sparse_attention.py:79-115  (_pad_to_multiple, _mean_pool_sequence,
# _mean_pool_sequence_preserve_prefix): the compensation branch's K/V pooling.
# ---------------------------------------------------------------------------------------
def mean_pool_tokens(x: torch.Tensor, gap: int, prefix: int = 0) -> torch.Tensor:
    """fp32 on CPU.  Rows [0, prefix) of dim 2 are kept as they are; the remaining rows
    are taken in groups of ``gap`` consecutive rows and each group becomes its mean; a
    short last group counts its last row again for every missing row (replicate
    padding).  ``gap`` <= 1 returns the input; ``prefix`` >= rows returns the input."""
    x = x.detach().cpu().float()
    n = x.size(2)
    if gap <= 1:
        return x
    prefix = min(max(int(prefix), 0), n)
    if prefix >= n:
        return x
    body = x[:, :, prefix:]
    m = body.size(2)
    groups = []
    for g0 in range(0, m, gap):
        rows = body[:, :, g0:min(g0 + gap, m)]
        missing = gap - rows.size(2)
        total = rows.sum(dim=2)
        if missing:
            total = total + missing * body[:, :, m - 1]
        groups.append(total / gap)
    return torch.cat([x[:, :, :prefix], torch.stack(groups, dim=2)], dim=2)


# ---------------------------------------------------------------------------------------
# QK-norm and rotary embedding in front of the attention:
#   wanx/runtime/fast_misc.py:308-340 (_rms_norm_fwd_fused), 432-500 (_rotary_qk_fwd_fused),
#   182-192 (_torch_real_apply_rotary_emb); zimg/runtime/modify_zimage.py:8-43.
# ---------------------------------------------------------------------------------------
def rms_norm_rows(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """fp32 on CPU: x * (1 / sqrt(mean(x^2) + eps)) * w over the last dim."""
    x = x.detach().cpu().float()
    var = (x * x).sum(-1, keepdim=True) / x.size(-1)
    return x * (1.0 / torch.sqrt(var + eps)) * w.detach().cpu().float()


def rotate_pairs(y: torch.Tensor, real: torch.Tensor, imag: torch.Tensor) -> torch.Tensor:
    """Channel pairs (2i, 2i+1) of the last dim rotated by (real[..., i], imag[..., i]):
    (y0*re - y1*im, y0*im + y1*re); real/imag broadcast against y[..., ::2]."""
    y0, y1 = y[..., 0::2], y[..., 1::2]
    out = torch.empty_like(y)
    out[..., 0::2] = y0 * real - y1 * imag
    out[..., 1::2] = y0 * imag + y1 * real
    return out
