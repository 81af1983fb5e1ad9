"""Torch-facing wrappers of the libsinkattn kernels.

Each wrapper checks device/dtype/shape, allocates outputs with torch on the inputs'
device, and launches on torch's current stream.  Inputs on the CPU, or any other
condition the kernels cannot handle, raise: there is no CPU or eager fallback.
"""
from __future__ import annotations

import math
import weakref
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from sinkattn_amd import _lib

KERNEL_BLOCK = 128


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def _require_cuda(name: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(f"{name}: tensors must be on a ROCm GPU (got {t.device})")


def _kernel_operand(t: torch.Tensor) -> torch.Tensor:
    """Return t if the kernels can address it in place, else a contiguous copy."""
    s = t.stride()
    ok = (
        t.dim() == 4
        and s[3] == 1
        and all(x % 8 == 0 and x >= 0 for x in s[:3])
        and t.data_ptr() % 16 == 0
    )
    return t if ok else t.contiguous()


def _pad_head_dim(t: torch.Tensor, to: Optional[int] = None) -> torch.Tensor:
    """Zero-pad the head dim of a pooling operand to `to`, or else to a multiple of 16
    (16-bit dtypes: the matrix-core score path) or 8 (fp32: the 8-element stride rule); dot
    products, the only use of the head dim in the pooling modes, are unchanged by zero
    padding."""
    D = int(t.shape[-1])
    if to is not None and D < to:
        return torch.nn.functional.pad(t, (0, to - D))
    mult = 8 if t.dtype == torch.float32 else 16
    if D % mult == 0:
        return t
    return torch.nn.functional.pad(t, (0, mult - D % mult))


# Block sizes of the matrix-core pooling kernels (exact block mass and max-pool; 16-bit
# inputs, head dim 128).
MASS_MFMA_BLOCKS = (16, 32, 64, 128)


@dataclass
class BlockSparsePlan:
    """Per-(b, h, q-block) ascending key-block lists built from a bool block mask."""

    counts: torch.Tensor  # int32 [B*H*nqb]
    idx: torch.Tensor  # int32 [B*H*nqb*nkb]
    order: torch.Tensor  # int32 launch slots (XCD-aware; -1 = empty slot)
    shape: Tuple[int, int, int, int]  # B, H, nqb, nkb

    @property
    def listed_tiles(self) -> torch.Tensor:
        return self.counts.sum()


def block_sparse_plan(block_mask: torch.Tensor, order_cache: Optional[torch.Tensor] = None,
                      cache_entries: int = 0) -> BlockSparsePlan:
    """Turn a bool [B, H, nqb, nkb] mask into the kernel's lists and launch order.  With
    `order_cache` (int32, order_cache_ints(B, H, nqb, cache_entries) entries, zero-filled
    when new, one shape, used on one stream) the launch order is copied from an earlier
    plan whose tile counts hash alike instead of being ranked again."""
    _require_cuda("block_sparse_plan", block_mask)
    if block_mask.dim() != 4:
        raise ValueError(f"block mask must be [B, H, nqb, nkb], got {tuple(block_mask.shape)}")
    m = block_mask
    if m.dtype != torch.bool and m.dtype != torch.uint8:
        m = m != 0
    B, H, nqb, nkb = (int(x) for x in m.shape)
    dev = m.device
    rows = B * H * nqb
    L = _lib.lib()
    counts = torch.empty(rows, dtype=torch.int32, device=dev)
    idx = torch.empty(rows * nkb, dtype=torch.int32, device=dev)
    order = torch.empty(max(int(L.sinkattn_block_sparse_order_slots(B, H, nqb)), 1), dtype=torch.int32,
                        device=dev)
    with torch.cuda.device(dev):
        st = _lib.strides4(m)
        if order_cache is None:
            rc = L.sinkattn_block_sparse_plan(m.data_ptr(), st, B, H, nqb, nkb, counts.data_ptr(),
                                              idx.data_ptr(), order.data_ptr(), _lib.stream_ptr(dev))
        else:
            need = int(L.sinkattn_block_sparse_order_cache_ints(B, H, nqb, int(cache_entries)))
            if (order_cache.dtype != torch.int32 or order_cache.device != dev or not order_cache.is_contiguous()
                    or order_cache.numel() < need or need <= 0):
                raise ValueError(f"order_cache must be a contiguous int32 tensor of {need} entries on {dev}")
            rc = L.sinkattn_block_sparse_plan_cached(m.data_ptr(), st, B, H, nqb, nkb, counts.data_ptr(),
                                                     idx.data_ptr(), order.data_ptr(), order_cache.data_ptr(),
                                                     int(cache_entries), _lib.stream_ptr(dev))
        _lib.check(rc, "block_sparse_plan")
    return BlockSparsePlan(counts, idx, order, (B, H, nqb, nkb))


def order_cache_ints(B: int, H: int, nqb: int, entries: int) -> int:
    return int(_lib.lib().sinkattn_block_sparse_order_cache_ints(B, H, nqb, entries))


class _PlanCache:
    """Plans keyed by mask tensor identity and version (runtime masks are cached objects).

    A mask tensor not seen before (callers such as the reference's Z-Image processor build a
    fresh one per call) gets a new plan: its lists are always built from the mask, and its
    launch order comes from a device-side launch-order cache per (shape, device, stream)
    when an earlier plan of that shape had tile counts that hash alike, so only the first
    call of each distinct count pattern ranks the order (no host synchronisation either
    way)."""

    ORDER_CACHE_ENTRIES = 64

    def __init__(self) -> None:
        self._entries: Dict[int, tuple] = {}
        self._order_caches: Dict[tuple, torch.Tensor] = {}

    def order_cache(self, mask: torch.Tensor) -> torch.Tensor:
        B, H, nqb, _ = (int(x) for x in mask.shape)
        key = (B, H, nqb, mask.device, torch.cuda.current_stream(mask.device).cuda_stream)
        oc = self._order_caches.get(key)
        if oc is None:
            n = order_cache_ints(B, H, nqb, self.ORDER_CACHE_ENTRIES)
            oc = torch.zeros(max(n, 1), dtype=torch.int32, device=mask.device)
            self._order_caches[key] = oc
        return oc

    def get(self, mask: torch.Tensor) -> BlockSparsePlan:
        key = id(mask)
        ent = self._entries.get(key)
        sig = (mask._version, mask.data_ptr(), tuple(mask.shape), tuple(mask.stride()), mask.device)
        if ent is not None:
            ref, esig, plan = ent
            if ref() is mask and esig == sig:
                return plan
        if mask.dim() == 4 and mask.numel() > 0:
            plan = block_sparse_plan(mask, self.order_cache(mask), self.ORDER_CACHE_ENTRIES)
        else:
            plan = block_sparse_plan(mask)
        entries = self._entries
        ref = weakref.ref(mask, lambda _r, k=key: entries.pop(k, None))
        entries[key] = (ref, sig, plan)
        return plan

    def clear(self) -> None:
        self._entries.clear()
        self._order_caches.clear()


PLAN_CACHE = _PlanCache()


def block_sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    plan: BlockSparsePlan,
    softmax_scale: Optional[float] = None,
    return_lse: bool = True,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Block-sparse attention forward on [B, H, N, D] views.

    Returns out as a [B, H, Nq, D] view of [B, Nq, H, D] memory (the layout the
    reference's varlen call returns) and lse as fp32 [B, H, Nq] (or None).
    """
    _require_cuda("block_sparse_attention", q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, H, N, D]")
    B, H, Nq, D = (int(x) for x in q.shape)
    Nk = int(k.shape[2])
    if tuple(k.shape) != (B, H, Nk, D) or tuple(v.shape) != (B, H, Nk, D):
        raise ValueError(f"k/v shapes {tuple(k.shape)}/{tuple(v.shape)} do not match q {tuple(q.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    dt = _lib.dtype_code(q.dtype)
    nqb, nkb = _cdiv(Nq, KERNEL_BLOCK), _cdiv(Nk, KERNEL_BLOCK)
    if plan.shape != (B, H, nqb, nkb):
        raise ValueError(f"block mask shape {plan.shape} does not match [{B}, {H}, {nqb}, {nkb}]")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    qk, kk, vk = _kernel_operand(q), _kernel_operand(k), _kernel_operand(v)
    out = torch.empty((B, Nq, H, D), dtype=q.dtype, device=q.device).permute(0, 2, 1, 3)
    lse = torch.empty((B, H, Nq), dtype=torch.float32, device=q.device) if return_lse else None
    L = _lib.lib()
    with torch.cuda.device(q.device):
        _lib.check(
            L.sinkattn_block_sparse_fwd(
                qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), dt, B, H, Nq, Nk, D,
                _lib.strides4(qk), _lib.strides4(kk), _lib.strides4(vk),
                out.data_ptr(), _lib.strides4(out), _lib.ptr(lse),
                plan.counts.data_ptr(), plan.idx.data_ptr(), plan.order.data_ptr(),
                nqb, nkb, float(softmax_scale), _lib.stream_ptr(q.device),
            ),
            "block_sparse_fwd",
        )
    return out, lse


def _empty_like_layout(t: torch.Tensor, rows: int) -> torch.Tensor:
    """Uninitialised [B, H, rows, D] tensor whose dims are laid out in memory in the same
    order as t's (so a [B, N, H, D]-memory view gets a [B, rows, H, D]-memory result and
    the two share row-stride structure)."""
    shape = list(t.shape)
    shape[2] = rows
    order = sorted(range(4), key=lambda d: (-t.stride(d), -d))  # outermost first
    buf = torch.empty([shape[d] for d in order], dtype=t.dtype, device=t.device)
    inv = [order.index(d) for d in range(4)]
    return buf.permute(*inv)


def mean_pool_tokens(x: torch.Tensor, gap: int, prefix: int = 0,
                     like: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rows [0, prefix) of dim 2 kept, the rest averaged in groups of `gap` (a short last
    group repeats the last row).  x is [B, H, N, D] on the GPU.  The result has the
    memory layout of `like` (default x) along (B, H, rows, D)."""
    _require_cuda("mean_pool_tokens", x)
    if x.dim() != 4:
        raise ValueError(f"x must be [B, H, N, D], got {tuple(x.shape)}")
    B, H, N, D = (int(s) for s in x.shape)
    L = _lib.lib()
    rows = int(L.sinkattn_mean_pool_tokens_rows(N, int(prefix), int(gap)))
    if rows < 0:
        raise ValueError(f"mean_pool_tokens: bad gap {gap}")
    xk = _kernel_operand(x)
    out = _empty_like_layout(like if like is not None else x, rows)
    if not (out.stride(3) == 1 and all(s % 8 == 0 for s in out.stride()[:3])):
        out = torch.empty((B, H, rows, D), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(
            L.sinkattn_mean_pool_tokens(
                xk.data_ptr(), _lib.dtype_code(x.dtype), B, H, N, D, _lib.strides4(xk), int(prefix), int(gap),
                out.data_ptr(), _lib.strides4(out), _lib.stream_ptr(x.device),
            ),
            "mean_pool_tokens",
        )
    return out


def block_sparse_attention_comp(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    plan: BlockSparsePlan,
    kd: torch.Tensor,
    vd: torch.Tensor,
    gap: int,
    comp_rows: Optional[int] = None,
    softmax_scale: Optional[float] = None,
    return_lse: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Block-sparse attention fused with the compensation branch: query rows below
    `comp_rows` (default all; must be a multiple of 128 or Nq) also attend every key of
    kd/vd with weight `gap` each, which equals the reference's LSE mix of the two
    branches.  kd/vd must share k's/v's row strides (see mean_pool_tokens(like=...))."""
    _require_cuda("block_sparse_attention_comp", q, k, v, kd, vd)
    B, H, Nq, D = (int(x) for x in q.shape)
    Nk, Nd = int(k.shape[2]), int(kd.shape[2])
    if tuple(k.shape) != (B, H, Nk, D) or tuple(v.shape) != (B, H, Nk, D):
        raise ValueError(f"k/v shapes {tuple(k.shape)}/{tuple(v.shape)} do not match q {tuple(q.shape)}")
    if tuple(kd.shape) != (B, H, Nd, D) or tuple(vd.shape) != (B, H, Nd, D):
        raise ValueError(f"kd/vd shapes {tuple(kd.shape)}/{tuple(vd.shape)} do not match [{B}, {H}, Nd, {D}]")
    if not (q.dtype == k.dtype == v.dtype == kd.dtype == vd.dtype) or q.dtype == torch.float32 or D != 128:
        raise TypeError("block_sparse_attention_comp: bf16/f16 operands of one dtype, head dim 128")
    nqb, nkb = _cdiv(Nq, KERNEL_BLOCK), _cdiv(Nk, KERNEL_BLOCK)
    if plan.shape != (B, H, nqb, nkb):
        raise ValueError(f"block mask shape {plan.shape} does not match [{B}, {H}, {nqb}, {nkb}]")
    comp_rows = Nq if comp_rows is None else int(comp_rows)
    if comp_rows != Nq and comp_rows % KERNEL_BLOCK != 0:
        raise ValueError(f"comp_rows {comp_rows} must be a multiple of {KERNEL_BLOCK} or Nq")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    qk, kk, vk = _kernel_operand(q), _kernel_operand(k), _kernel_operand(v)
    kdk, vdk = _kernel_operand(kd), _kernel_operand(vd)
    if kdk.stride(2) != kk.stride(2) or vdk.stride(2) != vk.stride(2):
        raise ValueError("kd/vd row strides must equal k/v row strides")
    out = torch.empty((B, Nq, H, D), dtype=q.dtype, device=q.device).permute(0, 2, 1, 3)
    lse = torch.empty((B, H, Nq), dtype=torch.float32, device=q.device) if return_lse else None
    L = _lib.lib()
    with torch.cuda.device(q.device):
        _lib.check(
            L.sinkattn_block_sparse_fwd_comp(
                qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), _lib.dtype_code(q.dtype), B, H, Nq, Nk, D,
                _lib.strides4(qk), _lib.strides4(kk), _lib.strides4(vk),
                kdk.data_ptr(), vdk.data_ptr(), _lib.strides4(kdk), _lib.strides4(vdk), Nd,
                _cdiv(comp_rows, KERNEL_BLOCK), float(math.log(max(1, int(gap)))),
                out.data_ptr(), _lib.strides4(out), _lib.ptr(lse),
                plan.counts.data_ptr(), plan.idx.data_ptr(), plan.order.data_ptr(),
                nqb, nkb, float(softmax_scale), _lib.stream_ptr(q.device),
            ),
            "block_sparse_fwd_comp",
        )
    return out, lse


def lse_mix(sink_out: torch.Tensor, sink_lse: torch.Tensor, dyn_out: torch.Tensor, dyn_lse: torch.Tensor,
            log_gap: float) -> torch.Tensor:
    """out = a*sink_out + (1-a)*dyn_out, a = sigmoid(sink_lse - dyn_lse - log_gap), with
    each step rounded to the tensors' dtype like the reference's torch ops.  Outputs
    [B, H, N, D], LSEs [B, H, N] or [B, H, N, 1], one dtype, on the GPU."""
    _require_cuda("lse_mix", sink_out, sink_lse, dyn_out, dyn_lse)
    B, H, N, D = (int(x) for x in sink_out.shape)
    if tuple(dyn_out.shape) != (B, H, N, D):
        raise ValueError("lse_mix: output shapes differ")
    ls = sink_lse.reshape(B, H, N) if sink_lse.dim() == 4 else sink_lse
    ld = dyn_lse.reshape(B, H, N) if dyn_lse.dim() == 4 else dyn_lse
    if tuple(ls.shape) != (B, H, N) or tuple(ld.shape) != (B, H, N):
        raise ValueError("lse_mix: LSE shapes must be [B, H, N] or [B, H, N, 1]")
    if not (sink_out.dtype == dyn_out.dtype == ls.dtype == ld.dtype):
        raise TypeError("lse_mix: one dtype for outputs and LSEs")
    so, do = _kernel_operand(sink_out), _kernel_operand(dyn_out)
    out = torch.empty((B, N, H, D), dtype=sink_out.dtype, device=sink_out.device).permute(0, 2, 1, 3)
    L = _lib.lib()
    with torch.cuda.device(sink_out.device):
        _lib.check(
            L.sinkattn_lse_mix(
                so.data_ptr(), _lib.strides4(so), ls.data_ptr(), _lib.strides3(ls),
                do.data_ptr(), _lib.strides4(do), ld.data_ptr(), _lib.strides3(ld),
                _lib.dtype_code(sink_out.dtype), B, H, N, D, float(log_gap),
                out.data_ptr(), _lib.strides4(out), _lib.stream_ptr(sink_out.device),
            ),
            "lse_mix",
        )
    return out


def qk_norm_rotary(q: torch.Tensor, k: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, eps_q: float,
                   eps_k: float, head_dim: int, freq_real: Optional[torch.Tensor] = None,
                   freq_imag: Optional[torch.Tensor] = None, rows_per_pos: int = 1,
                   out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm of every row of C = q.size(-1) channels (weights wq/wk, fp32 math) and the
    rotation of each head's channel pairs by the table row (row // rows_per_pos) %
    freq_rows, in one kernel for q and k.  q and k are [..., C] with contiguous rows
    (equal shapes); freq_real/freq_imag are [freq_rows, head_dim // 2] (None: no
    rotation).  Returns new tensors of q's shape (or writes `out`)."""
    _require_cuda("qk_norm_rotary", q, k)
    if q.shape != k.shape or q.dtype != k.dtype:
        raise ValueError("qk_norm_rotary: q and k must have one shape and dtype")
    C = int(q.size(-1))
    rows = q.numel() // max(C, 1)
    qc, kc = q.reshape(rows, C), k.reshape(rows, C)
    if qc.stride(1) != 1 or kc.stride(1) != 1 or qc.stride(0) != kc.stride(0):
        qc, kc = qc.contiguous(), kc.contiguous()
    wq32 = wq.detach().to(device=q.device, dtype=torch.float32).contiguous()
    wk32 = wk.detach().to(device=q.device, dtype=torch.float32).contiguous()
    if wq32.numel() != C or wk32.numel() != C:
        raise ValueError(f"qk_norm_rotary: weights must have {C} elements")
    if (freq_real is None) != (freq_imag is None):
        raise ValueError("qk_norm_rotary: give both rotation tables or neither")
    fr = fi = None
    freq_rows = 1
    if freq_real is not None:
        fr = freq_real.detach().to(device=q.device, dtype=torch.float32).reshape(-1, head_dim // 2).contiguous()
        fi = freq_imag.detach().to(device=q.device, dtype=torch.float32).reshape(-1, head_dim // 2).contiguous()
        freq_rows = int(fr.size(0))
    if out is None:
        qo, ko = torch.empty_like(qc), torch.empty_like(kc)
    else:
        qo, ko = out[0].reshape(rows, C), out[1].reshape(rows, C)
    L = _lib.lib()
    with torch.cuda.device(q.device):
        _lib.check(
            L.sinkattn_qk_norm_rotary(
                qc.data_ptr(), kc.data_ptr(), _lib.dtype_code(q.dtype), rows, C, int(head_dim), int(qc.stride(0)),
                wq32.data_ptr(), wk32.data_ptr(), float(eps_q), float(eps_k), _lib.ptr(fr), _lib.ptr(fi),
                int(rows_per_pos), freq_rows, qo.data_ptr(), ko.data_ptr(), int(qo.stride(0)),
                _lib.stream_ptr(q.device),
            ),
            "qk_norm_rotary",
        )
    return qo.view(q.shape), ko.view(k.shape)


def block_mass_scores(q: torch.Tensor, k: torch.Tensor, block_size: int = 128,
                      scale: Optional[float] = None) -> torch.Tensor:
    """Exact per-(q-block, k-block) mean softmax mass, fp32 [B, H, nqb, nkb]."""
    _require_cuda("block_mass_scores", q, k)
    B, H, Nq, D = (int(x) for x in q.shape)
    Nk = int(k.shape[2])
    if tuple(k.shape) != (B, H, Nk, D):
        raise ValueError(f"k shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if q.dtype != k.dtype:
        raise TypeError("q and k must share a dtype")
    dt = _lib.dtype_code(q.dtype)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    # a 16-bit head dim below 128 is zero-padded to 128 for the matrix-core kernel
    to = 128 if (q.dtype != torch.float32 and D < 128 and int(block_size) in MASS_MFMA_BLOCKS) else None
    qk, kk = _kernel_operand(_pad_head_dim(q, to)), _kernel_operand(_pad_head_dim(k, to))
    D = int(qk.shape[-1])
    out = torch.empty((B, H, _cdiv(Nq, block_size), _cdiv(Nk, block_size)), dtype=torch.float32,
                      device=q.device)
    L = _lib.lib()
    with torch.cuda.device(q.device):
        ws_bytes = int(L.sinkattn_block_mass_pool_workspace_bytes(B, H, Nq, Nk, int(block_size), dt))
        ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=q.device) if ws_bytes else None
        _lib.check(
            L.sinkattn_block_mass_pool(
                qk.data_ptr(), kk.data_ptr(), dt, B, H, Nq, Nk, D, _lib.strides4(qk),
                _lib.strides4(kk), int(block_size), float(scale), out.data_ptr(), _lib.ptr(ws),
                _lib.stream_ptr(q.device),
            ),
            "block_mass_pool",
        )
    return out


def max_pool_scores(q: torch.Tensor, k: torch.Tensor, sm_scale: float, block_size: int = 128,
                    causal: bool = False) -> torch.Tensor:
    """Row-normalised max-pool map in q.dtype, [B, H, nd, nd]."""
    _require_cuda("max_pool_scores", q, k)
    B, H, N, D = (int(x) for x in q.shape)
    Hk = int(k.shape[1])
    if int(k.shape[0]) != B or int(k.shape[2]) != N or int(k.shape[3]) != D:
        raise ValueError(f"k shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if q.dtype != k.dtype:
        raise TypeError("q and k must share a dtype")
    dt = _lib.dtype_code(q.dtype)
    if q.dtype != torch.float32 and D in (16, 32, 64) and int(block_size) in MASS_MFMA_BLOCKS:
        # the reference's head dims below 128, zero-padded for the matrix-core kernel (the
        # dot products, all the map depends on, are unchanged)
        q, k = _pad_head_dim(q, 128), _pad_head_dim(k, 128)
        D = 128
    qk, kk = _kernel_operand(q), _kernel_operand(k)
    nd = _cdiv(N, block_size)
    po = torch.empty((B, H, nd, nd), dtype=q.dtype, device=q.device)
    L = _lib.lib()
    with torch.cuda.device(q.device):
        ws_bytes = int(L.sinkattn_max_pool_workspace_bytes(B, H, N, int(block_size), dt))
        ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=q.device) if ws_bytes else None
        _lib.check(
            L.sinkattn_max_pool(
                qk.data_ptr(), kk.data_ptr(), dt, B, H, Hk, N, D, _lib.strides4(qk),
                _lib.strides4(kk), int(block_size), float(sm_scale), int(bool(causal)),
                po.data_ptr(), _lib.ptr(ws), _lib.stream_ptr(q.device),
            ),
            "max_pool",
        )
    return po


def mean_pool_scores(q: torch.Tensor, k: torch.Tensor, block_size: int = 128,
                     scale: Optional[float] = None) -> torch.Tensor:
    """softmax(mean-pooled Q . mean-pooled K^T * scale), fp32 [B, H, nqb, nkb]."""
    _require_cuda("mean_pool_scores", q, k)
    B, H, Nq, D = (int(x) for x in q.shape)
    Nk = int(k.shape[2])
    if tuple(k.shape) != (B, H, Nk, D):
        raise ValueError(f"k shape {tuple(k.shape)} does not match q {tuple(q.shape)}")
    if q.dtype != k.dtype:
        raise TypeError("q and k must share a dtype")
    dt = _lib.dtype_code(q.dtype)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    qk, kk = _kernel_operand(_pad_head_dim(q)), _kernel_operand(_pad_head_dim(k))
    D = int(qk.shape[-1])
    L = _lib.lib()
    ws_bytes = int(L.sinkattn_mean_pool_workspace_bytes(B, H, Nq, Nk, D, int(block_size)))
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=q.device)
    out = torch.empty((B, H, _cdiv(Nq, block_size), _cdiv(Nk, block_size)), dtype=torch.float32,
                      device=q.device)
    with torch.cuda.device(q.device):
        _lib.check(
            L.sinkattn_mean_pool_scores(
                qk.data_ptr(), kk.data_ptr(), dt, B, H, Nq, Nk, D, _lib.strides4(qk),
                _lib.strides4(kk), int(block_size), float(scale), ws.data_ptr(), out.data_ptr(),
                _lib.stream_ptr(q.device),
            ),
            "mean_pool_scores",
        )
    return out


def coverage_mask(
    scores: torch.Tensor,
    coverage: float,
    keep_diagonal: bool,
    req_q: int = 0,
    req_k: int = 0,
    video_residual_text_blocks: Optional[int] = None,
    want_lists: bool = False,
):
    """Coverage mask of fp32 [H, nq, nk] scores (on the GPU).

    Returns the bool mask, or (mask, counts int32 [H, nq], idx int32 [H, nq, nk]) when
    want_lists is set.
    """
    _require_cuda("coverage_mask", scores)
    if scores.dim() != 3:
        raise ValueError(f"Expected [heads, blocks_q, blocks_k] scores, got {tuple(scores.shape)}")
    s = scores.float().contiguous()
    H, nq, nk = (int(x) for x in s.shape)
    mask = torch.empty((H, nq, nk), dtype=torch.bool, device=s.device)
    counts = torch.empty((H, nq), dtype=torch.int32, device=s.device) if want_lists else None
    idx = torch.empty((H, nq, nk), dtype=torch.int32, device=s.device) if want_lists else None
    mode = 0 if video_residual_text_blocks is None else 1
    tb = 0 if video_residual_text_blocks is None else int(video_residual_text_blocks)
    L = _lib.lib()
    ws = torch.empty(max(int(L.sinkattn_coverage_mask_workspace_bytes(H, nq)), 1), dtype=torch.uint8,
                     device=s.device)
    with torch.cuda.device(s.device):
        _lib.check(
            L.sinkattn_coverage_mask(
                s.data_ptr(), H, nq, nk, float(coverage), int(bool(keep_diagonal)), int(req_q),
                int(req_k), mode, tb, mask.data_ptr(), _lib.ptr(counts), _lib.ptr(idx),
                ws.data_ptr(), _lib.stream_ptr(s.device),
            ),
            "coverage_mask",
        )
    if want_lists:
        return mask, counts, idx
    return mask
