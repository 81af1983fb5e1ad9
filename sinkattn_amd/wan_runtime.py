"""Wan2.1 runtime of the sink-sparse path on this build's kernels.

Mirrors `wanx/runtime/sink_sparse_wan.py` (the module the reference's Wan pipeline
installs): the per-layer inner attention that owns a calibrated `[H, nqb, nkb]` sink
mask, the two diffusers attention processors (sparse inference and calibration) and the
two installers.  The attention math goes through `sinkattn_amd.sparse_attention`
(block-sparse HIP kernel, compensation branch, LSE mix), so a model patched with these
installers runs the MI355X kernels end to end.

QK-norm and rotary embedding are the model's own ops in front of the hot path: one
fused kernel (`ops.qk_norm_rotary`) for weighted RMSNorms and complex or (cos, sin)
tables, otherwise plain torch (the reference's fallback arithmetic,
`wanx/runtime/fast_misc.py:173-192,834-864`).
"""
from __future__ import annotations

from contextlib import nullcontext
from typing import Dict, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .sparse_attention import (
    SinkMaskCalibrator,
    SinkRuntimeState,
    SinkSparseConfig,
    _BLOCK_SPARSE_KERNEL_BLOCK_SIZE,
    _adapt_block_mask_for_kernel,
    _block_sparse_attn,
    _block_sparse_attn_with_compensation,
    _build_offline_required_mask,
    _ceil_div,
    _dense_short_attention,
    _dense_short_attention_with_lse,
    _device_cache_key,
    _fused_compensation_supported,
    _make_full_block_mask,
    _mean_pool_sequence_preserve_prefix,
    _mix_attention_outputs,
    load_sink_mask_package,
)

__all__ = [
    "WanSinkSparseInnerAttention",
    "WanSinkSparseAttnProcessor2_0",
    "WanSinkCalibrationProcessor2_0",
    "apply_qk_norm",
    "apply_rotary_qk",
    "set_sink_calibration_attn_wanx",
    "set_sink_sparse_attn_wanx",
]


# With adaptive mixing the sparse call, the pooled-K/V attention and the LSE mix run as
# one kernel (sparse tiles then the pooled tiles, with ln(sample_gap) added to the pooled
# logits).  False runs the reference's three separate steps on the GPU kernels instead.
FUSE_COMPENSATION = True


def _section(runtime_state: Optional[SinkRuntimeState], name: str):
    return runtime_state.time_section(name) if runtime_state is not None else nullcontext()


class WanSinkSparseInnerAttention(nn.Module):
    """`attn.inner_attention(q, k, v)` for one Wan layer (sink_sparse_wan.py:30-236).

    q, k, v are `[B, H, N, d]`.  The layer's mask `[H, nqb, nkb]` is widened once per
    (device, shape) to `mask | required | band` and expanded to the batch; the result
    is cached, so the kernel plan built from it is cached too (the plan cache keys on the
    mask tensor)."""

    def __init__(self, layer_idx: int, sink_mask: torch.Tensor, config: SinkSparseConfig,
                 runtime_state: Optional[SinkRuntimeState] = None):
        super().__init__()
        self.layer_idx = layer_idx
        self.config = config
        self.runtime_state = runtime_state
        self.register_buffer("sink_mask", sink_mask.bool().cpu())
        self._runtime_mask_cache: Dict[tuple, torch.Tensor] = {}
        self._kernel_runtime_mask_cache: Dict[tuple, torch.Tensor] = {}
        self._dynamic_mask_cache: Dict[tuple, torch.Tensor] = {}
        self._local_band_mask_cache: Dict[tuple, torch.Tensor] = {}

    # -- plan ------------------------------------------------------------------------------
    def _resolve_dynamic_plan(self) -> tuple[str, int]:
        """(mode, gap): the compensation branch is "none" or "pooled_kv"
        (sink_sparse_wan.py:48-58)."""
        mode = str(self.config.dynamic_mode).strip().lower()
        if mode not in ("none", "pooled_kv"):
            raise ValueError(
                "Unsupported Sink dynamic_mode. The maintained runtime only keeps the two-branch "
                f"compensation path: none | pooled_kv. Got: {self.config.dynamic_mode}")
        return mode, max(int(self.config.sample_gap), 1)

    # -- masks -----------------------------------------------------------------------------
    def _get_runtime_mask(self, sink_mask: torch.Tensor, mask_tag: str, batch_size: int,
                          num_heads: int, seq_len_q: int, seq_len_k: int,
                          device: torch.device) -> torch.Tensor:
        """`[B, H, nqb, nkb]` kernel mask = (sink | required) expanded to B, OR the local
        band, re-tiled to the kernel's 128 block (sink_sparse_wan.py:60-132)."""
        nqb = _ceil_div(seq_len_q, self.config.block_size)
        nkb = _ceil_div(seq_len_k, self.config.block_size)
        if tuple(sink_mask.shape) != (num_heads, nqb, nkb):
            raise ValueError(
                "Sink mask shape does not match runtime sequence layout. "
                f"Expected [{num_heads}, {nqb}, {nkb}], got {list(sink_mask.shape)}. "
                "Re-calibrate the mask for this Wan setup.")
        dkey = _device_cache_key(device)
        key = (mask_tag, dkey, batch_size, num_heads, seq_len_q, seq_len_k)
        base = self._runtime_mask_cache.get(key)
        if base is None or base.device != device:
            m = sink_mask.to(device=device)
            required = _build_offline_required_mask(num_query_blocks=nqb, num_key_blocks=nkb,
                                                    config=self.config, device=device)
            if required is not None:
                m = m | required.unsqueeze(0)
            base = m.unsqueeze(0).expand(batch_size, num_heads, nqb, nkb).contiguous()
            self._runtime_mask_cache[key] = base

        band = self._get_runtime_local_band_mask(batch_size=batch_size, num_heads=num_heads,
                                                 seq_len_q=seq_len_q, seq_len_k=seq_len_k,
                                                 device=device)
        kkey = key + (int(self.config.block_size),)
        kmask = self._kernel_runtime_mask_cache.get(kkey)
        if kmask is None or kmask.device != device:
            src = base if band is None else (base | band).contiguous()
            kmask = _adapt_block_mask_for_kernel(src, source_block_size=int(self.config.block_size),
                                                 seq_len_q=seq_len_q, seq_len_k=seq_len_k)
            self._kernel_runtime_mask_cache[kkey] = kmask
        return kmask

    def _get_dynamic_mask(self, batch_size: int, num_heads: int, seq_len_q: int, seq_len_k: int,
                          device: torch.device) -> torch.Tensor:
        """All-true kernel mask for the compensation branch run through the sparse kernel
        (sink_sparse_wan.py:134-153)."""
        key = (_device_cache_key(device), batch_size, num_heads, seq_len_q, seq_len_k)
        m = self._dynamic_mask_cache.get(key)
        if m is None or m.device != device:
            m = _make_full_block_mask(batch_size=batch_size, num_heads=num_heads, seq_len_q=seq_len_q,
                                      seq_len_k=seq_len_k, block_size=_BLOCK_SPARSE_KERNEL_BLOCK_SIZE,
                                      device=device)
            self._dynamic_mask_cache[key] = m
        return m

    def _get_runtime_local_band_mask(self, batch_size: int, num_heads: int, seq_len_q: int,
                                     seq_len_k: int, device: torch.device) -> Optional[torch.Tensor]:
        """|qb - kb| <= runtime_diagonal_band_width, or None for width 0
        (sink_sparse_wan.py:155-178)."""
        width = max(int(self.config.runtime_diagonal_band_width), 0)
        if width <= 0:
            return None
        nqb = _ceil_div(seq_len_q, self.config.block_size)
        nkb = _ceil_div(seq_len_k, self.config.block_size)
        key = (_device_cache_key(device), batch_size, num_heads, nqb, nkb, width)
        m = self._local_band_mask_cache.get(key)
        if m is None or m.device != device:
            dist = (torch.arange(nqb, device=device)[:, None] - torch.arange(nkb, device=device)[None, :]).abs()
            m = (dist <= width).view(1, 1, nqb, nkb)
            if batch_size != 1 or num_heads != 1:
                m = m.expand(batch_size, num_heads, nqb, nkb).contiguous()
            self._local_band_mask_cache[key] = m
        return m

    # -- call ------------------------------------------------------------------------------
    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """Sparse main branch, then (pooled_kv) the compensation branch over K/V mean-pooled
        by `sample_gap` and the LSE mix (sink_sparse_wan.py:180-282)."""
        rs = self.runtime_state
        with _section(rs, "inner_total"):
            with _section(rs, "mask_prepare"):
                tag = "__base__"
                mode, gap = self._resolve_dynamic_plan()
                mask = self._get_runtime_mask(sink_mask=self.sink_mask, mask_tag=tag, batch_size=q.size(0),
                                              num_heads=q.size(1), seq_len_q=q.size(2), seq_len_k=k.size(2),
                                              device=q.device)
            dyn_len = None
            if mode == "none":
                with _section(rs, "sparse_main"):
                    out, _ = _block_sparse_attn(q, k, v, mask, return_lse=False)
            elif (self.config.mixing_mode == "adaptive" and FUSE_COMPENSATION
                  and _fused_compensation_supported(q, k, v)):
                with _section(rs, "comp_pool"):
                    prefix = max(int(self.config.text_length), 0)
                    k_dyn = ops.mean_pool_tokens(k, gap, prefix, like=k)
                    v_dyn = ops.mean_pool_tokens(v, gap, prefix, like=v)
                    dyn_len = int(k_dyn.size(2))
                with _section(rs, "sparse_main"):  # sparse + compensation + mix
                    out = _block_sparse_attn_with_compensation(q, k, v, mask, k_dyn, v_dyn, gap)
            else:
                adaptive = self.config.mixing_mode == "adaptive"
                with _section(rs, "sparse_main"):
                    sink_out, sink_lse = _block_sparse_attn(q, k, v, mask, return_lse=adaptive)
                with _section(rs, "comp_pool"):
                    prefix = max(int(self.config.text_length), 0)
                    k_dyn = _mean_pool_sequence_preserve_prefix(k, gap, prefix_tokens=prefix)
                    v_dyn = _mean_pool_sequence_preserve_prefix(v, gap, prefix_tokens=prefix)
                    dyn_len = int(k_dyn.size(2))
                with _section(rs, "comp_attn"):
                    kernel = self.config.dynamic_kernel
                    if kernel == "dense" or (kernel == "auto" and not adaptive):
                        if adaptive:
                            dyn_out, dyn_lse = _dense_short_attention_with_lse(q, k_dyn, v_dyn)
                        else:
                            dyn_out, dyn_lse = _dense_short_attention(q, k_dyn, v_dyn), None
                    else:
                        full = self._get_dynamic_mask(batch_size=q.size(0), num_heads=q.size(1),
                                                      seq_len_q=q.size(2), seq_len_k=dyn_len, device=q.device)
                        dyn_out, dyn_lse = _block_sparse_attn(q, k_dyn, v_dyn, full, return_lse=adaptive)
                with _section(rs, "mix"):
                    out = _mix_attention_outputs(sink_out=sink_out, sink_lse=sink_lse, dynamic_out=dyn_out,
                                                 dynamic_lse=dyn_lse, config=self.config, dynamic_sample_gap=gap)
            if rs is not None:
                with rs.time_section("stats"):
                    rs.record_mask_stats(layer_idx=self.layer_idx, sink_mask_tag=tag, dynamic_mode=mode,
                                         dynamic_sample_gap=gap, base_runtime_mask=mask, topup_mask=None,
                                         dynamic_seq_len_k=dyn_len, total_seq_len_k=int(k.size(2)))
            return out


# -- the model's own ops around the hot path ---------------------------------------------
def apply_qk_norm(attn, query: torch.Tensor, key: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """`attn.norm_q` / `attn.norm_k` when present (fast_misc.py:834-864, module path)."""
    nq = getattr(attn, "norm_q", None)
    nk = getattr(attn, "norm_k", None)
    return (query if nq is None else nq(query)), (key if nk is None else nk(key))


def _rotary_tables(freqs, hidden_states: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, bool]:
    """(cos, sin, interleaved_tuple): complex tensors give (real, imag) per pair; Wan's
    (cos, sin) tuple form holds per-channel tables `[1, L, 1, D]` (fast_misc.py:135-170)."""
    if isinstance(freqs, (tuple, list)) and len(freqs) == 2:
        cos, sin = freqs
        if hidden_states.ndim != 4 or cos.ndim != 4 or sin.ndim != 4:
            raise TypeError("Wan tuple rotary expects hidden_states [B, L/H, H/L, D] and freqs [1, L, 1, D].")
        if hidden_states.shape[1] != cos.shape[1]:
            if hidden_states.shape[2] != cos.shape[1]:
                raise ValueError(f"Cannot align Wan tuple rotary freqs {tuple(cos.shape)} "
                                 f"with hidden states {tuple(hidden_states.shape)}.")
            cos, sin = cos.transpose(1, 2), sin.transpose(1, 2)
        return cos[..., 0::2].float(), sin[..., 1::2].float(), True
    if isinstance(freqs, torch.Tensor) and torch.is_complex(freqs):
        return freqs.real.float(), freqs.imag.float(), False
    raise TypeError(f"Unsupported rotary embedding type: {type(freqs)!r}")


def _rotate(hidden_states: torch.Tensor, freqs) -> torch.Tensor:
    cos, sin, _ = _rotary_tables(freqs, hidden_states)
    pairs = hidden_states.float().unflatten(-1, (-1, 2))
    x1, x2 = pairs[..., 0], pairs[..., 1]
    out = torch.stack((x1 * cos - x2 * sin, x1 * sin + x2 * cos), dim=-1)
    return out.flatten(-2).to(hidden_states.dtype)


def apply_rotary_qk(query: torch.Tensor, key: torch.Tensor, freqs) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate adjacent channel pairs of q and k by the per-position angles in `freqs`
    (fp32 arithmetic, result in the input dtype; fast_misc.py:182-192,216-234)."""
    if freqs is None:
        return query, key
    return _rotate(query, freqs), _rotate(key, freqs)


# QK-norm + rotary as one kernel (sinkattn_qk_norm_rotary) whenever the layer's norms are
# weighted RMSNorms and the rotary table is given as complex values or (cos, sin).
FUSE_QK_PREP = True


def rms_norm_params(norm) -> Optional[tuple]:
    """(weight, eps) of a norm module the fused kernel restates: a weight, a numeric eps,
    no bias and not a LayerNorm (the same test as fast_misc.py:839-852), else None."""
    if norm is None:
        return None
    w, eps = getattr(norm, "weight", None), getattr(norm, "eps", None)
    if w is None or eps is None or getattr(norm, "bias", None) is not None:
        return None
    if "layernorm" in type(norm).__name__.lower():
        return None
    return w, float(eps)


def rotary_tables_2d(freqs, n: int, head_dim: int) -> Optional[tuple]:
    """(real, imag) fp32 [rows, head_dim/2] of a complex table or of Wan's (cos, sin)
    per-channel tables, or None for any other form."""
    half = head_dim // 2
    if isinstance(freqs, torch.Tensor) and torch.is_complex(freqs):
        if freqs.numel() % half != 0:
            return None
        return freqs.real.reshape(-1, half), freqs.imag.reshape(-1, half)
    if isinstance(freqs, (tuple, list)) and len(freqs) == 2:
        cos, sin = freqs
        if cos.dim() != 4 or cos.size(-1) != head_dim:
            return None
        if cos.size(1) == n:  # [1, N, 1, D]
            cos, sin = cos[0, :, 0], sin[0, :, 0]
        elif cos.size(2) == n:  # [1, 1, N, D]
            cos, sin = cos[0, 0], sin[0, 0]
        else:
            return None
        return cos[..., 0::2].reshape(-1, half), sin[..., 1::2].reshape(-1, half)
    return None


def _fused_qk_prep(attn, query: torch.Tensor, key: torch.Tensor, rotary_emb):
    """Q/K `[B, N, C]` after norm and rotary from one kernel, or None when the layer does
    not fit it (the torch path then runs)."""
    if not (FUSE_QK_PREP and query.is_cuda and query.dim() == 3 and query.shape == key.shape
            and query.dtype in (torch.bfloat16, torch.float16) and key.dtype == query.dtype):
        return None
    pq, pk = rms_norm_params(getattr(attn, "norm_q", None)), rms_norm_params(getattr(attn, "norm_k", None))
    if pq is None or pk is None:
        return None
    C = int(query.size(-1))
    if C % int(attn.heads) != 0 or pq[0].numel() != C or pk[0].numel() != C:
        return None
    D = C // int(attn.heads)
    tables = None
    if rotary_emb is not None:
        tables = rotary_tables_2d(rotary_emb, int(query.size(1)), D)
        if tables is None or tables[0].size(0) != int(query.size(1)):
            return None
    fr, fi = tables if tables is not None else (None, None)
    return ops.qk_norm_rotary(query, key, pq[0], pk[0], pq[1], pk[1], D, fr, fi, rows_per_pos=1)


def _prepare_attention_tensors(attn, hidden_states: torch.Tensor,
                               encoder_hidden_states: Optional[torch.Tensor] = None,
                               rotary_emb=None):
    """Projections, QK-norm, head split to `[B, H, N, d]` and rotary; the first 257 context
    tokens feed the image branch when the layer has one (sink_sparse_wan.py:285-315)."""
    timing = getattr(getattr(attn, "inner_attention", None), "timing", None)
    img_ctx = None
    if attn.add_k_proj is not None and encoder_hidden_states is not None:
        img_ctx = encoder_hidden_states[:, :257]
        encoder_hidden_states = encoder_hidden_states[:, 257:]
    if encoder_hidden_states is None:
        encoder_hidden_states = hidden_states
    query = attn.to_q(hidden_states)
    key = attn.to_k(encoder_hidden_states)
    value = attn.to_v(encoder_hidden_states)
    on = timing is not None and getattr(timing, "is_enabled", False)
    with (timing.section("qk_prep") if on else nullcontext()):
        fused = _fused_qk_prep(attn, query, key, rotary_emb)
    if fused is not None:
        query, key, value = (t.unflatten(2, (attn.heads, -1)).transpose(1, 2) for t in (*fused, value))
        return query, key, value, img_ctx
    with (timing.section("qk_norm") if on else nullcontext()):
        query, key = apply_qk_norm(attn, query, key)
    query, key, value = (t.unflatten(2, (attn.heads, -1)).transpose(1, 2) for t in (query, key, value))
    if rotary_emb is not None:
        with (timing.section("rotary_apply") if on else nullcontext()):
            query, key = apply_rotary_qk(query, key, rotary_emb)
    return query, key, value, img_ctx


def _compute_image_branch(attn, query: torch.Tensor, img_ctx: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """I2V image-context attention (dense SDPA over 257 tokens; sink_sparse_wan.py:318-339)."""
    if img_ctx is None:
        return None
    k_img = attn.norm_added_k(attn.add_k_proj(img_ctx)).unflatten(2, (attn.heads, -1)).transpose(1, 2)
    v_img = attn.add_v_proj(img_ctx).unflatten(2, (attn.heads, -1)).transpose(1, 2)
    out = F.scaled_dot_product_attention(query, k_img, v_img, attn_mask=None, dropout_p=0.0, is_causal=False)
    return out.transpose(1, 2).flatten(2, 3).type_as(query)


class WanSinkSparseAttnProcessor2_0:
    """Self-attention processor that routes through `attn.inner_attention`
    (sink_sparse_wan.py:342-386)."""

    def __init__(self, layer_idx: int, runtime_state: Optional[SinkRuntimeState] = None):
        if not hasattr(F, "scaled_dot_product_attention"):
            raise ImportError("WanSinkSparseAttnProcessor2_0 requires PyTorch 2.0+.")
        self.layer_idx = layer_idx
        self.runtime_state = runtime_state

    def __call__(self, attn, hidden_states: torch.Tensor, encoder_hidden_states: Optional[torch.Tensor] = None,
                 attention_mask: Optional[torch.Tensor] = None, rotary_emb=None) -> torch.Tensor:
        del attention_mask
        if self.runtime_state is not None:
            self.runtime_state.enter_layer(self.layer_idx)
        q, k, v, img_ctx = _prepare_attention_tensors(attn, hidden_states, encoder_hidden_states, rotary_emb)
        img = _compute_image_branch(attn, q, img_ctx)
        out = attn.inner_attention(q, k, v).transpose(1, 2).flatten(2, 3).type_as(q)
        if img is not None:
            out = out + img
        return attn.to_out[1](attn.to_out[0](out))


class WanSinkCalibrationProcessor2_0:
    """Dense processor that records every call's Q/K/V block scores in a calibrator
    (sink_sparse_wan.py:389-429)."""

    def __init__(self, calibrator: SinkMaskCalibrator, layer_idx: int):
        if not hasattr(F, "scaled_dot_product_attention"):
            raise ImportError("WanSinkCalibrationProcessor2_0 requires PyTorch 2.0+.")
        self.calibrator = calibrator
        self.layer_idx = layer_idx

    def __call__(self, attn, hidden_states: torch.Tensor, encoder_hidden_states: Optional[torch.Tensor] = None,
                 attention_mask: Optional[torch.Tensor] = None, rotary_emb=None) -> torch.Tensor:
        del attention_mask
        q, k, v, img_ctx = _prepare_attention_tensors(attn, hidden_states, encoder_hidden_states, rotary_emb)
        self.calibrator.record(self.layer_idx, q, k, v)
        img = _compute_image_branch(attn, q, img_ctx)
        out = F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=False)
        out = out.transpose(1, 2).flatten(2, 3).type_as(q)
        if img is not None:
            out = out + img
        return attn.to_out[1](attn.to_out[0](out))


def set_sink_calibration_attn_wanx(model, calibrator: SinkMaskCalibrator, verbose: bool = False) -> SinkMaskCalibrator:
    """Install the calibration processor on every `model.blocks[i].attn1`
    (sink_sparse_wan.py:432-439)."""
    for i, block in enumerate(model.blocks):
        attn = block.attn1
        attn.verbose = verbose
        previous = attn.get_processor()
        attn.set_processor(WanSinkCalibrationProcessor2_0(calibrator=calibrator, layer_idx=i))
        if not hasattr(attn, "origin_processor"):
            attn.origin_processor = previous
    return calibrator


def set_sink_sparse_attn_wanx(model, sink_mask_path: str, config_overrides: Optional[dict] = None,
                              verbose: bool = False) -> dict:
    """Load a v3 mask package and install the sparse processor plus a per-layer
    inner attention on every `model.blocks[i].attn1` (sink_sparse_wan.py:442-466)."""
    package = load_sink_mask_package(sink_mask_path)
    config = SinkSparseConfig.from_dict(package.get("config")).merged(config_overrides)
    masks = package.get("sink_masks", {})
    state = SinkRuntimeState()
    model._sink_runtime_state = state
    for i, block in enumerate(model.blocks):
        if str(i) not in masks:
            raise KeyError(f"Layer {i} does not exist in sink mask package: {sink_mask_path}")
        attn = block.attn1
        attn.verbose = verbose
        attn.inner_attention = WanSinkSparseInnerAttention(layer_idx=i, sink_mask=masks[str(i)], config=config,
                                                           runtime_state=state)
        previous = attn.get_processor()
        attn.set_processor(WanSinkSparseAttnProcessor2_0(layer_idx=i, runtime_state=state))
        if not hasattr(attn, "origin_processor"):
            attn.origin_processor = previous
    return {"config": config, "num_layers": len(model.blocks), "mask_path": sink_mask_path}
