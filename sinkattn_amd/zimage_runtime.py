"""Z-Image runtime of the sink-sparse path on this build's kernels.

Mirrors `zimg/runtime/sink_sparse_zimage.py`: the fixed image-prefix / text-suffix block
layout, the calibrator that aligns each call's `[H, n, n]` block scores into that layout
and counts how often each cell was observed, the static sink processor (per-sample
block-sparse call with the text rows and columns forced dense, optional compensation
branch), and the installers.  Attention math goes through `sinkattn_amd.sparse_attention`.

Layout: a sequence is `image_tokens` (token_width*token_height*token_depth padded to 32)
followed by up to `text_length` (padded to 32) text tokens.  In block space the calibrated
map is `[H, T, T]` with T = image_blocks + max_text_blocks; a call with `c` text blocks
uses the image blocks and the LAST `c` blocks of that layout (text is right-aligned).
"""
from __future__ import annotations

from contextlib import nullcontext
from dataclasses import asdict
from pathlib import Path
from typing import Any, Dict, Optional

import torch
import torch.nn.functional as F

from . import ops
from .sparse_attention import (
    SinkRuntimeState,
    SinkSparseConfig,
    _block_sparse_attn,
    _block_sparse_attn_with_compensation,
    _build_direct_mean_coverage_mask,
    _build_direct_mean_coverage_masks,
    _device_package_groups,
    _ceil_div,
    _compute_block_scores,
    _dense_short_attention_with_lse,
    _device_cache_key,
    _fused_compensation_supported,
    _mean_pool_sequence,
    _mix_attention_outputs,
    _to_host,
    load_sink_mask_package,
)

SEQ_MULTI_OF = 32
DEFAULT_TEXT_LENGTH = 512

# Image rows run sparse attention, the pooled-K/V attention and the LSE mix as one kernel
# when the image prefix is a whole number of 128-token blocks; False keeps the
# reference's three separate steps (on the GPU kernels).
FUSE_COMPENSATION = True

__all__ = [
    "DEFAULT_TEXT_LENGTH",
    "SinkRuntimeState",
    "SinkSparseConfig",
    "ZImageSinkMaskCalibrator",
    "ZImageSinkCalibrationProcessor",
    "ZImageStaticSinkProcessor",
    "apply_zimage_rotary_emb",
    "build_zimg_sink_config",
    "infer_zimg_token_layout",
    "prepare_zimage_attention_tensors",
    "reset_sink_runtime_state_zimage",
    "set_sink_calibration_attn_zimage",
    "set_sink_sparse_attn_zimage",
]


def _pad_len_to_multiple(value: int, multiple: int = SEQ_MULTI_OF) -> int:
    return _ceil_div(int(value), int(multiple)) * int(multiple)


def infer_zimg_token_layout(*, height: int, width: int) -> tuple[int, int, int]:
    """(token_width, token_height, token_depth) for an image of height x width pixels
    (16-pixel patches, one frame; sink_sparse_zimage.py:38-42)."""
    return max(int(width) // 16, 1), max(int(height) // 16, 1), 1


def build_zimg_sink_config(*, package_config: Optional[dict] = None,
                           config_overrides: Optional[dict] = None) -> SinkSparseConfig:
    """Z-Image defaults (one frame, no band, text forced global, text_length 512) under the
    package's config and then the overrides (None values ignored at each layer).  Only
    dynamic_mode none|pooled_kv and mixing_mode adaptive are accepted
    (sink_sparse_zimage.py:45-81)."""
    data = asdict(SinkSparseConfig())
    data.update(token_depth=1, dynamic_mode="none", runtime_diagonal_band_width=0,
                force_text_global_attention=True, text_length=DEFAULT_TEXT_LENGTH)
    for layer in (package_config, config_overrides):
        if layer:
            data.update({k: v for k, v in layer.items() if v is not None})
    config = SinkSparseConfig.from_dict(data)
    config.force_text_global_attention = True
    if str(config.dynamic_mode).strip().lower() not in ("none", "pooled_kv"):
        raise ValueError("Unsupported Z-Image Sink dynamic_mode. "
                         f"Expected one of: none, pooled_kv. Got: {config.dynamic_mode}")
    if str(config.mixing_mode).strip().lower() != "adaptive":
        raise ValueError(f"Unsupported Z-Image Sink mixing_mode. Expected adaptive. Got: {config.mixing_mode}")
    config.dynamic_kernel = str(config.dynamic_kernel or "auto").strip().lower()
    return config


def _resolve_negative_indices(raw: Optional[list], total: Optional[int]) -> set[int]:
    """Non-negative entries as given; negative ones count from `total` and are dropped
    when `total` is unknown (sink_sparse_zimage.py:84-119)."""
    out: set[int] = set()
    for r in raw or ():
        val = int(r)
        if val < 0:
            if total is None:
                continue
            val += int(total)
        if val >= 0:
            out.add(val)
    return out


def _resolve_forced_dense_step_list(config: SinkSparseConfig, runtime_state: Optional[SinkRuntimeState]) -> set[int]:
    total = None if runtime_state is None else runtime_state.total_steps
    return _resolve_negative_indices(config.force_dense_steps, total)


def _resolve_forced_dense_layer_list(config: SinkSparseConfig, *, total_layers: Optional[int] = None) -> set[int]:
    return _resolve_negative_indices(config.force_dense_layers, total_layers)


def _image_token_count(config: SinkSparseConfig) -> int:
    return _pad_len_to_multiple(int(config.token_width) * int(config.token_height) * int(config.token_depth))


def _max_text_token_count(config: SinkSparseConfig) -> int:
    return _pad_len_to_multiple(int(config.text_length))


def _fixed_block_shape(config: SinkSparseConfig) -> tuple[int, int, int]:
    """(image_tokens, image_blocks, total_blocks) of the calibrated layout."""
    image_tokens = _image_token_count(config)
    image_blocks = _ceil_div(image_tokens, int(config.block_size))
    return image_tokens, image_blocks, image_blocks + _ceil_div(_max_text_token_count(config), int(config.block_size))


def _suffix_block_index(image_blocks: int, current_text_blocks: int, total_blocks: int,
                        device: torch.device) -> torch.Tensor:
    """Layout index of each block of a call: image blocks in place, the call's text blocks
    at the end of the layout."""
    img = torch.arange(image_blocks, device=device)
    if current_text_blocks <= 0:
        return img
    return torch.cat([img, torch.arange(total_blocks - current_text_blocks, total_blocks, device=device)])


def _align_scores_image_text_suffix(scores: torch.Tensor, *, image_blocks: int, current_text_blocks: int,
                                    total_blocks: int) -> torch.Tensor:
    """Scatter a call's `[H, n, n]` scores (n = image + current text blocks) into the
    `[H, T, T]` layout, zeros elsewhere (sink_sparse_zimage.py:136-163)."""
    if scores.dim() != 3:
        raise ValueError(f"Expected [heads, blocks_q, blocks_k] scores, got {tuple(scores.shape)}")
    n = image_blocks + current_text_blocks
    if scores.size(1) != n or scores.size(2) != n:
        raise ValueError("Unexpected Z-Image block score shape. "
                         f"Expected {n}x{n}, got {scores.size(1)}x{scores.size(2)}.")
    idx = _suffix_block_index(image_blocks, current_text_blocks, total_blocks, scores.device)
    out = scores.new_zeros(scores.size(0), total_blocks, total_blocks)
    out[:, idx[:, None], idx[None, :]] = scores
    return out


def _alignment_presence_mask(*, num_heads: int, image_blocks: int, current_text_blocks: int, total_blocks: int,
                             device: torch.device) -> torch.Tensor:
    """fp32 `[H, T, T]`, 1 where `_align_scores_image_text_suffix` wrote a score
    (sink_sparse_zimage.py:166-182)."""
    idx = _suffix_block_index(image_blocks, current_text_blocks, total_blocks, device)
    mask = torch.zeros(num_heads, total_blocks, total_blocks, dtype=torch.float32, device=device)
    mask[:, idx[:, None], idx[None, :]] = 1.0
    return mask


def _slice_runtime_sink_mask(sink_mask: torch.Tensor, *, image_blocks: int, current_text_blocks: int,
                             total_blocks: int) -> torch.Tensor:
    """The `[H, n, n]` sub-mask of a call with `current_text_blocks` text blocks
    (sink_sparse_zimage.py:185-208)."""
    if sink_mask.dim() != 3:
        raise ValueError(f"Expected [heads, blocks_q, blocks_k] sink mask, got {tuple(sink_mask.shape)}")
    if sink_mask.size(1) != total_blocks or sink_mask.size(2) != total_blocks:
        raise ValueError("Z-Image sink mask shape does not match the calibrated fixed block layout. "
                         f"Expected {total_blocks}x{total_blocks}, got {sink_mask.size(1)}x{sink_mask.size(2)}.")
    if current_text_blocks <= 0:
        return sink_mask[:, :image_blocks, :image_blocks].contiguous()
    idx = _suffix_block_index(image_blocks, current_text_blocks, total_blocks, sink_mask.device)
    return sink_mask.index_select(1, idx).index_select(2, idx).contiguous()


def _force_text_dense_runtime_mask(runtime_mask: torch.Tensor, *, image_blocks: int,
                                   current_text_blocks: int) -> torch.Tensor:
    """Text rows and text columns all True (a copy; sink_sparse_zimage.py:211-222)."""
    if current_text_blocks <= 0:
        return runtime_mask
    out = runtime_mask.clone()
    out[..., :, int(image_blocks):] = True
    out[..., int(image_blocks):, :] = True
    return out


def _dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    return F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=False)


# -- the model's own ops in front of the hot path ------------------------------------------
def apply_zimage_rotary_emb(x_in: torch.Tensor, freqs_cis: torch.Tensor) -> torch.Tensor:
    """Rotate channel pairs of `[B, N, H, d]` by complex `freqs_cis` `[B, N, d/2]`, fp32
    math, result in the input dtype (zimg/runtime/modify_zimage.py:8-13)."""
    pairs = x_in.float().unflatten(-1, (-1, 2))
    f = freqs_cis.unsqueeze(2)
    c, s = f.real.float(), f.imag.float()
    x1, x2 = pairs[..., 0], pairs[..., 1]
    return torch.stack((x1 * c - x2 * s, x1 * s + x2 * c), dim=-1).flatten(-2).type_as(x_in)


# Per-head QK-norm + rotary as one kernel when both norms are weighted RMSNorms.
FUSE_QK_PREP = True


def _fused_qk_prep(attn: Any, q: torch.Tensor, k: torch.Tensor, freqs_cis: Optional[torch.Tensor]):
    """q, k `[B, N, H, d]` normed and rotated by `ops.qk_norm_rotary` (rows = B*N*H of d
    channels, one table row per (b, n) position), or None when the layer does not fit."""
    from .wan_runtime import rms_norm_params
    if not (FUSE_QK_PREP and q.is_cuda and q.dtype in (torch.bfloat16, torch.float16) and q.dim() == 4):
        return None
    pq, pk = rms_norm_params(attn.norm_q), rms_norm_params(attn.norm_k)
    D = int(q.size(-1))
    if pq is None or pk is None or pq[0].numel() != D or pk[0].numel() != D:
        return None
    fr = fi = None
    if freqs_cis is not None:
        if not torch.is_complex(freqs_cis) or freqs_cis.size(-1) != D // 2:
            return None
        f = freqs_cis.reshape(-1, D // 2)
        B, N = int(q.size(0)), int(q.size(1))
        if f.size(0) not in (N, B * N):
            return None
        fr, fi = f.real, f.imag
    return ops.qk_norm_rotary(q, k, pq[0], pk[0], pq[1], pk[1], D, fr, fi, rows_per_pos=int(q.size(2)))


def prepare_zimage_attention_tensors(attn: Any, hidden_states: torch.Tensor, *,
                                     freqs_cis: Optional[torch.Tensor] = None):
    """Q/K/V `[B, N, H, d]`: projections, head split, optional norms and rotary, all cast
    to V's dtype (zimg/runtime/modify_zimage.py:16-43); norm + rotary as one kernel when
    the layer fits it."""
    q, k, v = (proj(hidden_states).unflatten(-1, (attn.heads, -1)) for proj in (attn.to_q, attn.to_k, attn.to_v))
    fused = _fused_qk_prep(attn, q, k, freqs_cis) if q.dtype == v.dtype else None
    if fused is not None:
        return fused[0], fused[1], v
    if attn.norm_q is not None:
        q = attn.norm_q(q)
    if attn.norm_k is not None:
        k = attn.norm_k(k)
    if freqs_cis is not None:
        q = apply_zimage_rotary_emb(q, freqs_cis)
        k = apply_zimage_rotary_emb(k, freqs_cis)
    return q.to(v.dtype), k.to(v.dtype), v


# -- calibration (a5, Z-Image) -------------------------------------------------------------
class ZImageSinkMaskCalibrator:
    """Per-layer sums of aligned scores, of their squares and of the presence mask; the
    package's mean/std divide by presence (clamped to 1), so cells a call never covered
    do not dilute the mean (sink_sparse_zimage.py:248-366).  The sums live on the device
    the scores come from (no per-call host copy); the package holds host tensors."""

    def __init__(self, config: SinkSparseConfig):
        self.config = build_zimg_sink_config(package_config=asdict(config))
        self.current_step = -1
        self.score_sums: Dict[int, torch.Tensor] = {}
        self.score_sq_sums: Dict[int, torch.Tensor] = {}
        self.score_presence_sums: Dict[int, torch.Tensor] = {}
        self.score_counts: Dict[int, int] = {}
        self.image_token_count, self.image_blocks, self.total_blocks = _fixed_block_shape(self.config)
        self.max_text_tokens = _max_text_token_count(self.config)

    def reset_generation(self) -> None:
        self.current_step = -1

    # The per-layer sums (and presence counts) stay on the scores' device unless this is set:
    # 3 x 4 bytes x heads x blocks^2 per layer while calibrating; True copies each call's
    # aligned scores to the host first, as the reference does (one sync per call).  The
    # package is bit-identical either way.
    accumulate_on_host: bool = False

    def _accumulate(self, *, layer_idx: int, scores: torch.Tensor, presence: torch.Tensor) -> None:
        if self.accumulate_on_host:
            scores, presence = scores.cpu(), presence.cpu()
        if layer_idx not in self.score_sums:
            self.score_sums[layer_idx] = scores
            self.score_sq_sums[layer_idx] = scores.square()
            self.score_presence_sums[layer_idx] = presence
            self.score_counts[layer_idx] = 1
            return
        self.score_sums[layer_idx] += scores
        self.score_sq_sums[layer_idx] += scores.square()
        self.score_presence_sums[layer_idx] += presence
        self.score_counts[layer_idx] += 1

    @torch.no_grad()
    def record(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
               text_token_count: int) -> None:
        """One sample `[1, H, n_tokens, d]`: block scores on the GPU kernels, then the
        alignment and accumulation on the host in fp32."""
        if layer_idx == 0:
            self.current_step += 1
        if text_token_count < 0:
            raise ValueError(f"Invalid Z-Image text token count: {text_token_count}")
        if text_token_count > self.max_text_tokens:
            raise ValueError("Observed Z-Image text token count exceeds calibrated maximum. "
                             f"Observed {text_token_count}, configured max {self.max_text_tokens}.")
        samples = _compute_block_scores(q, k, v, self.config).detach().float()
        if samples.size(0) != 1:
            raise ValueError("Z-Image calibration expects one sample at a time after valid-token slicing.")
        # stays on the scores' device: alignment and accumulation are copies and
        # elementwise fp32 adds, identical to the reference's host accumulation
        scores = samples.mean(dim=0)
        text_blocks = _ceil_div(int(text_token_count), int(self.config.block_size))
        aligned = _align_scores_image_text_suffix(scores, image_blocks=self.image_blocks,
                                                  current_text_blocks=text_blocks, total_blocks=self.total_blocks)
        presence = _alignment_presence_mask(num_heads=int(aligned.size(0)), image_blocks=self.image_blocks,
                                            current_text_blocks=text_blocks, total_blocks=self.total_blocks,
                                            device=aligned.device)
        self._accumulate(layer_idx=layer_idx, scores=aligned, presence=presence)

    def build_package(self, include_scores: bool = True, config_override: Optional[SinkSparseConfig] = None) -> dict:
        cfg = self.config if config_override is None else build_zimg_sink_config(package_config=asdict(config_override))
        means, stds, masks, counts = {}, {}, {}, {}
        layers = sorted(self.score_sums)
        if not layers:
            pass
        elif all(self.score_sums[i].is_cuda and self.score_sums[i].shape == self.score_sums[layers[0]].shape
                 and self.score_sums[i].device == self.score_sums[layers[0]].device for i in layers):
            # mean and std on the device in groups of layers (elementwise IEEE divisions by the
            # presence counts, as the reference's host math); the masks are built from the
            # device means and only what the package holds comes to the host
            mask_list, mean_list, std_list = _device_package_groups(
                [self.score_sums[i] for i in layers], [self.score_sq_sums[i] for i in layers],
                [self.score_presence_sums[i] for i in layers], cfg, include_scores, denom_min=1.0)
            for j, layer in enumerate(layers):
                key = str(layer)
                if include_scores:
                    means[key] = mean_list[j]
                    stds[key] = std_list[j]
                masks[key] = mask_list[j]
                counts[key] = int(self.score_counts[layer])
        else:
            # sums on the host (accumulate_on_host, or mixed shapes): the reference's host math
            pres = _to_host([self.score_presence_sums[i] for i in layers])
            sums = _to_host([self.score_sums[i] for i in layers])
            sq_sums = _to_host([self.score_sq_sums[i] for i in layers])
            for j, layer in enumerate(layers):
                key = str(layer)
                presence = pres[j].clamp_min(1.0)
                mean = sums[j] / presence
                var = (sq_sums[j] / presence - mean.square()).clamp_min_(0.0)
                means[key] = mean
                stds[key] = torch.sqrt(var)
                counts[key] = int(self.score_counts[layer])
            for layer, m in zip(layers, _build_direct_mean_coverage_masks([means[str(i)] for i in layers], cfg)):
                masks[str(layer)] = m.cpu()
        return {
            "version": 3,
            "config": asdict(cfg),
            "mean_scores": means if include_scores else {},
            "std_scores": stds if include_scores else {},
            "sink_masks": masks,
            "counts": counts,
            "meta": {"route": "zimg_static_only", "text_layout": "image_prefix_text_suffix_aligned",
                     "image_token_count": self.image_token_count, "max_text_token_count": self.max_text_tokens,
                     "total_blocks": self.total_blocks},
        }

    def save(self, output_path: str, include_scores: bool = True,
             config_override: Optional[SinkSparseConfig] = None) -> dict:
        package = self.build_package(include_scores=include_scores, config_override=config_override)
        path = Path(output_path)
        path.parent.mkdir(parents=True, exist_ok=True)
        torch.save(package, path)
        return package


def _valid_lengths(attention_mask: Optional[torch.Tensor], batch_size: int, seq_len: int) -> list[int]:
    if attention_mask is None:
        return [seq_len] * batch_size
    return [int(m.sum().item()) for m in attention_mask]


def _sample_bhsd(t: torch.Tensor, b: int, n: int) -> torch.Tensor:
    """Sample b's first n tokens of `[B, N, H, d]` as contiguous `[1, H, n, d]`."""
    return t[b:b + 1, :n].permute(0, 2, 1, 3).contiguous()


class ZImageSinkCalibrationProcessor:
    """Records each sample's block scores, then runs the original dense processor
    (sink_sparse_zimage.py:369-417)."""

    def __init__(self, calibrator: ZImageSinkMaskCalibrator, layer_idx: int, origin_processor: Any):
        self.calibrator = calibrator
        self.layer_idx = int(layer_idx)
        self.origin_processor = origin_processor

    def __call__(self, attn: Any, hidden_states: torch.Tensor, encoder_hidden_states: Optional[torch.Tensor] = None,
                 attention_mask: Optional[torch.Tensor] = None, freqs_cis: Optional[torch.Tensor] = None) -> torch.Tensor:
        if encoder_hidden_states is not None:
            raise AssertionError("Z-Image uses single-stream attention only.")
        if self.origin_processor is None:
            raise RuntimeError("Z-Image calibration requires access to the original dense attention processor.")
        q, k, v = prepare_zimage_attention_tensors(attn, hidden_states, freqs_cis=freqs_cis)
        image_tokens = self.calibrator.image_token_count
        for b, n in enumerate(_valid_lengths(attention_mask, int(hidden_states.size(0)), int(hidden_states.size(1)))):
            if n < image_tokens:
                raise ValueError("Observed valid sequence shorter than the padded image token prefix. "
                                 f"valid_len={n}, image_token_count={image_tokens}")
            self.calibrator.record(self.layer_idx, _sample_bhsd(q, b, n), _sample_bhsd(k, b, n),
                                   _sample_bhsd(v, b, n), text_token_count=n - image_tokens)
        return self.origin_processor(attn, hidden_states, encoder_hidden_states=encoder_hidden_states,
                                     attention_mask=attention_mask, freqs_cis=freqs_cis)


class ZImageStaticSinkProcessor:
    """Static sink-mask inference processor (sink_sparse_zimage.py:420-614).

    Per sample: the layer mask restricted to the call's text length with text rows and
    columns forced dense (cached per device and text-block count, so the kernel plan is
    built once per distinct prompt length), the block-sparse call, and for pooled_kv the
    compensation branch on the image queries (image K/V mean-pooled by `sample_gap` plus
    the full text K/V) mixed by LSE.  Forced-dense steps/layers use dense SDPA."""

    def __init__(self, *, layer_idx: int, total_layers: Optional[int], sink_mask: torch.Tensor,
                 config: SinkSparseConfig, runtime_state: Optional[SinkRuntimeState] = None):
        self.layer_idx = int(layer_idx)
        self.total_layers = None if total_layers is None else int(total_layers)
        self.sink_mask = sink_mask.bool().cpu()
        self.config = config
        self.runtime_state = runtime_state
        self.image_token_count, self.image_blocks, self.total_blocks = _fixed_block_shape(self.config)
        self.max_text_tokens = _max_text_token_count(self.config)
        self._runtime_mask_cache: Dict[tuple, torch.Tensor] = {}

    def _resolve_dynamic_plan(self) -> tuple[str, int]:
        mode = str(self.config.dynamic_mode).strip().lower()
        if mode not in ("none", "pooled_kv"):
            raise ValueError("Unsupported Z-Image Sink dynamic_mode. "
                             f"Expected one of: none, pooled_kv. Got: {self.config.dynamic_mode}")
        return mode, max(int(self.config.sample_gap), 1)

    def _should_force_dense_current_step(self) -> bool:
        if self.runtime_state is None:
            return False
        step = int(self.runtime_state.current_step)
        return step >= 0 and step in _resolve_forced_dense_step_list(self.config, self.runtime_state)

    def _should_force_dense_current_layer(self) -> bool:
        return self.layer_idx in _resolve_forced_dense_layer_list(self.config, total_layers=self.total_layers)

    def _runtime_mask(self, text_blocks: int, device: torch.device) -> torch.Tensor:
        key = (_device_cache_key(device), int(text_blocks))
        m = self._runtime_mask_cache.get(key)
        if m is None:
            m = _slice_runtime_sink_mask(self.sink_mask.to(device=device), image_blocks=self.image_blocks,
                                         current_text_blocks=text_blocks, total_blocks=self.total_blocks)
            m = _force_text_dense_runtime_mask(m, image_blocks=self.image_blocks,
                                               current_text_blocks=text_blocks).unsqueeze(0)
            self._runtime_mask_cache[key] = m
        return m

    def __call__(self, attn: Any, hidden_states: torch.Tensor, encoder_hidden_states: Optional[torch.Tensor] = None,
                 attention_mask: Optional[torch.Tensor] = None, freqs_cis: Optional[torch.Tensor] = None) -> torch.Tensor:
        if encoder_hidden_states is not None:
            raise AssertionError("Z-Image uses single-stream attention only.")
        rs = self.runtime_state
        if rs is not None:
            rs.enter_layer(self.layer_idx)
        sec = (lambda name: rs.time_section(name)) if rs is not None else (lambda name: nullcontext())
        with sec("inner_total"):
            with sec("qkv"):
                query, key, value = prepare_zimage_attention_tensors(attn, hidden_states, freqs_cis=freqs_cis)
            B, N = int(hidden_states.size(0)), int(hidden_states.size(1))
            out_padded = hidden_states.new_zeros((B, N, attn.heads, int(query.size(-1))))
            mode, gap = self._resolve_dynamic_plan()
            dense_step = self._should_force_dense_current_step()
            force_dense = dense_step or self._should_force_dense_current_layer()
            for b, n in enumerate(_valid_lengths(attention_mask, B, N)):
                if n < self.image_token_count:
                    raise ValueError("Observed valid sequence shorter than the padded image token prefix. "
                                     f"valid_len={n}, image_token_count={self.image_token_count}")
                text_tokens = n - self.image_token_count
                if text_tokens > self.max_text_tokens:
                    raise ValueError("Observed Z-Image text token count exceeds the mask package maximum. "
                                     f"Observed {text_tokens}, configured max {self.max_text_tokens}.")
                text_blocks = _ceil_div(int(text_tokens), int(self.config.block_size))
                mask = self._runtime_mask(text_blocks, query.device)
                q_i, k_i, v_i = _sample_bhsd(query, b, n), _sample_bhsd(key, b, n), _sample_bhsd(value, b, n)
                dyn_len = None
                if force_dense:
                    with sec("dense_override"):
                        out_i = _dense_attention(q_i, k_i, v_i)
                    mask = torch.ones_like(mask, dtype=torch.bool)
                    run_mode = "forced_dense_step" if dense_step else "forced_dense_layer"
                elif (mode == "pooled_kv" and FUSE_COMPENSATION and self.image_token_count % 128 == 0
                      and _fused_compensation_supported(q_i, k_i, v_i)):
                    il = self.image_token_count
                    with sec("comp_pool"):
                        dyn_k = ops.mean_pool_tokens(k_i[:, :, :il], gap)
                        dyn_v = ops.mean_pool_tokens(v_i[:, :, :il], gap)
                        if text_tokens > 0:
                            dyn_k = torch.cat([dyn_k, k_i[:, :, il:n]], dim=2)
                            dyn_v = torch.cat([dyn_v, v_i[:, :, il:n]], dim=2)
                        dyn_len = int(dyn_k.size(2))
                    with sec("sparse_main"):  # sparse + compensation on the image rows + mix
                        out_i = _block_sparse_attn_with_compensation(q_i, k_i, v_i, mask, dyn_k, dyn_v, gap,
                                                                     compensated_rows=il)
                    run_mode = mode
                else:
                    with sec("sparse_main"):
                        out_i, sink_lse = _block_sparse_attn(q_i, k_i, v_i, mask, return_lse=mode == "pooled_kv")
                    run_mode = mode
                    if mode == "pooled_kv":
                        il = self.image_token_count
                        with sec("comp_pool"):
                            dyn_k = _mean_pool_sequence(k_i[:, :, :il], gap)
                            dyn_v = _mean_pool_sequence(v_i[:, :, :il], gap)
                            if text_tokens > 0:
                                dyn_k = torch.cat([dyn_k, k_i[:, :, il:n]], dim=2)
                                dyn_v = torch.cat([dyn_v, v_i[:, :, il:n]], dim=2)
                            dyn_len = int(dyn_k.size(2))
                        with sec("comp_attn"):
                            image_q = q_i[:, :, :il]
                            if self.config.dynamic_kernel == "dense":
                                dyn_out, dyn_lse = _dense_short_attention_with_lse(image_q, dyn_k, dyn_v)
                            else:
                                full = torch.ones(image_q.size(0), image_q.size(1),
                                                  _ceil_div(image_q.size(2), int(self.config.block_size)),
                                                  _ceil_div(dyn_k.size(2), int(self.config.block_size)),
                                                  dtype=torch.bool, device=image_q.device)
                                dyn_out, dyn_lse = _block_sparse_attn(image_q, dyn_k, dyn_v, full, return_lse=True)
                        with sec("mix"):
                            mixed = _mix_attention_outputs(sink_out=out_i[:, :, :il], sink_lse=sink_lse[:, :, :il],
                                                           dynamic_out=dyn_out, dynamic_lse=dyn_lse,
                                                           config=self.config, dynamic_sample_gap=gap)
                            out_i = out_i.clone()
                            out_i[:, :, :il] = mixed
                out_padded[b, :n] = out_i.transpose(1, 2)[0]
                if rs is not None:
                    rs.record_mask_stats(layer_idx=self.layer_idx, sink_mask_tag="__base__", dynamic_mode=run_mode,
                                         dynamic_sample_gap=0 if force_dense else int(gap), base_runtime_mask=mask,
                                         topup_mask=None, dynamic_seq_len_k=dyn_len, total_seq_len_k=n)
            with sec("proj_out"):
                out = attn.to_out[0](out_padded.flatten(2, 3).to(dtype=hidden_states.dtype))
                if len(attn.to_out) > 1:
                    out = attn.to_out[1](out)
            return out


def set_sink_calibration_attn_zimage(model: Any, calibrator: ZImageSinkMaskCalibrator) -> ZImageSinkMaskCalibrator:
    """Wrap every `model.layers[i].attention` processor with the calibration processor
    (sink_sparse_zimage.py:617-633)."""
    build_zimg_sink_config(package_config=asdict(calibrator.config))
    for i, block in enumerate(model.layers):
        previous = block.attention.get_processor()
        block.attention.set_processor(ZImageSinkCalibrationProcessor(calibrator=calibrator, layer_idx=i,
                                                                     origin_processor=previous))
        if not hasattr(block.attention, "origin_processor"):
            block.attention.origin_processor = previous
    return calibrator


def set_sink_sparse_attn_zimage(model: Any, sink_mask_path: str, config_overrides: Optional[dict] = None) -> dict:
    """Load a v3 mask package and install the static processor on every layer
    (sink_sparse_zimage.py:636-673)."""
    package = load_sink_mask_package(sink_mask_path)
    config = build_zimg_sink_config(package_config=package.get("config"), config_overrides=config_overrides)
    state = SinkRuntimeState()
    model._sink_runtime_state = state
    masks = package.get("sink_masks", {})
    n_layers = len(model.layers)
    for i, block in enumerate(model.layers):
        if str(i) not in masks:
            raise KeyError(f"Layer {i} does not exist in sink mask package: {sink_mask_path}")
        previous = block.attention.get_processor()
        block.attention.set_processor(ZImageStaticSinkProcessor(layer_idx=i, total_layers=n_layers,
                                                                sink_mask=masks[str(i)], config=config,
                                                                runtime_state=state))
        if not hasattr(block.attention, "origin_processor"):
            block.attention.origin_processor = previous
    route = "zimg_static_only" if str(config.dynamic_mode).strip().lower() == "none" else "zimg_static_comp"
    return {"config": config, "num_layers": n_layers, "mask_path": sink_mask_path, "route": route}


def reset_sink_runtime_state_zimage(model: Any, num_inference_steps: Optional[int] = None) -> None:
    state = getattr(model, "_sink_runtime_state", None)
    if state is not None:
        state.reset_generation(total_steps=num_inference_steps)
