"""SinkAttention sparse-attention core on MI355X kernels.

Drop-in for the reference module ``sinkattention.sparse_attention``
(sinkattention/sparse_attention.py): every public and private name the reference's
callers import exists here with the same signature and error behaviour.  The hot path
runs on libsinkattn (hand-written gfx950 HIP kernels):

* ``_compute_block_scores`` / ``_compute_exact_block_mass_scores`` /
  ``_compute_pooled_qk_block_scores``  -> block_mass_pool / max_pool / mean_pool kernels
* ``_build_direct_mean_coverage_mask``  -> coverage_mask kernel (bit-exact with the
  reference's CPU torch arithmetic)
* ``_block_sparse_attn``                -> block_sparse_plan + block_sparse_fwd kernels

These need a ROCm GPU and the built library; nothing falls back to CPU.  The remaining
helpers (config, calibrator bookkeeping, package I/O, mask re-tiling, the dense short
attention and LSE mixing of the compensation branch) keep the reference's torch
semantics.
"""
from __future__ import annotations

import math
import os
import weakref
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from sinkattn_amd import _lib, ops
from sinkattn_amd.timing import AttentionTimingCollector

try:
    _lib.load_library()
    _HAS_BLOCK_SPARSE = True
    _HAS_TRITON_POOLING = True  # name kept for callers; the max-pool path is a HIP kernel
except ImportError:
    _HAS_BLOCK_SPARSE = False
    _HAS_TRITON_POOLING = False

from sinkattn_amd.pooling_kernel import attn_with_pooling  # noqa: E402

_BLOCK_SPARSE_RUNTIME_CACHE: Dict[Tuple[str, int, int, int, int, int], tuple] = {}
_EXACT_BLOCK_SCORE_KEY_CHUNK_BLOCKS = 16
_BLOCK_SPARSE_KERNEL_BLOCK_SIZE = 128

_VIDEO_RESIDUAL_MODES = {"video_residual", "video_residual_only", "residual_video"}


@dataclass
class SinkSparseConfig:
    """Same fields and defaults as the reference (sinkattention/sparse_attention.py:35-68)."""

    block_size: int = 128
    sample_gap: int = 30
    token_width: int = 52
    token_height: int = 30
    token_depth: int = 21
    text_length: int = 0
    force_text_global_attention: bool = False
    offline_text_video_coverage_mode: str = "joint"
    keep_diagonal: bool = True
    runtime_diagonal_band_width: int = 0
    pooling_mode: str = "triton"
    dynamic_mode: str = "pooled_kv"
    dynamic_kernel: str = "auto"
    mixing_mode: str = "adaptive"
    force_dense_steps: Optional[list[int]] = None
    force_dense_layers: Optional[list[int]] = None
    offline_direct_coverage: float = 0.85

    @classmethod
    def from_dict(cls, data: Optional[dict]) -> "SinkSparseConfig":
        """Unknown keys are dropped."""
        if not data:
            return cls()
        known = set(cls.__dataclass_fields__)
        return cls(**{key: val for key, val in data.items() if key in known})

    def merged(self, overrides: Optional[dict] = None) -> "SinkSparseConfig":
        """A copy with the non-None entries of ``overrides`` applied."""
        data = asdict(self)
        if overrides:
            data.update({key: val for key, val in overrides.items() if val is not None})
        return SinkSparseConfig.from_dict(data)


def _ceil_div(value: int, divisor: int) -> int:
    return (value + divisor - 1) // divisor


def _device_cache_key(device: torch.device) -> tuple[str, int]:
    return device.type, -1 if device.index is None else int(device.index)


# --- sequence pooling helpers (torch; used by the compensation branch) -------------------
def _pad_to_multiple(x: torch.Tensor, multiple: int) -> torch.Tensor:
    """Replicate-pad dim 2 up to a multiple (sinkattention/sparse_attention.py:79-85)."""
    rem = x.size(2) % multiple
    if rem == 0:
        return x
    return F.pad(x, (0, 0, 0, multiple - rem), mode="replicate")


def _token_pool_on_gpu(x: torch.Tensor) -> bool:
    """GPU tensors go to the mean_pool_tokens kernel; host tensors keep the torch ops."""
    return x.is_cuda and x.dim() == 4


def _mean_pool_sequence(x: torch.Tensor, pool_size: int) -> torch.Tensor:
    """Mean over groups of ``pool_size`` rows of dim 2, the last group replicate-padded
    (sparse_attention.py:88-94).  On the GPU: one mean_pool_tokens launch."""
    if pool_size <= 1:
        return x
    if _token_pool_on_gpu(x):
        return ops.mean_pool_tokens(x, int(pool_size), 0)
    x = _pad_to_multiple(x, pool_size)
    b, h, n, d = x.shape
    return x.view(b, h, n // pool_size, pool_size, d).mean(dim=-2)


def _mean_pool_sequence_preserve_prefix(x: torch.Tensor, pool_size: int, *,
                                        prefix_tokens: int = 0) -> torch.Tensor:
    """Keep the first ``prefix_tokens`` rows, mean-pool the rest (sparse_attention.py:97-115).
    On the GPU: one mean_pool_tokens launch (no concatenation)."""
    if pool_size <= 1:
        return x
    n = int(x.size(2))
    prefix = min(max(int(prefix_tokens), 0), n)
    if prefix >= n:
        return x
    if _token_pool_on_gpu(x):
        return ops.mean_pool_tokens(x, int(pool_size), prefix)
    if prefix <= 0:
        return _mean_pool_sequence(x, pool_size)
    return torch.cat([x[:, :, :prefix, :], _mean_pool_sequence(x[:, :, prefix:, :], pool_size)], dim=2)


# --- block scores (a1-a4) ---------------------------------------------------------------
def _compute_pooled_qk_block_scores(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                    config: SinkSparseConfig) -> torch.Tensor:
    """'triton' (max-pool) and 'mean' modes (sparse_attention.py:118-142).

    'triton' runs the max-pool HIP kernel; as in the reference a RuntimeError there falls
    back to the mean-pooled scores.
    """
    block = int(config.block_size)
    scale = 1.0 / math.sqrt(q.size(-1))
    if config.pooling_mode == "triton" and q.is_cuda:
        try:
            return ops.max_pool_scores(q, k, scale, block_size=block, causal=False).float()
        except RuntimeError:
            pass
    return ops.mean_pool_scores(q, k, block_size=block, scale=scale)


def _compute_exact_block_mass_scores(q: torch.Tensor, k: torch.Tensor,
                                     config: SinkSparseConfig) -> torch.Tensor:
    """Mean softmax mass per (q-block, k-block), fp32 (sparse_attention.py:145-227)."""
    return ops.block_mass_scores(q, k, block_size=int(config.block_size),
                                 scale=1.0 / math.sqrt(q.size(-1)))


def _compute_block_scores(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          config: SinkSparseConfig) -> torch.Tensor:
    """Dispatch on ``config.pooling_mode`` (sparse_attention.py:230-238)."""
    mode = str(config.pooling_mode).strip().lower()
    if mode == "exact":
        return _compute_exact_block_mass_scores(q, k, config)
    if mode in {"triton", "mean"}:
        return _compute_pooled_qk_block_scores(q, k, v, config)
    raise ValueError(
        f"Unsupported pooling_mode: {config.pooling_mode}. Expected one of: exact, triton, mean."
    )


# --- mask builder (a6) ----------------------------------------------------------------------
def _required_block_counts(num_query_blocks: int, num_key_blocks: int,
                           config: SinkSparseConfig) -> Tuple[int, int]:
    """(#leading rows, #leading columns) forced on by text-global attention."""
    if bool(getattr(config, "force_text_global_attention", False)) and int(config.text_length) > 0:
        text_blocks = _ceil_div(int(config.text_length), int(config.block_size))
        rq = min(text_blocks, int(num_query_blocks))
        rk = min(text_blocks, int(num_key_blocks))
        if rq > 0 and rk > 0:
            return rq, rk
    return 0, 0


def _build_offline_required_mask(*, num_query_blocks: int, num_key_blocks: int,
                                 config: SinkSparseConfig,
                                 device: torch.device) -> Optional[torch.Tensor]:
    """Leading text rows/cols forced on (sparse_attention.py:241-265); None when unused."""
    rq, rk = _required_block_counts(num_query_blocks, num_key_blocks, config)
    if rq == 0:
        return None
    req = torch.zeros(num_query_blocks, num_key_blocks, dtype=torch.bool, device=device)
    req[:, :rk] = True
    req[:rq, :] = True
    return req


def _gpu_device_for(t: torch.Tensor) -> torch.device:
    if t.is_cuda:
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("the coverage-mask kernel needs a ROCm GPU")
    return torch.device("cuda", torch.cuda.current_device())


def _coverage_mask_args(mean_scores: torch.Tensor, config: SinkSparseConfig) -> tuple:
    """Checks the [heads, blocks_q, blocks_k] shape; returns the kernel's (coverage,
    keep_diagonal, required rows, required columns, video_residual text blocks or None)."""
    if mean_scores.dim() != 3:
        raise ValueError(f"Expected [heads, blocks_q, blocks_k] scores, got {tuple(mean_scores.shape)}")
    _, nq, nk = (int(x) for x in mean_scores.shape)
    coverage = min(max(float(config.offline_direct_coverage), 0.0), 1.0)
    mode = str(getattr(config, "offline_text_video_coverage_mode", "joint")).strip().lower()
    rq, rk = _required_block_counts(nq, nk, config)
    video_tb = None
    if (mode in _VIDEO_RESIDUAL_MODES and bool(getattr(config, "force_text_global_attention", False))
            and int(getattr(config, "text_length", 0)) > 0):
        tb = min(_ceil_div(int(config.text_length), int(config.block_size)), nq, nk)
        if tb > 0:
            video_tb = tb
    return coverage, bool(config.keep_diagonal), rq, rk, video_tb


def _build_direct_mean_coverage_mask(mean_scores: torch.Tensor,
                                     config: SinkSparseConfig) -> torch.Tensor:
    """Per (head, q-block) row, keep the top key blocks until their mean mass reaches
    ``offline_direct_coverage`` of the row, plus required blocks and the diagonal
    (sparse_attention.py:268-376).  Runs the coverage_mask kernel; the result is a bool
    tensor on ``mean_scores``' device, bit-identical to the reference's CPU result."""
    args = _coverage_mask_args(mean_scores, config)
    dev = _gpu_device_for(mean_scores)
    scores = mean_scores.float().to(dev)
    mask = ops.coverage_mask(scores, *args)
    return mask.to(mean_scores.device)


def _build_direct_mean_coverage_masks(means: Sequence[torch.Tensor],
                                      config: SinkSparseConfig) -> List[torch.Tensor]:
    """`_build_direct_mean_coverage_mask` of every tensor of `means` (each its own call, its
    own empty-row fallback included), with the host<->device traffic batched: equal-shaped
    inputs go to the GPU in one copy, the kernels run back to back, and the masks come back
    in one copy.  Results are on the inputs' device, as for the single call."""
    if not means:
        return []
    args = [_coverage_mask_args(m, config) for m in means]
    dev = _gpu_device_for(means[0])
    home = means[0].device
    if any(m.shape != means[0].shape or m.device != home for m in means):
        return [_build_direct_mean_coverage_mask(m, config) for m in means]
    scores = torch.stack([m.float() for m in means]).to(dev)
    masks = torch.stack([ops.coverage_mask(scores[i], *args[i]) for i in range(len(means))])
    return list(masks.to(home).unbind(0))


def _device_package_groups(sums: Sequence[torch.Tensor], sq_sums: Sequence[torch.Tensor],
                           denoms: Sequence[torch.Tensor], config: SinkSparseConfig, need_scores: bool,
                           denom_min: Optional[float] = None, group_bytes: int = 256 << 20):
    """The package's statistics of calibration sums that live on one GPU, layer by layer as
    the reference's host math computes them: mean = sum / denom, var = clamp(sq / denom -
    mean^2, 0) (elementwise IEEE operations, bit-identical on either side), and the coverage
    masks of the means.  denoms[j] is a device tensor broadcastable to sums[j] (a layer's
    call count, or Z-Image's presence counts, clamped below at `denom_min` when given).
    Layers go in groups whose stacked sums take at most `group_bytes`, with in-place
    arithmetic, so the transient device memory is about three such stacks (768 MB by
    default) whatever the layer count.  Returns host lists: masks, and means and stds (None
    unless need_scores; the square roots are taken on the host, since torch's device sqrt is
    not correctly rounded)."""
    per = max(1, sums[0].numel() * sums[0].element_size())
    G = max(1, group_bytes // per)
    args = _coverage_mask_args(sums[0], config)
    masks: List[torch.Tensor] = []
    means: Optional[List[torch.Tensor]] = [] if need_scores else None
    stds: Optional[List[torch.Tensor]] = [] if need_scores else None
    for g0 in range(0, len(sums), G):
        sl = slice(g0, g0 + G)
        den = torch.stack(list(denoms[sl]))
        if denom_min is not None:
            den.clamp_min_(denom_min)
        mean = torch.stack(list(sums[sl]))
        mean.div_(den)
        masks.extend(_to_host([ops.coverage_mask(mean[i], *args) for i in range(mean.size(0))]))
        if need_scores:
            var = torch.stack(list(sq_sums[sl]))
            var.div_(den)
            sq = torch.mul(mean, mean)
            var.sub_(sq)
            del sq
            var.clamp_min_(0.0)
            means.extend(_to_host(list(mean.unbind(0))))
            stds.extend(torch.sqrt(x) for x in _to_host(list(var.unbind(0))))
        del mean, den
    return masks, means, stds


def _to_host(tensors: Sequence[torch.Tensor], chunk_bytes: int = 256 << 20) -> List[torch.Tensor]:
    """Host copies of equal-shaped tensors, stacked on their device in chunks of at most
    `chunk_bytes` so that one copy moves many of them (the values are untouched)."""
    out: List[torch.Tensor] = []
    i = 0
    while i < len(tensors):
        t0 = tensors[i]
        per = max(1, chunk_bytes // max(1, t0.numel() * t0.element_size()))
        group = [t0]
        while (i + len(group) < len(tensors) and len(group) < per
               and tensors[i + len(group)].shape == t0.shape
               and tensors[i + len(group)].dtype == t0.dtype
               and tensors[i + len(group)].device == t0.device):
            group.append(tensors[i + len(group)])
        out.extend(torch.stack(group).cpu().unbind(0))
        i += len(group)
    return out


# --- runtime statistics ----------------------------------------------------------------------
class SinkRuntimeState:
    """Step counter, per-call mask statistics and timing sections
    (sparse_attention.py:379-523)."""

    def __init__(self):
        self.current_step = -1
        self.total_steps: Optional[int] = None
        self.sparsity_events: list[dict] = []
        self.timing = AttentionTimingCollector(label="sink")
        self._density_cache: Dict[tuple, float] = {}

    def reset_generation(self, total_steps: Optional[int] = None) -> None:
        self.current_step = -1
        self.total_steps = total_steps
        self.sparsity_events = []
        self.timing.reset()

    def time_section(self, name: str):
        return self.timing.section(name)

    def summarize_timing(self) -> dict:
        return self.timing.summarize()

    def enter_layer(self, layer_idx: int) -> None:
        if layer_idx == 0:
            self.current_step += 1

    @staticmethod
    def _mask_density(mask: Optional[torch.Tensor]) -> float:
        if mask is None:
            return 0.0
        total = mask.numel()
        if total <= 0:
            return 0.0
        return float(int(mask.sum().item())) / float(total)

    @staticmethod
    def _mean_metric(events: list[dict], key: str) -> float:
        if not events:
            return 0.0
        return float(sum(float(e[key]) for e in events) / len(events))

    def _cached_density(self, mask: Optional[torch.Tensor]) -> float:
        """Density of a mask, computed once per mask object (and content version).  The
        runtimes pass the same cached kernel mask on every call, so the device-to-host
        read happens on the first call only, not on every layer call as in the reference."""
        if mask is None:
            return 0.0
        key = id(mask)
        sig = (mask._version, mask.data_ptr(), tuple(mask.shape), str(mask.device))
        ent = self._density_cache.get(key)
        if ent is not None and ent[0]() is mask and ent[1] == sig:
            return ent[2]
        val = self._mask_density(mask)
        cache = self._density_cache
        cache[key] = (weakref.ref(mask, lambda _r, k=key: cache.pop(k, None)), sig, val)
        return val

    def record_mask_stats(self, *, layer_idx: int, sink_mask_tag: str, dynamic_mode: str,
                          dynamic_sample_gap: int, base_runtime_mask: torch.Tensor,
                          topup_mask: Optional[torch.Tensor] = None,
                          dynamic_seq_len_k: Optional[int] = None,
                          total_seq_len_k: Optional[int] = None) -> None:
        base = self._cached_density(base_runtime_mask)
        topup = self._cached_density(topup_mask)
        combined = base if topup_mask is None else self._mask_density(base_runtime_mask | topup_mask)
        ratio = 0.0
        if dynamic_seq_len_k is not None and total_seq_len_k is not None and total_seq_len_k > 0:
            ratio = float(dynamic_seq_len_k) / float(total_seq_len_k)
        dense_eq = combined + ratio
        self.sparsity_events.append({
            "step": int(self.current_step),
            "layer_idx": int(layer_idx),
            "sink_mask_tag": str(sink_mask_tag),
            "dynamic_mode": str(dynamic_mode),
            "dynamic_sample_gap": int(dynamic_sample_gap),
            "base_density": base,
            "base_sparsity": 1.0 - base,
            "topup_density": topup,
            "combined_density": combined,
            "combined_sparsity": 1.0 - combined,
            "dynamic_key_ratio": ratio,
            "dense_equivalent_density": dense_eq,
            "dense_equivalent_sparsity": 1.0 - dense_eq,
            "dynamic_seq_len_k": None if dynamic_seq_len_k is None else int(dynamic_seq_len_k),
            "total_seq_len_k": None if total_seq_len_k is None else int(total_seq_len_k),
        })

    _SUMMARY_KEYS = ("base_density", "base_sparsity", "topup_density", "combined_density",
                     "combined_sparsity", "dynamic_key_ratio", "dense_equivalent_density",
                     "dense_equivalent_sparsity")

    def _summarize_events(self, events: list[dict]) -> dict:
        if not events:
            return {}
        out = {"count": len(events)}
        for key in self._SUMMARY_KEYS:
            out[f"{key}_mean"] = self._mean_metric(events, key)
        return out

    def summarize_sparsity(self) -> dict:
        ev = self.sparsity_events
        if not ev:
            return {"num_events": 0, "total_steps_expected": self.total_steps, "steps_recorded": [],
                    "layers_recorded": [], "overall": {}, "by_step": {}, "by_layer": {},
                    "by_dynamic_mode": {}, "by_sink_mask_tag": {}}
        steps = sorted({int(e["step"]) for e in ev})
        layers = sorted({int(e["layer_idx"]) for e in ev})
        modes = sorted({str(e["dynamic_mode"]) for e in ev})
        tags = sorted({str(e["sink_mask_tag"]) for e in ev})
        return {
            "num_events": len(ev),
            "total_steps_expected": self.total_steps,
            "steps_recorded": steps,
            "layers_recorded": layers,
            "overall": self._summarize_events(ev),
            "by_step": {str(s): self._summarize_events([e for e in ev if int(e["step"]) == s]) for s in steps},
            "by_layer": {str(l): self._summarize_events([e for e in ev if int(e["layer_idx"]) == l]) for l in layers},
            "by_dynamic_mode": {m: self._summarize_events([e for e in ev if str(e["dynamic_mode"]) == m]) for m in modes},
            "by_sink_mask_tag": {t: self._summarize_events([e for e in ev if str(e["sink_mask_tag"]) == t]) for t in tags},
        }


# --- calibration (a5) ------------------------------------------------------------------------
class SinkMaskCalibrator:
    """Accumulates per-layer block scores over calibration calls and builds the mask
    package (sparse_attention.py:526-608).

    The reference copies every call's batch-mean map to the host (a device sync per layer
    call) and accumulates there.  Here the per-layer fp32 sums stay on the device the
    scores were computed on; the accumulation is elementwise fp32 adds and squares (exact
    IEEE operations on either side), and `build_package` copies the sums to the host once
    and finishes there like the reference, so the package is bit-identical to host
    accumulation."""

    # Where the per-layer sums live.  On the GPU (default) they cost 2 x 4 bytes x heads x
    # q-blocks x k-blocks per layer of device memory for the whole calibration (Wan2.1-1.3B:
    # 30 x 12 x 256 x 256 -> 189 MB; Wan2.1-14B at 720p: 40 x 40 x 591 x 591 -> 4.5 GB) and
    # no host sync per call.  Set to True for the reference's behaviour: each call's batch
    # mean is copied to the host (one sync per call) and accumulated there.  The package is
    # bit-identical either way (the same fp32 adds and squares).
    accumulate_on_host: bool = False

    def __init__(self, config: SinkSparseConfig):
        self.config = config
        self.current_step = -1
        self.score_sums: Dict[int, torch.Tensor] = {}
        self.score_sq_sums: Dict[int, torch.Tensor] = {}
        self.score_counts: Dict[int, int] = {}

    def reset_generation(self) -> None:
        self.current_step = -1

    def _accumulate_score(self, layer_idx: int, scores: torch.Tensor) -> None:
        if self.accumulate_on_host:
            scores = scores.cpu()
        if layer_idx not in self.score_sums:
            self.score_sums[layer_idx] = scores
            self.score_sq_sums[layer_idx] = scores.square()
            self.score_counts[layer_idx] = 1
        else:
            self.score_sums[layer_idx] += scores
            self.score_sq_sums[layer_idx] += scores.square()
            self.score_counts[layer_idx] += 1

    def _build_mean_and_masks(self, config: Optional[SinkSparseConfig] = None, *,
                              need_scores: bool = True) -> tuple[dict, dict, dict, dict]:
        config = self.config if config is None else config
        mean_scores, std_scores, sink_masks, counts = {}, {}, {}, {}
        layers = sorted(self.score_sums)
        if not layers:
            return mean_scores, std_scores, sink_masks, counts
        first = self.score_sums[layers[0]]
        on_device = first.is_cuda and all(self.score_sums[i].shape == first.shape
                                          and self.score_sums[i].device == first.device for i in layers)
        if on_device:
            # Mean and std where the sums are, in groups of layers.  The count is a device
            # tensor, so the division is an elementwise IEEE division, as the reference's host
            # division (a division by a Python number would be a multiply by its reciprocal).
            # The package lives on the host: the masks always, the scores when asked for.
            n = [torch.full([1] * first.dim(), float(self.score_counts[i]), device=first.device) for i in layers]
            masks, means, stds = _device_package_groups([self.score_sums[i] for i in layers],
                                                        [self.score_sq_sums[i] for i in layers], n, config,
                                                        need_scores)
        else:
            # sums on the host (accumulate_on_host, or mixed shapes): the reference's host math
            sums = _to_host([self.score_sums[i] for i in layers])
            sq_sums = _to_host([self.score_sq_sums[i] for i in layers])
            means, stds = [], []
            for j, layer_idx in enumerate(layers):
                n = self.score_counts[layer_idx]
                mean = sums[j] / n
                second = sq_sums[j] / n
                means.append(mean)
                stds.append(torch.sqrt((second - mean.square()).clamp_min_(0.0)))
            masks = [m.cpu() for m in _build_direct_mean_coverage_masks(means, config)]
        for j, layer_idx in enumerate(layers):
            key = str(layer_idx)
            if means is not None:
                mean_scores[key] = means[j]
                std_scores[key] = stds[j]
            sink_masks[key] = masks[j]
            counts[key] = int(self.score_counts[layer_idx])
        return mean_scores, std_scores, sink_masks, counts

    @torch.no_grad()
    def record(self, layer_idx: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """Block scores of one call on the GPU kernels; their batch mean is added to the
        layer's device-resident sums (no host copy, no sync)."""
        if layer_idx == 0:
            self.current_step += 1
        samples = _compute_block_scores(q, k, v, self.config).detach().float()
        self._accumulate_score(layer_idx, samples.mean(dim=0))

    def build_package(self, include_scores: bool = True,
                      config_override: Optional[SinkSparseConfig] = None) -> dict:
        cfg = self.config if config_override is None else config_override
        mean_scores, std_scores, sink_masks, counts = self._build_mean_and_masks(config=cfg,
                                                                               need_scores=include_scores)
        return {
            "version": 3,
            "config": asdict(cfg),
            "mean_scores": mean_scores if include_scores else {},
            "std_scores": std_scores if include_scores else {},
            "sink_masks": sink_masks,
            "counts": counts,
            "meta": {"route": "wanx_direct_coverage"},
        }

    def save(self, output_path: str, include_scores: bool = True,
             config_override: Optional[SinkSparseConfig] = None) -> dict:
        package = self.build_package(include_scores=include_scores, config_override=config_override)
        out = Path(output_path)
        out.parent.mkdir(parents=True, exist_ok=True)
        torch.save(package, out)
        return package


# --- package I/O -----------------------------------------------------------------------------
_LFS_PREFIX = b"version https://git-lfs.github.com/spec/v1"


def load_sink_mask_package(mask_path: str) -> dict:
    """Load and validate a mask package (sparse_attention.py:611-666)."""
    if not os.path.exists(mask_path):
        raise FileNotFoundError(f"Sink mask file not found: {mask_path}")
    try:
        package = torch.load(mask_path, map_location="cpu", weights_only=True)
    except Exception as exc:
        try:
            with open(mask_path, "rb") as fh:
                head = fh.read(128)
        except OSError:
            head = b""
        if head.startswith(_LFS_PREFIX):
            raise RuntimeError(
                "Sink mask file is still a Git LFS pointer, not the real package: "
                f"{mask_path}. Download the actual .pt asset before running Sink-Sparse."
            ) from exc
        raise RuntimeError(f"Failed to load sink mask package: {mask_path}: {exc}") from exc
    if not isinstance(package, dict):
        raise TypeError(f"Sink mask package must deserialize to a dict, got {type(package).__name__}: {mask_path}")
    masks = package.get("sink_masks")
    if not isinstance(masks, dict) or not masks:
        raise ValueError(f"Sink mask package does not contain usable sink_masks: {mask_path}")
    cfg = package.get("config") or {}
    if not isinstance(cfg, dict):
        raise TypeError(f"Sink mask package config must be a dict: {mask_path}")

    def reject(reason: str) -> None:
        raise ValueError(
            "Incompatible Sink mask package for the current SinkAttention runtime: "
            f"{mask_path}. {reason} Current runtime only supports one shared-step mask in "
            "the original token order. Re-calibrate or re-export a no-rearrange shared-step package."
        )

    if bool(cfg.get("use_rearrange", False)):
        reject("The package was calibrated with use_rearrange=True.")
    if package.get("step_groups"):
        reject("The package still contains step-group metadata.")
    if package.get("step_group_sink_masks"):
        reject("The package still contains per-step-group mask banks.")
    if bool(cfg.get("use_step_mask_bank", False)):
        reject("The package config still enables the legacy step mask bank.")
    for legacy in ("step_group_boundaries", "step_group_names"):
        if cfg.get(legacy) not in (None, False, "", [], {}):
            reject(f"The package config still carries populated legacy field {legacy}.")
    return package


# --- block-sparse attention (a7) ---------------------------------------------------------------
def _ensure_block_sparse_available() -> None:
    """ImportError when the HIP library is absent (sparse_attention.py:669-674)."""
    if not _HAS_BLOCK_SPARSE:
        raise ImportError(
            "Sink-Sparse online inference requires libsinkattn.so; build it with "
            "`python -m sinkattn_amd.build` before using --attn_mode sink."
        )


def _get_block_sparse_runtime_tensors(batch_size: int, num_heads: int, seq_len_q: int, seq_len_k: int,
                                      device: torch.device) -> tuple:
    """Varlen descriptors of the reference's external call (sparse_attention.py:677-707).
    Kept for callers; the HIP kernel addresses [B, H, N, D] views directly."""
    key = (*_device_cache_key(device), batch_size, num_heads, seq_len_q, seq_len_k)
    hit = _BLOCK_SPARSE_RUNTIME_CACHE.get(key)
    if hit is not None:
        return hit
    cu_q = torch.arange(0, (batch_size + 1) * seq_len_q, step=seq_len_q, dtype=torch.int32, device=device)
    cu_k = torch.arange(0, (batch_size + 1) * seq_len_k, step=seq_len_k, dtype=torch.int32, device=device)
    head_mask_type = torch.ones(num_heads, dtype=torch.int32, device=device)
    streaming_info = torch.zeros(2 * num_heads, dtype=torch.int32, device=device)
    hit = (cu_q, cu_k, head_mask_type, streaming_info)
    _BLOCK_SPARSE_RUNTIME_CACHE[key] = hit
    return hit


def _block_sparse_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_mask: torch.Tensor,
                       return_lse: bool = True) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    """softmax(QK^T/sqrt(d) + M) V over the listed 128x128 tiles (sparse_attention.py:710-776).

    q [B,H,Nq,D], k/v [B,H,Nk,D]; block_mask bool [B,H,ceil(Nq/128),ceil(Nk/128)].
    Returns out [B,H,Nq,D] (a view of [B,Nq,H,D] memory) and lse [B,H,Nq,1] in q.dtype
    (or None).  The kernel's list form of the mask is cached per mask tensor.
    """
    _ensure_block_sparse_available()
    plan = ops.PLAN_CACHE.get(block_mask if block_mask.is_cuda else block_mask.to(q.device))
    out, lse = ops.block_sparse_attention(q, k, v, plan, softmax_scale=None, return_lse=return_lse)
    if lse is None:
        return out, None
    return out, lse.unsqueeze(-1).to(device=q.device, dtype=q.dtype)


def _fused_compensation_supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """The fused sparse + compensation kernel covers bf16/f16 GPU tensors with d = 128."""
    return (q.is_cuda and q.dim() == 4 and q.dtype in (torch.bfloat16, torch.float16)
            and q.dtype == k.dtype == v.dtype and int(q.size(-1)) == 128)


def _block_sparse_attn_with_compensation(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                         block_mask: torch.Tensor, k_dynamic: torch.Tensor,
                                         v_dynamic: torch.Tensor, sample_gap: int,
                                         compensated_rows: Optional[int] = None) -> torch.Tensor:
    """Sparse attention and the pooled-K/V compensation with adaptive mixing in one kernel.

    The reference runs `_block_sparse_attn(..., return_lse=True)`, an attention over
    (k_dynamic, v_dynamic) with LSE and `_mix_attention_outputs`
    (wanx/runtime/sink_sparse_wan.py:194-265, zimg/runtime/sink_sparse_zimage.py:553-592).
    The mix weights exp(lse_s) : gap*exp(lse_d) make the result the attention over the
    listed keys plus every pooled key counted `sample_gap` times, which this computes in
    one online softmax (fp32 LSEs; the reference rounds both LSEs to q.dtype first).
    Rows at or beyond `compensated_rows` (a multiple of 128) get the sparse part only.
    k_dynamic/v_dynamic must share k's/v's row strides (ops.mean_pool_tokens(like=k)).
    """
    _ensure_block_sparse_available()
    plan = ops.PLAN_CACHE.get(block_mask if block_mask.is_cuda else block_mask.to(q.device))
    out, _ = ops.block_sparse_attention_comp(q, k, v, plan, k_dynamic, v_dynamic, int(sample_gap),
                                             comp_rows=compensated_rows, return_lse=False)
    return out


def _make_full_block_mask(batch_size: int, num_heads: int, seq_len_q: int, seq_len_k: int,
                          block_size: int, device: torch.device) -> torch.Tensor:
    return torch.ones(batch_size, num_heads, _ceil_div(seq_len_q, block_size),
                      _ceil_div(seq_len_k, block_size), dtype=torch.bool, device=device)


def _adapt_block_mask_for_kernel(block_mask: torch.Tensor, *, source_block_size: int, seq_len_q: int,
                                 seq_len_k: int,
                                 kernel_block_size: int = _BLOCK_SPARSE_KERNEL_BLOCK_SIZE) -> torch.Tensor:
    """Re-tile a mask to the kernel's tile size (sparse_attention.py:797-852): identity
    (shape-checked) at equal sizes, repeat for coarser masks, OR-group finer ones."""
    src, ker = int(source_block_size), int(kernel_block_size)
    if src <= 0 or ker <= 0:
        raise ValueError(f"Invalid block sizes: source={src}, kernel={ker}")
    tq, tk = _ceil_div(int(seq_len_q), ker), _ceil_div(int(seq_len_k), ker)
    if src == ker:
        if block_mask.size(-2) != tq or block_mask.size(-1) != tk:
            raise ValueError(
                "Runtime block mask is already at kernel tile size but has the wrong shape: "
                f"expected [..., {tq}, {tk}], got {list(block_mask.shape)}"
            )
        return block_mask.contiguous()
    if src > ker:
        if src % ker != 0:
            raise ValueError(
                "Cannot adapt a coarse Sink mask to the block-sparse kernel because "
                f"source block size {src} is not a multiple of kernel block size {ker}."
            )
        rep = src // ker
        out = block_mask.repeat_interleave(rep, dim=-2).repeat_interleave(rep, dim=-1)
        return out[..., :tq, :tk].contiguous()
    if ker % src != 0:
        raise ValueError(
            "Cannot adapt a fine Sink mask to the block-sparse kernel because "
            f"kernel block size {ker} is not a multiple of source block size {src}."
        )
    g = ker // src
    nqs, nks = int(block_mask.size(-2)), int(block_mask.size(-1))
    pq, pk = (-nqs) % g, (-nks) % g
    if pq or pk:
        block_mask = F.pad(block_mask, (0, pk, 0, pq), value=False)
    grouped = block_mask.view(*block_mask.shape[:-2], (nqs + pq) // g, g, (nks + pk) // g, g)
    return grouped.any(dim=-1).any(dim=-2)[..., :tq, :tk].contiguous()


# --- compensation branch helpers (torch semantics of the reference) ---------------------------
def _dense_short_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    return F.scaled_dot_product_attention(q, k, v, attn_mask=None, dropout_p=0.0, is_causal=False)


def _dense_short_attention_with_lse(q: torch.Tensor, k: torch.Tensor,
                                    v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense attention plus LSE, chunked over queries (sparse_attention.py:870-895)."""
    scale = 1.0 / math.sqrt(q.size(-1))
    per_q = int(q.size(0)) * int(q.size(1)) * int(k.size(2))
    limit = int(os.environ.get("SINK_DENSE_LSE_MAX_SCORE_ELEMENTS", "67108864"))
    chunk = int(q.size(2)) if per_q * int(q.size(2)) <= limit else max(1, limit // max(per_q, 1))
    kt = k.float().transpose(-1, -2)
    outs, lses = [], []
    for start in range(0, int(q.size(2)), chunk):
        sc = torch.matmul(q[:, :, start:start + chunk, :].float(), kt) * scale
        probs = torch.softmax(sc, dim=-1)
        outs.append(torch.matmul(probs.to(dtype=v.dtype), v).to(dtype=q.dtype))
        lses.append(torch.logsumexp(sc, dim=-1, keepdim=True).to(device=q.device, dtype=q.dtype))
    if len(outs) == 1:
        return outs[0], lses[0]
    return torch.cat(outs, dim=2), torch.cat(lses, dim=2)


_LOG_GAP_CACHE: Dict[tuple, float] = {}


def _log_gap_value(gap, dtype: torch.dtype) -> float:
    """The reference's ``sink_lse.new_tensor(gap).log()`` as a Python float: log of the
    dtype-rounded gap, rounded to the dtype (evaluated once per (gap, dtype) on the host,
    so the GPU path needs no device-to-host read)."""
    key = (int(gap), dtype)
    val = _LOG_GAP_CACHE.get(key)
    if val is None:
        val = float(torch.tensor(float(max(1, int(gap))), dtype=dtype).log().item())
        _LOG_GAP_CACHE[key] = val
    return val


def _mix_on_gpu(sink_out, sink_lse, dyn_out, dyn_lse) -> bool:
    """The lse_mix kernel covers one dtype for all four tensors, [B,H,N,D] outputs and
    [B,H,N] / [B,H,N,1] LSEs."""
    if not (sink_out.dim() == 4 and dyn_out.shape == sink_out.shape):
        return False
    if not (sink_out.dtype == dyn_out.dtype == sink_lse.dtype == dyn_lse.dtype):
        return False
    want = tuple(sink_out.shape[:3])
    return all(t.is_cuda and tuple(t.shape[:3]) == want and (t.dim() == 3 or (t.dim() == 4 and t.shape[3] == 1))
               for t in (sink_lse, dyn_lse)) and dyn_out.is_cuda


def _mix_attention_outputs(sink_out: torch.Tensor, sink_lse: Optional[torch.Tensor],
                           dynamic_out: torch.Tensor, dynamic_lse: Optional[torch.Tensor],
                           config: SinkSparseConfig, dynamic_sample_gap: Optional[int] = None) -> torch.Tensor:
    """alpha = sigmoid(lse_s - lse_d - log(gap)); out = alpha*sink + (1-alpha)*dynamic
    (sparse_attention.py:898-919)."""
    if config.mixing_mode != "adaptive":
        raise ValueError(f"Unsupported mixing_mode: {config.mixing_mode}")
    if sink_lse is None or dynamic_lse is None:
        raise ValueError("Adaptive Sink-Sparse mixing requires both sink_lse and dynamic_lse.")
    gap = config.sample_gap if dynamic_sample_gap is None else int(dynamic_sample_gap)
    if sink_out.is_cuda and _mix_on_gpu(sink_out, sink_lse, dynamic_out, dynamic_lse):
        return ops.lse_mix(sink_out, sink_lse, dynamic_out, dynamic_lse, _log_gap_value(gap, sink_lse.dtype))
    log_gap = sink_lse.new_tensor(float(max(1, int(gap)))).log()
    w_s = sink_lse
    w_d = dynamic_lse + log_gap
    mx = torch.maximum(w_s, w_d)
    e_s = torch.exp(w_s - mx)
    e_d = torch.exp(w_d - mx)
    alpha = e_s / (e_s + e_d)
    return sink_out * alpha + dynamic_out * (1.0 - alpha)


# --- package summaries / CLI helpers ---------------------------------------------------------
def summarize_sink_package(package: dict) -> str:
    counts = package.get("counts", {})
    masks = package.get("sink_masks", {})
    total = sum(counts.values()) if counts else 0
    cfg = package.get("config", {})
    dens = [float(m.float().mean().item()) for m in masks.values()]
    mean_density = sum(dens) / len(dens) if dens else 0.0
    cov = cfg.get("offline_direct_coverage")
    density_str = f", mean_density={mean_density:.4f}" if dens else ""
    coverage_str = f", coverage={float(cov):.3f}" if cov is not None else ""
    return (f"sink_masks={len(masks)}, mask_strategy=direct_mean_coverage{coverage_str}, "
            f"aggregated_calls={total}{density_str}")


def parse_int_list(values: Optional[str]) -> Optional[list[int]]:
    if values is None or values == "":
        return None
    return [int(item.strip()) for item in values.split(",") if item.strip()]


def iter_seed_list(seed_values: Iterable[int]) -> list[int]:
    return [int(seed) for seed in seed_values]
