"""Static quantization tables from calibration samples, and the calibration-JSON loader.

Scale production follows scripts/calibrate_behavior.py:228-259 and 764-811: per
calibration sample, the absmax of every (kv head, group) over the sample's tokens
(``compute_absmax_per_group``); per layer, torch.quantile of those sample maxima at
``clip_percentile / 100`` over the samples, clamped to 1e-5 and divided by qmax
(``scales_from_absmax_samples``).  ``absmax_scale`` is the percentile-100 case over one
pooled sample.  ``calibration_json`` writes the tables in the schema read by
src/engine/generate_loop.py:751-889:

* ``k_scale`` / ``v_scale`` [L, Hkv, G];
* ``inv_tau`` [L, Hq];
* ``group_size_k``, ``int4_outlier_ratio``, ``int4_mixed_rescue``.

INT8 scales load as fp16 and INT4 scales as fp32 (generate_loop.py:811-820).

The asymmetric group-32 tables (scale, zero-point) and the K outlier-channel choice
belong to the build-native INT4 format.  Per (head, group) they use
``s = max(max - min, 9.1552734375e-4) / 15`` and ``zp = min + 8 s``; that is
src/quant/asymmetric_quant.py:116-136 applied to calibration statistics.  The outlier
channels are excluded from the group statistics.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from typing import Optional

import torch

RANGE_FLOOR_INT4 = max(1e-5, float(torch.finfo(torch.float16).tiny) * 15)  # 9.1552734375e-4


def _groups(x: torch.Tensor, group_size: int) -> torch.Tensor:
    """[..., Hkv, T, D] -> [Hkv, N, G, gs] with all leading/token dims flattened."""
    if x.ndim == 3:
        x = x[None]
    N, H, T, D = x.shape
    return x.permute(1, 0, 2, 3).reshape(H, N * T, D // group_size, group_size)


def absmax_scale(sample: torch.Tensor, group_size: int, qmax: float) -> torch.Tensor:
    """fp32 [Hkv, G]: absmax over calibration tokens / qmax (calibrate_behavior.py:784-811)."""
    am = _groups(sample.float(), group_size).abs().amax(dim=(1, 3))
    return am.clamp(min=1e-5) / qmax


def compute_absmax_per_group(tensor: torch.Tensor, group_size: int) -> torch.Tensor:
    """[heads, seq, head_dim] -> [heads, head_dim // group_size]: per (head, group) absmax
    over the whole sequence (scripts/calibrate_behavior.py:228-259)."""
    if tensor.ndim != 3:
        raise ValueError(f"expected [heads, seq, head_dim], got {tuple(tensor.shape)}")
    heads, seq_len, head_dim = tensor.shape
    if group_size <= 0 or head_dim % group_size != 0:
        raise ValueError(f"head_dim ({head_dim}) must be divisible by group_size ({group_size})")
    view = tensor.reshape(heads, seq_len, head_dim // group_size, group_size)
    return view.abs().amax(dim=3).amax(dim=1)


def collect_absmax_samples(kv_samples, group_size: int):
    """kv_samples: list over samples -> list over layers -> [kv_heads, seq, head_dim].
    Returns list over layers -> list over samples -> [kv_heads, num_groups]
    (scripts/calibrate_behavior.py:764-781)."""
    if not kv_samples:
        return []
    num_layers = len(kv_samples[0])
    out = [[] for _ in range(num_layers)]
    for sample in kv_samples:
        for layer_idx in range(num_layers):
            out[layer_idx].append(compute_absmax_per_group(sample[layer_idx], group_size))
    return out


def scales_from_absmax_samples(absmax_samples, clip_percentile: float, qmax: float):
    """Per-layer static scales fp32 [kv_heads, num_groups]: torch.quantile of the
    sample-level absmax at clip_percentile / 100 over the samples, clamped to 1e-5, divided
    by qmax (scripts/calibrate_behavior.py:784-811).  An empty layer raises ValueError."""
    scales = []
    for layer_idx, layer in enumerate(absmax_samples):
        if not layer:
            raise ValueError(f"absmax_samples[{layer_idx}] is empty — no calibration samples "
                             f"collected for layer {layer_idx}. Check that num_layers matches "
                             "the model.")
        stack = torch.stack(list(layer), dim=0).float()
        absmax = torch.quantile(stack, clip_percentile / 100.0, dim=0)
        scales.append(absmax.clamp(min=1e-5) / float(qmax))
    return scales


def calibration_json(k_scales, v_scales, *, group_size: int, clip_percentile_k: float,
                     clip_percentile_v: Optional[float] = None, inv_tau=None,
                     quant_bits: int = 8, outlier_ratio: float = 0.0,
                     mixed_rescue: bool = False) -> dict:
    """The calibration JSON (as a dict) that ``load_calibration_json`` and the reference's
    loader read (src/engine/generate_loop.py:769-849): k_scale / v_scale [L, Hkv, G],
    optional inv_tau [L, Hq], the group size and clip percentiles, and for INT4 the rescue
    settings."""
    ks = torch.stack([t.float() for t in k_scales]).tolist()
    vs = torch.stack([t.float() for t in v_scales]).tolist()
    out = {"version": 2, "quant_bits": int(quant_bits), "k_scale": ks, "v_scale": vs,
           "group_size_k": int(group_size), "group_size_v": int(group_size),
           "clip_percentile_k": float(clip_percentile_k),
           "clip_percentile_v": float(clip_percentile_k if clip_percentile_v is None
                                      else clip_percentile_v)}
    if inv_tau is not None:
        out["inv_tau"] = torch.as_tensor(inv_tau).float().tolist()
    if quant_bits == 4:
        out["int4_outlier_ratio"] = float(outlier_ratio)
        out["int4_mixed_rescue"] = bool(mixed_rescue)
    return out


def int8_static_scale(sample: torch.Tensor, group_size: int) -> torch.Tensor:
    """fp16 [Hkv, G] (INT8 tables are loaded as fp16, generate_loop.py:816-817)."""
    return absmax_scale(sample, group_size, 127.0).to(torch.float16)


def int4_static_scale(sample: torch.Tensor, group_size: int) -> torch.Tensor:
    """fp32 [Hkv, G] (INT4 tables stay fp32, generate_loop.py:818-820)."""
    return absmax_scale(sample, group_size, 7.0)


def select_outlier_channels(sample: torch.Tensor, n: int = 4) -> torch.Tensor:
    """int32 [Hkv, n]: the n channels with the largest absmax per kv head (sorted)."""
    x = sample.float()
    if x.ndim == 3:
        x = x[None]
    am = x.abs().amax(dim=(0, 2))  # [Hkv, D]
    idx = am.topk(n, dim=-1).indices
    return idx.sort(dim=-1).values.to(torch.int32)


def asym_g32_params(sample: torch.Tensor, outlier_idx: Optional[torch.Tensor] = None):
    """(scale fp16 [Hkv, 4], zero_point fp16 [Hkv, 4]) for the asymmetric group-32 format."""
    x = sample.float()
    if x.ndim == 3:
        x = x[None]
    N, H, T, D = x.shape
    lo = x.clone()
    hi = x.clone()
    if outlier_idx is not None:
        for h in range(H):
            ch = outlier_idx[h].long()
            lo[:, h, :, ch] = float("inf")
            hi[:, h, :, ch] = float("-inf")
    g = lambda t: t.permute(1, 0, 2, 3).reshape(H, N * T, D // 32, 32)
    t_min = g(lo).amin(dim=(1, 3))
    t_max = g(hi).amax(dim=(1, 3))
    scale = (t_max - t_min).clamp(min=RANGE_FLOOR_INT4) / 15.0
    zp = t_min + 8.0 * scale
    return scale.to(torch.float16), zp.to(torch.float16)


@dataclass
class CalibTables:
    k_scale: Optional[torch.Tensor]
    v_scale: Optional[torch.Tensor]
    inv_tau: Optional[torch.Tensor]
    group_size: Optional[int]
    outlier_ratio: float
    mixed_rescue: bool


def load_calibration_json(path: str, quant_bits: int = 8) -> CalibTables:
    """Read a calibration JSON with the schema of generate_loop.py:769-849.

    Raises ValueError when a required table is missing or malformed, as the reference
    loader does.
    """
    with open(path, "r", encoding="utf-8") as f:
        data = json.load(f)
    dtype = torch.float16 if quant_bits == 8 else torch.float32
    ks = data.get("k_scale")
    vs = data.get("v_scale")
    if ks is None or vs is None:
        raise ValueError(f"calibration file {path} has no k_scale/v_scale")
    k_scale = torch.tensor(ks, dtype=torch.float32).to(dtype)
    v_scale = torch.tensor(vs, dtype=torch.float32).to(dtype)
    if k_scale.ndim != 3 or v_scale.shape != k_scale.shape:
        raise ValueError(f"k_scale/v_scale must be [L, Hkv, G], got {tuple(k_scale.shape)}")
    inv_tau = data.get("inv_tau")
    inv_tau_t = None if inv_tau is None else torch.tensor(inv_tau, dtype=torch.float32)
    if inv_tau_t is not None and inv_tau_t.ndim != 2:
        raise ValueError(f"inv_tau must be [L, Hq], got {tuple(inv_tau_t.shape)}")
    gs = data.get("group_size_k", data.get("group_size"))
    return CalibTables(
        k_scale=k_scale,
        v_scale=v_scale,
        inv_tau=inv_tau_t,
        group_size=None if gs is None else int(gs),
        outlier_ratio=float(data.get("int4_outlier_ratio", 0.0) or 0.0),
        mixed_rescue=bool(data.get("int4_mixed_rescue", False)),
    )
