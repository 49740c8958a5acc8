"""CPU restatement of the reference quantize-on-append arithmetic (test infrastructure).

Every function follows a reference function op for op, using PyTorch-CPU tensor
ops in the same dtypes.  The reference path is itself PyTorch, so this is the most
direct restatement.  The citations are to /root/reference/src.

Scalar divisions (``absmax / 127.0`` etc.) are true divisions here, as on torch-CPU.
On CUDA, torch multiplies by the reciprocal instead; only the dynamic and adaptive
scale paths contain such divisions.  The static-scale paths of the north star divide
tensor by tensor and agree on both devices.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

CLAMP_MIN = 1e-5


def check_finite(x: torch.Tensor, name: str) -> None:
    """src/quant/_common.py:13-20 -- NaN/Inf inputs are rejected with ValueError."""
    if x.numel() == 0:
        return
    if torch.isnan(x).any():
        raise ValueError(f"{name}: input contains NaN — refusing to quantize corrupt data")
    if torch.isinf(x).any():
        raise ValueError(f"{name}: input contains Inf — refusing to quantize corrupt data")


def normalize_static_scale(scale: torch.Tensor, B: int, H: int, S: int, G: int) -> torch.Tensor:
    """Broadcast a static scale to [B, H, S, G, 1] (src/quant/_common.py:37-135).

    Accepted layouts: [H, G]; [B, H, G] / [1, H, G]; [B, H, S, G]; [B, H, S, G, 1].
    """
    if scale.ndim == 2:
        if scale.shape[0] != H:
            raise ValueError(f"calibration vs model heads mismatch: {scale.shape[0]} vs {H}")
        view = scale[None, :, None, :, None]
    elif scale.ndim == 3:
        if scale.shape[1] != H or scale.shape[2] != G or scale.shape[0] not in (1, B):
            raise ValueError(f"Unsupported 3D scale shape: {tuple(scale.shape)}")
        view = scale[:, :, None, :, None]
    elif scale.ndim == 4:
        if scale.shape[1] != H:
            raise ValueError(f"calibration vs model heads mismatch: {scale.shape[1]} vs {H}")
        view = scale[..., None]
    elif scale.ndim == 5:
        view = scale
    else:
        raise ValueError(f"Unsupported scale ndim={scale.ndim}, shape={tuple(scale.shape)}")
    return view.expand(B, H, S, G, 1)


def quantize_symmetric_int8_with_scale(
    x: torch.Tensor, scale: torch.Tensor, group_size: int
) -> Tuple[torch.Tensor, torch.Tensor]:
    """src/quant/int8_basic.py:111-164.

    The scale is clamped to 1e-5 and cast to x's dtype (fp16).  The quotient
    x / s is computed in fp16, so it is rounded to fp16 before torch.round
    (ties to even).  The result is clamped to [-127, 127].
    """
    if not x.is_floating_point():
        raise ValueError(f"Input tensor must be float, got {x.dtype}")
    check_finite(x, "quantize_symmetric_int8_with_scale")
    D = x.shape[-1]
    gs = D if group_size == -1 else group_size
    if D % gs:
        raise ValueError(f"head_dim {D} must be divisible by group_size {gs}")
    B, H, S, _ = x.shape
    G = D // gs
    xr = x.view(B, H, S, G, gs)
    s = normalize_static_scale(scale, B, H, S, G).clamp(min=CLAMP_MIN).to(x.dtype)
    q = torch.round(xr / s).clamp(-127, 127).to(torch.int8)
    return q.view(B, H, S, D), s.squeeze(-1)


def _group_absmax(xr: torch.Tensor, percentile: float) -> torch.Tensor:
    """|x| per group: its maximum (in x's dtype), or below percentile 100 its torch.quantile
    at percentile / 100 in fp32 (src/quant/int8_basic.py:76-85, int4_basic.py:80-92)."""
    a = xr.abs()
    if percentile < 100.0:
        q = max(min(percentile / 100.0, 1.0), 0.0)
        return torch.quantile(a.float(), q, dim=-1, keepdim=True)
    return torch.amax(a, dim=-1, keepdim=True)


def quantize_symmetric_int8(
    x: torch.Tensor, percentile: float = 100.0, group_size: int = 128
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dynamic INT8 (src/quant/int8_basic.py:18-108): abs_max per group (absmax, or the
    percentile's torch.quantile), clamped to 1e-5, cast to x's dtype, divided by 127 in that
    dtype; codes round(x / s) in x's dtype, clamped to [-127, 127]."""
    check_finite(x, "quantize_symmetric_int8")
    B, H, S, D = x.shape
    gs = D if group_size == -1 else group_size
    G = D // gs
    xr = x.view(B, H, S, G, gs)
    am = _group_absmax(xr, percentile).clamp(min=CLAMP_MIN).to(x.dtype)
    s = am / 127.0
    q = torch.round(xr / s).clamp(-127, 127).to(torch.int8)
    return q.view(B, H, S, D), s.squeeze(-1)


def quantize_symmetric_int4_with_scale(
    x: torch.Tensor, scale: torch.Tensor, group_size: int
) -> Tuple[torch.Tensor, torch.Tensor]:
    """src/quant/int4_basic.py:115-159: fp32 scale clamped to 1e-5, fp32 quotient,
    round half to even, clamp to [-7, 7]."""
    if not x.is_floating_point():
        raise ValueError(f"Input tensor must be float, got {x.dtype}")
    check_finite(x, "quantize_symmetric_int4_with_scale")
    B, H, S, D = x.shape
    gs = D if group_size == -1 else group_size
    G = D // gs
    xr = x.view(B, H, S, G, gs)
    s = normalize_static_scale(scale, B, H, S, G).to(torch.float32).clamp(min=CLAMP_MIN)
    q = torch.round(xr / s).clamp(-7, 7).to(torch.int8)
    return q.view(B, H, S, D), s.squeeze(-1)


def quantize_symmetric_int4(
    x: torch.Tensor, percentile: float = 100.0, group_size: int = 32
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dynamic INT4 (src/quant/int4_basic.py:24-112): abs_max per group (absmax, or the
    percentile's torch.quantile), clamped to 1e-5, in fp32, divided by 7; codes
    round(x / s) in fp32, clamped to [-7, 7]; fp32 scales."""
    check_finite(x, "quantize_symmetric_int4")
    B, H, S, D = x.shape
    gs = D if group_size == -1 else group_size
    G = D // gs
    xr = x.view(B, H, S, G, gs)
    am = _group_absmax(xr, percentile).clamp(min=CLAMP_MIN).to(torch.float32)
    s = am / 7.0
    q = torch.round(xr / s).clamp(-7, 7).to(torch.int8)
    return q.view(B, H, S, D), s.to(torch.float32).squeeze(-1)


def dequantize_symmetric(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """src/quant/int8_basic.py:167-246 and src/quant/int4_basic.py:162-227 with a 4-D scale
    [B, H, S, G] (paths B / B'): the codes in the scale's dtype times the group's scale,
    result in the scale's dtype."""
    if q.dtype != torch.int8:
        raise ValueError(f"quantized must be torch.int8, got {q.dtype}")
    B, H, S, D = q.shape
    G = scale.shape[-1]
    if G <= 0 or D % G:
        raise ValueError(f"Invalid scale shape: quantized={tuple(q.shape)}, scale={tuple(scale.shape)}")
    if G == 1:
        return q.to(scale.dtype) * scale
    return (q.view(B, H, S, G, D // G).to(scale.dtype) * scale.unsqueeze(-1)).view(B, H, S, D)


def cache_get_kv(codes: torch.Tensor, scale: torch.Tensor, dtype=torch.float16) -> torch.Tensor:
    """INT8KVCache / INT4KVCache.get_kv of one side (src/cache/int8_cache.py:490-542,
    src/cache/int4_cache.py:591-649): the stored fp32 scales (INT8 keeps its fp16 scale
    widened) times the codes in fp32, then cast to the cache dtype."""
    return dequantize_symmetric(codes, scale.to(torch.float32)).to(dtype)


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """src/quant/int4_basic.py:230-272: +8 offset, high nibble = element 2i."""
    if q.dtype != torch.int8:
        raise ValueError(f"pack_int4 expects int8 input, got {q.dtype}")
    if q.shape[-1] % 2:
        raise ValueError("Last dimension must be even for packing")
    u = (q.to(torch.int16) + 8).to(torch.uint8)
    u = u.view(*q.shape[:-1], q.shape[-1] // 2, 2)
    return ((u[..., 0] << 4) | u[..., 1]).to(torch.int8)


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """src/quant/int4_basic.py:275-303."""
    if packed.dtype not in (torch.int8, torch.uint8):
        raise ValueError(f"unpack_int4 expects int8 packed input, got {packed.dtype}")
    u = packed.view(torch.uint8) if packed.dtype == torch.int8 else packed
    hi = (u >> 4) & 0x0F
    lo = u & 0x0F
    out = torch.stack([hi, lo], dim=-1).view(*packed.shape[:-1], packed.shape[-1] * 2)
    return (out.to(torch.int16) - 8).to(torch.int8)


# ---------------------------------------------------------------- cache scale policies


def int8_cache_quantize(
    x: torch.Tensor,
    static_scale: Optional[torch.Tensor],
    group_size: int,
    adaptive: bool = False,
    margin: float = 1.0,
    clip_percentile: float = 100.0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The quantize step of INT8KVCache.append (src/cache/int8_cache.py:389-453).

    Returns (codes int8 [B,H,S,D], scale [B,H,S,G] in the quantizer's dtype).
    """
    if static_scale is None:
        return quantize_symmetric_int8(x, clip_percentile, group_size)
    scale = static_scale
    if adaptive:
        B, H, S, D = x.shape
        G = D // group_size
        st = _expand_cache_scale(scale, B, H, S, G).to(torch.float32).clamp(min=CLAMP_MIN)
        dyn = x.view(B, H, S, G, group_size).abs().amax(dim=-1).float().clamp(min=CLAMP_MIN) / 127.0
        scale = torch.maximum(st * float(margin), dyn)
    return quantize_symmetric_int8_with_scale(x, scale, group_size)


def _expand_cache_scale(scale, B, H, S, G):
    """src/cache/int8_cache.py:298-326 / int4_cache.py:317-342."""
    if scale.ndim == 2:
        v = scale[None, :, None, :]
    elif scale.ndim == 4:
        v = scale
    elif scale.ndim == 5 and scale.shape[-1] == 1:
        v = scale.squeeze(-1)
    else:
        raise ValueError(f"Unsupported static scale shape: {tuple(scale.shape)}")
    return v.expand(B, H, S, G)


def int4_dynamic_group_scale(x: torch.Tensor, group_size: int) -> torch.Tensor:
    """src/cache/int4_cache.py:344-358: absmax/7 per (b, h, s, group), fp32."""
    B, H, S, D = x.shape
    am = x.view(B, H, S, D // group_size, group_size).abs().amax(dim=-1)
    return am.float().clamp(min=CLAMP_MIN) / 7.0


def outlier_rescue(x: torch.Tensor, scale: torch.Tensor, ratio: float, group_size: int) -> torch.Tensor:
    """src/cache/int4_cache.py:360-390 (global torch.quantile threshold)."""
    if ratio <= 0.0:
        return scale
    dyn = int4_dynamic_group_scale(x, group_size)
    if ratio >= 1.0:
        return torch.maximum(scale, dyn)
    thr = torch.quantile(dyn.float().reshape(-1), max(0.0, min(1.0, 1.0 - ratio))).to(dyn.dtype)
    return torch.where(dyn >= thr, torch.maximum(scale, dyn), scale)


def int4_cache_quantize(
    x: torch.Tensor,
    static_scale: Optional[torch.Tensor],
    group_size: int,
    adaptive: bool = False,
    margin: float = 1.0,
    mixed_rescue: bool = False,
    outlier_rescue_ratio: float = 0.0,
    clip_percentile: float = 100.0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The quantize step of INT4KVCache.append (src/cache/int4_cache.py:447-529).

    Returns (codes int8 in [-7, 7] [B,H,S,D], fp32 scale [B,H,S,G]).
    """
    if static_scale is None:
        return quantize_symmetric_int4(x, clip_percentile, group_size)
    B, H, S, D = x.shape
    G = D // group_size
    s = _expand_cache_scale(static_scale, B, H, S, G).to(torch.float32).clamp(min=CLAMP_MIN)
    if adaptive:
        s = torch.maximum(s * float(margin), int4_dynamic_group_scale(x, group_size))
    if mixed_rescue:
        s = torch.maximum(s, int4_dynamic_group_scale(x, group_size))
    s = outlier_rescue(x, s, outlier_rescue_ratio, group_size)
    q, s = quantize_symmetric_int4_with_scale(x, s, group_size)
    return q, s.to(torch.float32)


# ---------------------------------------------------------------- asymmetric, static g32


def quantize_asymmetric_static(
    x: torch.Tensor, scale16: torch.Tensor, zp16: torch.Tensor, group_size: int = 32
) -> torch.Tensor:
    """Asymmetric INT4 with static per-(head, group) parameters.

    The element formula is the reference's static-parameter K quantizer:
    q = clamp(round((fp32(x) - zp) / s), -8, 7).  See
    tests/test_fused_quantize_pack.py:8-17 and src/kernels/triton_quantize_pack_int4.py:51-55.
    Here it is applied per group of 32 channels with fp16 parameters widened to fp32
    (the BASELINE g32 format).  Returns int8 codes [B,H,S,D] in [-8, 7].
    """
    check_finite(x, "quantize_asymmetric_static")
    B, H, S, D = x.shape
    G = D // group_size
    xr = x.float().view(B, H, S, G, group_size)
    s = scale16.float()[None, :, None, :, None]
    z = zp16.float()[None, :, None, :, None]
    q = torch.round((xr - z) / s).clamp(-8, 7).to(torch.int8)
    return q.view(B, H, S, D)


def dequantize_asymmetric_static(q: torch.Tensor, scale16, zp16, group_size: int = 32) -> torch.Tensor:
    """q * s + zp in fp32 (src/quant/asymmetric_quant.py:196 with fp32 parameters)."""
    B, H, S, D = q.shape
    G = D // group_size
    s = scale16.float()[None, :, None, :, None]
    z = zp16.float()[None, :, None, :, None]
    return (q.view(B, H, S, G, group_size).float() * s + z).view(B, H, S, D)


# ---------------------------------------------------------------- KIVI (asymmetric, fp32)


def quantize_asymmetric(x: torch.Tensor, axis: int, quant_bits: int = 4,
                        percentile: float = 100.0):
    """Asymmetric quantization along one axis (src/quant/asymmetric_quant.py:24-141):
    t_min / t_max over the axis in fp32 (torch.quantile of both tails for percentile < 100),
    s = max(t_max - t_min, max(1e-5, fp16_tiny * (qmax - qmin))) / (qmax - qmin),
    z = t_min - qmin * s, q = clamp(round((x - z) / s), qmin, qmax).
    Returns (int8 codes, fp32 s, fp32 z) with the axis removed from s and z."""
    check_finite(x, "quantize_asymmetric")
    if quant_bits not in (4, 8):
        raise ValueError(f"quant_bits must be 4 or 8, got {quant_bits}")
    if not (50.0 < percentile <= 100.0):
        raise ValueError(f"percentile must be in (50.0, 100.0], got {percentile}")
    qmin, qmax = (-128, 127) if quant_bits == 8 else (-8, 7)
    axis = axis + x.ndim if axis < 0 else axis
    xf = x.float()
    if percentile < 100.0:
        t_min = torch.quantile(xf, (100.0 - percentile) / 100.0, dim=axis, keepdim=True)
        t_max = torch.quantile(xf, percentile / 100.0, dim=axis, keepdim=True)
    else:
        t_min = xf.amin(dim=axis, keepdim=True)
        t_max = xf.amax(dim=axis, keepdim=True)
    floor = max(1e-5, float(torch.finfo(torch.float16).tiny) * (qmax - qmin))
    s = (t_max - t_min).clamp(min=floor) / (qmax - qmin)
    z = t_min - qmin * s
    q = torch.round((xf - z) / s).clamp(qmin, qmax).to(torch.int8)
    return q, s.squeeze(axis), z.squeeze(axis)


def quantize_asymmetric_per_channel(k: torch.Tensor, quant_bits: int = 4, percentile: float = 100.0):
    """K [B,H,S,D] over the tokens: s, z [B,H,D] (src/quant/asymmetric_quant.py:199-224)."""
    return quantize_asymmetric(k, 2, quant_bits, percentile)


def quantize_asymmetric_per_token(v: torch.Tensor, quant_bits: int = 4, percentile: float = 100.0):
    """V [B,H,S,D] over the channels: s, z [B,H,S] (src/quant/asymmetric_quant.py:246-270)."""
    return quantize_asymmetric(v, 3, quant_bits, percentile)


def kivi_quantize_k_static(k: torch.Tensor, s: torch.Tensor, z: torch.Tensor, bits: int = 4) -> torch.Tensor:
    """Decode-time K with the frozen per-channel parameters [B,H,D]
    (src/cache/kivi_style_cache.py:548-566, src/cache/role_aware_allocator_cache.py:292-309):
    clamp(round((fp32(k) - z) / s), qmin, qmax), [-8, 7] for 4 bits, [-128, 127] for 8."""
    check_finite(k, "kivi_quantize_k_static")
    qmin, qmax = (-8, 7) if bits == 4 else (-128, 127)
    return torch.round((k.float() - z.float().unsqueeze(2)) / s.float().unsqueeze(2)) \
        .clamp(qmin, qmax).to(torch.int8)


def dequantize_kivi(q: torch.Tensor, s: torch.Tensor, z: torch.Tensor, per_channel: bool) -> torch.Tensor:
    """q * s + z in fp32 (src/quant/asymmetric_quant.py:144-196): s, z [B,H,D] broadcast
    over tokens (per channel) or [B,H,S] over channels (per token)."""
    if per_channel:
        return q.float() * s.float().unsqueeze(2) + z.float().unsqueeze(2)
    return q.float() * s.float().unsqueeze(-1) + z.float().unsqueeze(-1)
