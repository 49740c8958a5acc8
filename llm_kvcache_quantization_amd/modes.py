"""The kv_mode switch of the decode path (src/engine/generate_loop.py:393-1581, subset).

* :func:`load_calibration` -- the calibration-JSON rules of generate_loop.py:751-889 (the
  tables' dtypes, group-size / percentile precedence, the warnings, the missing-file and
  load-failure policy).
* :func:`create_kv_cache` -- the engine of each mode (generate_loop.py:891-1176):
  ``fp16`` -> :class:`FP16KVCache`; ``int8_baseline`` / ``int8_fused`` / ``int8_ours`` ->
  :class:`INT8KVCache`; ``int4_baseline`` / ``int4_fused`` / ``int4_ours`` /
  ``int4_ours_mixed`` -> :class:`INT4KVCache`; ``kivi_style`` / ``int4_kivi_aligned`` ->
  :class:`KIVIStyleKVCache`; ``int4_ours_asym`` / ``int4_ours_asym_ba`` ->
  :class:`RoleAwareAsymKVCache`; ``int4_ours_asym_alloc`` -> :class:`RoleAwareAllocatorKVCache`
  (per-layer bits from a policy JSON); ``int4_mixed_kv`` -> :class:`MixedKVCache`.
* :func:`generate_from_ids` -- greedy generation with an explicit prefill (the model's own
  attention; the quantized cache is filled from its past_key_values) and token-by-token
  decode, timed per step with a device synchronisation as the reference's CUDATimer does.
  The fused modes decode through the attention hook (:mod:`patch`); fp16 decodes through
  the model's own cache; the baseline modes hand the dequantized cache to the model.

The KIVI-family and mixed modes (``kivi_style``, ``int4_kivi_aligned``, ``int4_ours_asym*``,
``int4_mixed_kv``): the reference decodes them by dequantizing before attention (it forces
decode_attn_impl="torch_ref" for all but ``int4_ours_asym*``); here "torch_ref" keeps that,
and the kernel names ("triton_fused", "hip_fused", "triton_int4_asym*") decode through the
hook with the HIP kernel of each layer's format.
"""
from __future__ import annotations

import json
import os
import time
import warnings
from dataclasses import dataclass, field
from typing import List, Optional

import torch

from .cache import (FP16KVCache, INT4KVCache, INT8KVCache, KIVIStyleKVCache, MixedKVCache,
                    RoleAwareAllocatorKVCache, RoleAwareAsymKVCache, load_per_layer_bits_from_policy)

# src/engine/generate_loop.py:44-46
_FUSED_KV_MODES = frozenset({"int8_fused", "int8_ours", "int4_fused", "int4_ours", "int4_ours_mixed"})
# modes whose engines the reference decodes by dequantizing (torch_ref) and the HIP kernels
# can decode in place
_KERNEL_FUSABLE = frozenset({"kivi_style", "int4_kivi_aligned", "int4_ours_asym", "int4_ours_asym_ba",
                             "int4_ours_asym_alloc", "int4_mixed_kv"})
KV_MODES = ("fp16", "int8_baseline", "int8_fused", "int8_ours", "int4_baseline", "int4_fused",
            "int4_ours", "int4_ours_mixed", "kivi_style", "int4_kivi_aligned", "int4_mixed_kv",
            "int4_ours_asym", "int4_ours_asym_ba", "int4_ours_asym_alloc")
_NOT_BUILT_MODES: tuple = ()
# the reference's kernel names map to the HIP kernels; torch_ref is its torch decode path
DECODE_ATTN_IMPLS = ("triton_fused", "hip_fused", "torch_ref", "triton_int4_asym",
                     "triton_int4_asym_v2", "triton_int4_asym_gqa")
_CALIB_MODES = ("int8_ours", "int4_ours", "int4_ours_mixed", "int4_fused")


@dataclass
class Calibration:
    """What load_calibration resolved for a mode (None: not used / not present)."""
    static_k_scale: Optional[torch.Tensor] = None
    static_v_scale: Optional[torch.Tensor] = None
    inv_tau: Optional[torch.Tensor] = None
    group_size: Optional[int] = None
    clip_percentile: Optional[float] = None
    outlier_rescue_ratio: float = 0.0
    mixed_rescue: bool = False
    path: Optional[str] = None


def check_kv_mode(kv_mode: str) -> None:
    if kv_mode not in KV_MODES:
        raise ValueError(f"kv_mode='{kv_mode}' not supported. Choose from {list(KV_MODES)}.")


def load_calibration(kv_mode: str, calib_file: Optional[str], group_size: int = 128,
                     clip_percentile: float = 99.9, use_static_scales: bool = True,
                     use_attn_temperature: bool = True, allow_missing_calib: bool = False,
                     device=None) -> Calibration:
    """The calibration tables of a mode (src/engine/generate_loop.py:751-889).

    Only int8_ours / int4_ours / int4_ours_mixed / int4_fused read a table.  INT8 scales
    load as fp16, INT4 scales as fp32, inv_tau as fp32 [L, Hq]; ``group_size_k`` and
    ``clip_percentile_k`` override the arguments.  A missing file raises FileNotFoundError
    and an unreadable one RuntimeError, unless allow_missing_calib, which warns and
    continues without tables.  The reference's default table paths
    (artifacts/kv_calib_*.json of its checkout) are not shipped here: calib_file is needed.
    """
    cal = Calibration(group_size=group_size, clip_percentile=clip_percentile)
    if kv_mode not in _CALIB_MODES:
        return cal
    if not calib_file or not os.path.exists(calib_file):
        msg = f"kv_mode={kv_mode} requires a calibration file, but it was not found: {calib_file}."
        if allow_missing_calib:
            warnings.warn(f"Calibration file not found: {calib_file}. Falling back to baseline behavior.",
                          UserWarning)
            return cal
        raise FileNotFoundError(msg + " Produce one with the reference's calibration script.")
    try:
        with open(calib_file, "r", encoding="utf-8") as f:
            data = json.load(f)
        if data.get("version", 0) < 2:
            warnings.warn(
                f"Calibration file '{calib_file}' has version={data.get('version', 0)} (expected >=2). "
                "Legacy v1 calibration lacks provenance fields (model_revision, seed, dataset_source). "
                "Results may not be reproducible.", UserWarning)
        gk = data.get("group_size_k", data.get("group_size", group_size))
        gv = data.get("group_size_v", data.get("group_size", group_size))
        ck = data.get("clip_percentile_k", data.get("clip_percentile", clip_percentile))
        cv = data.get("clip_percentile_v", data.get("clip_percentile", clip_percentile))
        if gk and gv and gk != gv:
            warnings.warn(f"CAL-022: Calibration group_size_k ({gk}) != group_size_v ({gv}); the cache "
                          "engine uses a single group_size for both K and V. group_size_k will be used "
                          "for both; group_size_v is discarded.", UserWarning)
        if ck and cv and ck != cv:
            warnings.warn(f"CAL-022: Calibration clip_percentile_k ({ck}) != clip_percentile_v ({cv}); "
                          "clip_percentile_k will be used for both; clip_percentile_v is discarded.",
                          UserWarning)
        cal.group_size = int(gk) if gk is not None else group_size
        cal.clip_percentile = float(ck) if ck is not None else clip_percentile
        dt = torch.float32 if kv_mode.startswith("int4") else torch.float16
        if use_static_scales and "k_scale" in data:
            cal.static_k_scale = torch.tensor(data["k_scale"], dtype=dt)
        if use_static_scales and "v_scale" in data:
            cal.static_v_scale = torch.tensor(data["v_scale"], dtype=dt)
        if use_static_scales:
            if "k_scale" in data and "v_scale" not in data:
                warnings.warn("ENG-048: Calibration file has 'k_scale' but no 'v_scale'. K uses static "
                              "scales; V will use dynamic quantization.", UserWarning)
            elif "v_scale" in data and "k_scale" not in data:
                warnings.warn("ENG-048: Calibration file has 'v_scale' but no 'k_scale'. V uses static "
                              "scales; K will use dynamic quantization.", UserWarning)
        if use_attn_temperature and "inv_tau" in data:
            cal.inv_tau = torch.tensor(data["inv_tau"], dtype=torch.float32)
        cal.outlier_rescue_ratio = float(data.get("int4_outlier_ratio", 0.0) or 0.0)
        cal.mixed_rescue = bool(data.get("int4_mixed_rescue", False)) or kv_mode == "int4_ours_mixed"
        cal.path = calib_file
        if device is not None:
            for name in ("static_k_scale", "static_v_scale", "inv_tau"):
                t = getattr(cal, name)
                if t is not None:
                    setattr(cal, name, t.to(device))
    except Exception as exc:
        if allow_missing_calib:
            warnings.warn(
                f"Failed to load calibration file {calib_file}: {exc}. Falling back to dynamic-only "
                f"quantization (no static scales, no inv_tau temperature). kv_mode is still "
                f"'{kv_mode}' but effective behavior is equivalent to baseline.", UserWarning)
            return Calibration(group_size=group_size, clip_percentile=clip_percentile)
        raise RuntimeError(f"Failed to load calibration file {calib_file}: {exc}.") from exc
    return cal


@dataclass
class RoleCalibration:
    """What the KIVI-family modes read from a calibration file (None / 100: not present)."""
    k_percentile: float = 100.0
    v_percentile: float = 100.0
    inv_tau: Optional[torch.Tensor] = None


def _resolve_calib_path(kv_mode: str, calib_file: str, project_root: Optional[str]) -> str:
    path = calib_file if os.path.isabs(calib_file) or project_root is None \
        else os.path.join(project_root, calib_file)
    if not os.path.exists(path):
        raise FileNotFoundError(f"{kv_mode}: calib_file={calib_file!r} not found (resolved to {path!r}). "
                                "Use an absolute path or run from the project root.")
    return path


def load_role_calibration(kv_mode: str, calib_file: Optional[str], project_root: Optional[str] = None,
                          device=None) -> RoleCalibration:
    """The calibration of the KIVI-family modes (src/engine/generate_loop.py:955-1131).

    * int4_kivi_aligned: inv_tau from ``k_calibration.inv_tau`` (v3 schema), else top-level
      ``inv_tau``; v_percentile from ``v_calibration.v_percentile``.
    * int4_ours_asym / _ba / _alloc: k_percentile and v_percentile from the ``role_aware``
      section, else (warning) from ``k_calibration.k_percentile`` / the top level and
      ``v_calibration.v_percentile``; int4_ours_asym_ba also takes inv_tau (``role_aware``,
      then ``k_calibration``, then top level).
    A relative path resolves against project_root (the reference's repository root); a
    missing file raises FileNotFoundError."""
    rc = RoleCalibration()
    if calib_file is None or kv_mode not in ("int4_kivi_aligned", "int4_ours_asym", "int4_ours_asym_ba",
                                             "int4_ours_asym_alloc"):
        return rc
    with open(_resolve_calib_path(kv_mode, calib_file, project_root), "r") as fh:
        data = json.load(fh)
    raw_tau = None
    if kv_mode == "int4_kivi_aligned":
        if "k_calibration" in data and "inv_tau" in data["k_calibration"]:
            raw_tau = data["k_calibration"]["inv_tau"]
        elif "inv_tau" in data:
            raw_tau = data["inv_tau"]
        if "v_calibration" in data and "v_percentile" in data["v_calibration"]:
            rc.v_percentile = float(data["v_calibration"]["v_percentile"])
    else:
        if "role_aware" in data:
            ra = data["role_aware"]
            rc.k_percentile = float(ra.get("k_percentile", 100.0))
            rc.v_percentile = float(ra.get("v_percentile", 100.0))
        elif "k_calibration" in data:
            if kv_mode == "int4_ours_asym_alloc":
                warnings.warn("Allocator RoleAlign mode using k_calibration fallback schema; consider "
                              "re-generating calibration with role_aware schema.", UserWarning)
            else:
                warnings.warn(f"RoleAlign mode '{kv_mode}' using k_calibration fallback schema; consider "
                              "re-generating calibration with role_aware schema.", UserWarning)
            kc = data["k_calibration"]
            rc.k_percentile = float(kc.get("k_percentile", data.get("k_percentile", 100.0)))
            if "v_calibration" in data:
                rc.v_percentile = float(data["v_calibration"].get("v_percentile", 100.0))
        if kv_mode == "int4_ours_asym_ba":
            if "role_aware" in data and "inv_tau" in data["role_aware"]:
                raw_tau = data["role_aware"]["inv_tau"]
            elif "k_calibration" in data and "inv_tau" in data["k_calibration"]:
                raw_tau = data["k_calibration"]["inv_tau"]
            elif "inv_tau" in data:
                raw_tau = data["inv_tau"]
    if raw_tau is not None:
        rc.inv_tau = torch.tensor(raw_tau, dtype=torch.float32, device=device)
    return rc


def create_kv_cache(kv_mode: str, num_layers: int, device="cuda", max_seq_len: Optional[int] = None,
                    calib: Optional[Calibration] = None, group_size: int = 128,
                    clip_percentile: float = 99.9, decode_attn_impl: str = "triton_fused",
                    use_attn_temperature: bool = True, adaptive_static_scales: bool = False,
                    adaptive_static_margin: float = 1.0, adaptive_static_k: bool = True,
                    adaptive_static_v: bool = True, quant_bits: Optional[int] = None, residual_length: int = 0,
                    check_numerics: bool = True, role: Optional[RoleCalibration] = None,
                    k_bits: Optional[int] = None, v_bits: Optional[int] = None,
                    per_layer_bits=None):
    """The cache engine of kv_mode (src/engine/generate_loop.py:891-1176)."""
    check_kv_mode(kv_mode)
    role = role or RoleCalibration()
    if kv_mode == "int4_kivi_aligned":
        return KIVIStyleKVCache(num_layers=num_layers, device=device, max_seq_len=max_seq_len, quant_bits=4,
                                v_percentile=role.v_percentile, inv_tau=role.inv_tau,
                                use_attn_temperature=use_attn_temperature, residual_length=residual_length,
                                decode_attn_impl=decode_attn_impl, check_numerics=check_numerics)
    if kv_mode in ("int4_ours_asym", "int4_ours_asym_ba"):
        ba = kv_mode == "int4_ours_asym_ba"
        return RoleAwareAsymKVCache(num_layers=num_layers, device=device, max_seq_len=max_seq_len, quant_bits=4,
                                    k_percentile=role.k_percentile, v_percentile=role.v_percentile,
                                    inv_tau=role.inv_tau if ba else None,
                                    use_attn_temperature=use_attn_temperature and ba,
                                    framework="ours_asym_ba" if ba else "ours_asym",
                                    decode_attn_impl=decode_attn_impl, check_numerics=check_numerics)
    if kv_mode == "int4_ours_asym_alloc":
        if per_layer_bits is None:
            raise ValueError("kv_mode='int4_ours_asym_alloc' requires a non-empty policy_json")
        return RoleAwareAllocatorKVCache(num_layers, per_layer_bits=per_layer_bits, device=device,
                                         max_seq_len=max_seq_len, k_percentile=role.k_percentile,
                                         v_percentile=role.v_percentile, framework="ours_asym_allocator",
                                         residual_length=residual_length, decode_attn_impl=decode_attn_impl,
                                         check_numerics=check_numerics)
    if kv_mode == "int4_mixed_kv":
        return MixedKVCache(num_layers=num_layers, device=device, max_seq_len=max_seq_len,
                            k_group_size=group_size, v_group_size=group_size, k_clip_percentile=clip_percentile,
                            v_percentile=clip_percentile, k_bits=8 if k_bits is None else int(k_bits),
                            v_bits=4 if v_bits is None else int(v_bits), per_layer_bits=per_layer_bits,
                            decode_attn_impl=decode_attn_impl, check_numerics=check_numerics)
    cal = calib or Calibration(group_size=group_size, clip_percentile=clip_percentile)
    gs = cal.group_size if cal.group_size is not None else group_size
    cp = cal.clip_percentile if cal.clip_percentile is not None else clip_percentile
    if kv_mode == "fp16":
        return FP16KVCache(num_layers=num_layers, device=device, max_seq_len=max_seq_len)
    common = dict(num_layers=num_layers, device=device, clip_percentile=cp, group_size=gs,
                  max_seq_len=max_seq_len, decode_attn_impl=decode_attn_impl,
                  static_k_scale=cal.static_k_scale, static_v_scale=cal.static_v_scale,
                  inv_tau=cal.inv_tau, use_attn_temperature=use_attn_temperature,
                  adaptive_static_scales=adaptive_static_scales,
                  adaptive_static_margin=adaptive_static_margin, adaptive_static_k=adaptive_static_k,
                  adaptive_static_v=adaptive_static_v, check_numerics=check_numerics)
    if kv_mode in ("int8_baseline", "int8_fused", "int8_ours"):
        return INT8KVCache(**common)
    if kv_mode in ("int4_baseline", "int4_fused", "int4_ours", "int4_ours_mixed"):
        return INT4KVCache(**common, outlier_rescue_ratio=cal.outlier_rescue_ratio,
                           mixed_rescue=cal.mixed_rescue)
    return KIVIStyleKVCache(num_layers=num_layers, device=device, max_seq_len=max_seq_len,
                            quant_bits=8 if quant_bits is None else int(quant_bits),
                            residual_length=residual_length,
                            decode_attn_impl=decode_attn_impl, check_numerics=check_numerics)


@dataclass
class GenerationBatchOutput:
    """src/engine/generate_loop.py GenerationBatchOutput (the fields this subset fills)."""
    generated_ids: torch.Tensor
    ttft_ms: float
    tpot_ms: float
    decode_times_ms: List[float] = field(default_factory=list)
    kv_mode: str = "fp16"
    decode_attn_impl: str = "triton_fused"
    kv_cache_mem_mb: float = 0.0
    decode_stats: Optional[dict] = None


def _past_layers(pkv):
    """(k, v) per layer of a model's past_key_values: a legacy tuple, or a transformers
    Cache (whose iteration yields (keys, values, ...) in 5.x)."""
    if pkv is None:
        return []
    if hasattr(pkv, "layers"):
        return [(layer.keys, layer.values) for layer in pkv.layers]
    return [(item[0], item[1]) for item in pkv]


def _to_model_cache(pairs):
    from transformers.cache_utils import DynamicCache

    return DynamicCache(ddp_cache_data=[(k, v) for k, v in pairs])


def _temperature_hooks(model, inv_tau: torch.Tensor, all_steps: bool = False):
    """Per-head inv_tau on the prefill's queries: q_proj's output (or q_norm's) is scaled
    when the step has more than one token; decode steps are scaled by the fused forward
    (src/engine/generate_loop.py:276-390).  all_steps: decode steps too, for the modes whose
    decode runs the model's own attention over the dequantized cache
    (_register_all_temperature_hooks, generate_loop.py:184-274)."""
    lo = 0 if all_steps else 1
    handles = []
    layers = getattr(getattr(model, "model", None), "layers", None)
    if layers is None:
        warnings.warn("Cannot register prefill temperature hooks: model.model.layers not found. "
                      "Per-head temperature scaling will NOT be applied during prefill.", UserWarning)
        return handles
    if not isinstance(inv_tau, torch.Tensor) or inv_tau.ndim != 2:
        raise ValueError(f"inv_tau must be a 2D tensor [layers, heads], got {getattr(inv_tau, 'shape', None)}")
    heads_cfg = getattr(getattr(model, "config", None), "num_attention_heads", None)
    for li, layer in enumerate(layers):
        attn = getattr(layer, "self_attn", None)
        if attn is None:
            continue
        nh = getattr(attn, "num_heads", None) or getattr(attn, "_kv_num_attention_heads", None) or heads_cfg
        hd = getattr(attn, "head_dim", None)
        if nh is None or hd is None:
            continue
        if li >= inv_tau.shape[0]:
            raise ValueError(f"inv_tau has {inv_tau.shape[0]} layers but model has layer_idx={li}.")
        if inv_tau.shape[1] != int(nh):
            raise ValueError(f"inv_tau head count mismatch at layer {li}: inv_tau.shape[1]="
                             f"{inv_tau.shape[1]} vs model.num_heads={nh}.")
        tau = inv_tau[li]
        if getattr(attn, "q_norm", None) is not None:
            def hook(module, inputs, out, _t=tau, _h=int(nh)):
                if not isinstance(out, torch.Tensor) or out.ndim != 4:
                    return out
                if out.shape[1] == _h and out.shape[2] > lo:
                    return out * _t.to(out.device, out.dtype).view(1, -1, 1, 1)
                if out.shape[2] == _h and out.shape[1] > lo:
                    return out * _t.to(out.device, out.dtype).view(1, 1, -1, 1)
                return out
            handles.append(attn.q_norm.register_forward_hook(hook))
        elif getattr(attn, "q_proj", None) is not None:
            def hook(module, inputs, out, _t=tau, _h=int(nh), _d=int(hd)):
                if not isinstance(out, torch.Tensor) or out.ndim != 3 or out.shape[1] <= lo \
                        or out.shape[2] != _h * _d:
                    return out
                b, s, _ = out.shape
                return (out.view(b, s, _h, _d) * _t.to(out.device, out.dtype).view(1, 1, -1, 1)).view(b, s, -1)
            handles.append(attn.q_proj.register_forward_hook(hook))
    return handles


def _append_delta(kv_cache, layers, prev_lens, step_q_len: int) -> None:
    """Append the step's new K / V rows of each layer (src/engine/generate_loop.py:1368-1440):
    the whole returned slice when the model returned only the new rows, the tail past the
    cached length when it returned the whole cache; other growth warns (ENG-045A) and
    appends the tail, no growth warns (ENG-045B) and appends nothing."""
    for i, (k, v) in enumerate(layers):
        got, before = int(k.shape[2]), int(prev_lens[i])
        delta = got - before
        if got == step_q_len:
            kn, vn = k, v
        elif delta == step_q_len:
            kn, vn = k[:, :, before:got], v[:, :, before:got]
        elif delta > 0:
            warnings.warn(f"ENG-045A: Layer {i} unexpected KV growth: returned_len={got}, prev_len={before}, "
                          f"delta={delta}, expected_step_q_len={step_q_len}. Appending delta tail to "
                          "preserve forward progress.", RuntimeWarning, stacklevel=2)
            kn, vn = k[:, :, before:got], v[:, :, before:got]
        else:
            warnings.warn(f"ENG-045B: Layer {i} non-growing KV in decode: returned_len={got}, "
                          f"prev_len={before}. Skipping append.", RuntimeWarning, stacklevel=2)
            continue
        kv_cache.append(i, kn, vn)


def _sync():
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def generate_from_ids(model, tokenizer, input_ids: torch.Tensor, attention_mask=None,
                      max_new_tokens: int = 128, kv_mode: str = "fp16", group_size: int = 128,
                      clip_percentile: float = 99.9, seed: int = 1234, calib_file: Optional[str] = None,
                      use_attn_temperature: bool = True, use_static_scales: bool = True,
                      adaptive_static_scales: bool = False, adaptive_static_margin: float = 1.0,
                      adaptive_static_k: bool = True, adaptive_static_v: bool = True,
                      decode_attn_impl: str = "triton_fused", allow_missing_calib: bool = False,
                      stop_on_eos: bool = True, quant_bits: Optional[int] = None, residual_length: int = 0,
                      check_numerics: bool = True, k_bits: Optional[int] = None, v_bits: Optional[int] = None,
                      policy_json: Optional[str] = None,
                      project_root: Optional[str] = None) -> GenerationBatchOutput:
    """Greedy generation with explicit prefill + token-by-token decode
    (src/engine/generate_loop.py:393-1581, the modes of ``KV_MODES``).  Batches need
    uniform lengths (an all-ones attention mask), as in the reference."""
    from .patch import INT8CacheWrapperContainer, apply_int8_fused_patch, remove_int8_fused_patch

    check_kv_mode(kv_mode)
    if decode_attn_impl not in DECODE_ATTN_IMPLS:
        raise ValueError(f"decode_attn_impl={decode_attn_impl!r} not supported. Choose from "
                         f"{sorted(DECODE_ATTN_IMPLS)}.")
    if kv_mode == "int4_ours_asym_alloc" and policy_json is None:
        raise ValueError("kv_mode='int4_ours_asym_alloc' requires a non-empty policy_json")
    if not torch.cuda.is_available():
        raise RuntimeError("CUDA is required for generation. Please run on a GPU-enabled server.")
    if not isinstance(input_ids, torch.Tensor):
        raise TypeError(f"input_ids must be a torch.Tensor, got {type(input_ids)}")
    if input_ids.ndim != 2:
        raise ValueError(f"input_ids must have shape [B, S], got {tuple(input_ids.shape)}")
    dev = model.device
    input_ids = input_ids.to(device=dev, dtype=torch.long)
    B, S = int(input_ids.shape[0]), int(input_ids.shape[1])
    if B == 0 or S == 0:
        raise ValueError(f"input_ids must be non-empty, got shape {tuple(input_ids.shape)}")
    if attention_mask is None:
        attention_mask = torch.ones_like(input_ids)
    else:
        if attention_mask.shape != input_ids.shape:
            raise ValueError(f"attention_mask shape must match input_ids. Got attention_mask="
                             f"{tuple(attention_mask.shape)} input_ids={tuple(input_ids.shape)}")
        attention_mask = attention_mask.to(device=dev, dtype=torch.long)
    if B > 1 and not bool(torch.all(attention_mask == 1).item()):
        raise ValueError(f"Batched generation requires attention_mask to be all ones (no padding). "
                         f"Got batch={B} kv_mode={kv_mode}.")
    if decode_attn_impl.startswith("triton_int4_asym") and kv_mode not in _KERNEL_FUSABLE:
        raise ValueError(f"decode_attn_impl={decode_attn_impl!r} serves the asymmetric layouts "
                         f"(kv_mode in {sorted(_KERNEL_FUSABLE)})")
    if kv_mode == "int4_kivi_aligned":
        quant_bits = 4
        if calib_file is None and use_attn_temperature:
            warnings.warn("kv_mode='int4_kivi_aligned' with use_attn_temperature=True but no calib_file "
                          "— inv_tau will not be applied.", UserWarning)
        if use_static_scales:
            warnings.warn("kv_mode='int4_kivi_aligned' ignores use_static_scales (KIVI skeleton).", UserWarning)
    per_layer_bits = None
    if kv_mode in ("int4_mixed_kv", "int4_ours_asym_alloc") and policy_json is not None:
        per_layer_bits = load_per_layer_bits_from_policy(policy_json, project_root=project_root or os.getcwd())
    if kv_mode == "int4_ours_asym_alloc" and per_layer_bits is None:
        raise ValueError("kv_mode='int4_ours_asym_alloc' requires a non-empty policy_json")
    if kv_mode == "kivi_style":
        quant_bits = 8 if quant_bits is None else int(quant_bits)
        if quant_bits not in (4, 8):
            raise ValueError(f"kv_mode='kivi_style' requires quant_bits in {{4, 8}}, got {quant_bits}")
        ignored = [name for name, on in (
            ("calib_file", calib_file is not None), ("use_attn_temperature", use_attn_temperature),
            ("use_static_scales", use_static_scales), ("adaptive_static_scales", adaptive_static_scales),
            ("adaptive_static_margin", adaptive_static_margin != 1.0),
            ("adaptive_static_k", not adaptive_static_k), ("adaptive_static_v", not adaptive_static_v),
            ("allow_missing_calib", allow_missing_calib)) if on]
        if ignored:
            warnings.warn("kv_mode='kivi_style' ignores calibration/static-scale parameters: "
                          + ", ".join(sorted(ignored)), UserWarning)
        calib_file, use_attn_temperature = None, False
    torch.manual_seed(seed)
    # kivi_style: the reference always dequantizes before attention (its torch_ref); here
    # decode_attn_impl="torch_ref" keeps that, the kernel names run the INT4_KIVI HIP kernel
    fused = kv_mode in _FUSED_KV_MODES or (kv_mode in _KERNEL_FUSABLE and decode_attn_impl != "torch_ref")
    num_layers = int(getattr(model.config, "num_hidden_layers", 28))
    max_len = getattr(model.config, "max_position_embeddings", None)
    if max_len is not None and S + max_new_tokens > int(max_len):
        raise ValueError(f"prompt_len + max_new_tokens = {S + max_new_tokens} exceeds the model's "
                         f"max_position_embeddings={max_len}")
    cal = load_calibration(kv_mode, calib_file, group_size, clip_percentile, use_static_scales,
                           use_attn_temperature, allow_missing_calib, device=dev)
    role = load_role_calibration(kv_mode, calib_file, project_root, device=dev)
    kv_cache = create_kv_cache(kv_mode, num_layers, device=dev, max_seq_len=S + max_new_tokens, calib=cal,
                               group_size=group_size, clip_percentile=clip_percentile,
                               decode_attn_impl=decode_attn_impl, use_attn_temperature=use_attn_temperature,
                               adaptive_static_scales=adaptive_static_scales,
                               adaptive_static_margin=adaptive_static_margin,
                               adaptive_static_k=adaptive_static_k, adaptive_static_v=adaptive_static_v,
                               quant_bits=quant_bits, residual_length=residual_length,
                               check_numerics=check_numerics, role=role, k_bits=k_bits, v_bits=v_bits,
                               per_layer_bits=per_layer_bits)
    patched = False
    hooks = []
    try:
        if fused:
            apply_int8_fused_patch(model)
            patched = True
            if use_attn_temperature and cal.inv_tau is not None and kv_mode in _FUSED_KV_MODES:
                hooks = _temperature_hooks(model, cal.inv_tau)
            elif use_attn_temperature and role.inv_tau is not None and \
                    kv_mode in ("int4_kivi_aligned", "int4_ours_asym_ba"):
                # prefill only; decode steps apply the engine's inv_tau.  (The reference
                # registers none for a fused int4_ours_asym_ba decode, so its prefill runs
                # unscaled there while its torch_ref path scales it: here both scale it.)
                hooks = _temperature_hooks(model, role.inv_tau)
        elif use_attn_temperature and role.inv_tau is not None and \
                kv_mode in ("int4_kivi_aligned", "int4_ours_asym_ba"):
            # dequantized decode through the model's attention: every step's queries
            hooks = _temperature_hooks(model, role.inv_tau, all_steps=True)
        # ---- prefill (the model's own attention; q_len > 1 never takes the fused path)
        _sync()
        t0 = time.perf_counter()
        with torch.no_grad():
            out = model(input_ids=input_ids, attention_mask=attention_mask, use_cache=True)
            layers = _past_layers(out.past_key_values)
            if len(layers) != num_layers:
                warnings.warn(f"ENG-065: Prefill returned {len(layers)} layers but kv_cache expects "
                              f"{num_layers}.", RuntimeWarning)
            model_cache = None
            if kv_mode == "fp16":
                model_cache = out.past_key_values
            else:
                for i, (k, v) in enumerate(layers):
                    kv_cache.append(i, k, v)
            nxt = torch.argmax(out.logits[:, -1, :], dim=-1)
        _sync()
        ttft_ms = (time.perf_counter() - t0) * 1e3
        if fused:  # prefill-only hooks; the all-step ones stay for the decode
            for h in hooks:
                h.remove()
            hooks = []
        steps = [nxt]
        times: List[float] = []
        eos = getattr(tokenizer, "eos_token_id", None) if tokenizer is not None else None
        if isinstance(eos, (list, tuple)):
            eos = eos[0] if eos else None
        done = (nxt == eos) if (stop_on_eos and eos is not None) else torch.zeros_like(nxt, dtype=torch.bool)
        cur = nxt.view(B, 1)
        for _ in range(max(max_new_tokens - 1, 0)):
            if stop_on_eos and eos is not None and bool(torch.all(done).item()):
                break
            attention_mask = torch.cat([attention_mask, torch.ones((B, 1), device=dev,
                                                                   dtype=attention_mask.dtype)], dim=1)
            _sync()
            t0 = time.perf_counter()
            with torch.no_grad():
                if kv_mode == "fp16":
                    pkv = model_cache
                elif fused:
                    pkv = INT8CacheWrapperContainer(kv_cache, num_layers)
                else:
                    prev = list(kv_cache._layer_seq_lens)
                    pkv = _to_model_cache(kv_cache.get_kv(i) for i in range(num_layers))
                out = model(input_ids=cur, attention_mask=None if fused else attention_mask,
                            past_key_values=pkv, use_cache=True)
                if kv_mode == "fp16":
                    model_cache = out.past_key_values
                elif not fused:
                    _append_delta(kv_cache, _past_layers(out.past_key_values), prev, 1)
                nxt = torch.argmax(out.logits[:, -1, :], dim=-1)
                if stop_on_eos and eos is not None:
                    nxt = torch.where(done, torch.full_like(nxt, eos), nxt)
                    done = done | (nxt == eos)
            _sync()
            times.append((time.perf_counter() - t0) * 1e3)
            steps.append(nxt)
            cur = nxt.view(B, 1)
        gen = torch.stack(steps, dim=1) if steps else torch.empty(B, 0, dtype=torch.long, device=dev)
        mem = kv_cache.get_memory_mb() if kv_mode != "fp16" else 0.0
        stats = kv_cache.get_decode_stats() if hasattr(kv_cache, "get_decode_stats") else None
        return GenerationBatchOutput(
            generated_ids=gen, ttft_ms=ttft_ms, tpot_ms=(sum(times) / len(times)) if times else 0.0,
            decode_times_ms=times, kv_mode=kv_mode, decode_attn_impl=decode_attn_impl,
            kv_cache_mem_mb=mem, decode_stats=stats)
    finally:
        for h in hooks:
            h.remove()
        if patched:
            remove_int8_fused_patch(model)
        kv_cache.clear()
