"""The HF attention hook of the decode step (src/engine/patch_model.py).

``apply_int8_fused_patch(model)`` replaces the forward of the model's attention class by a
proxy.  For a one-token step whose ``past_key_values`` is an
:class:`INT8CacheWrapperContainer` (or one of its per-layer :class:`INT8CacheWrapper`), the
proxy runs :func:`_fused_forward_impl`:

1. q / k / v projections (and q_norm / k_norm where the model has them), RoPE;
2. the per-head ``inv_tau`` of the cache engine (validated as the reference does);
3. quantize-on-append of the new K / V row and split-K decode attention over the cache,
   through the engine's ``append_decode_attn`` (one HIP launch for the static group-32
   formats, append then attention otherwise);
4. ``o_proj``.

Every other call (prefill, no quantized cache) goes to the original forward.  The decode
implementation is the engine's ``decode_attn_impl``: ``"hip_fused"`` and the reference's
``"triton_fused"`` run the HIP kernels; ``"torch_ref"`` is the reference's own torch
decode path (:func:`_decode_attn_int8_torch_ref`), a mode the caller selects explicitly for
comparisons, never a fallback.  Unknown names raise ``ValueError``.

Differences from the reference, for transformers 5.x (the reference was written against
4.57): the container answers ``get_query_offset`` and ``get_mask_sizes(query_length,
layer_idx)`` (an int query length; a ``cache_position`` tensor is still accepted) and has
``is_sliding``; the proxy takes ``past_key_values`` by keyword as 5.x passes it.
"""
from __future__ import annotations

import inspect
import logging
import math
import os
import warnings
from typing import Optional, Tuple

import torch

logger = logging.getLogger(__name__)

# every attention class this module has patched (remove_int8_fused_patch() restores them)
_patched_classes: set = set()

# decode_attn_impl names that run the HIP kernels
_HIP_IMPLS = ("hip_fused", "triton_fused")


def _reset_fused_state() -> None:
    """Forget every patched class (test isolation; src/engine/patch_model.py:31-51)."""
    global _patched_classes
    _patched_classes = set()


# ---------------------------------------------------------------- HF cache duck types


class INT8CacheWrapper:
    """One layer's view of a quantized cache engine, in the shape HF attention expects
    (src/engine/patch_model.py:95-131).  The fused path reads ``engine`` and
    ``layer_idx``; ``update`` is the fallback the original forward calls."""

    def __init__(self, cache_engine, layer_idx: int):
        self.engine = cache_engine
        self.layer_idx = layer_idx

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        self.engine.append(layer_idx, key_states, value_states)
        return self.engine.get_kv(layer_idx)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.engine.get_seq_len()

    def __getitem__(self, idx):
        return self.engine.get_kv(idx)

    def __iter__(self):
        for i in range(self.engine.num_layers):
            yield self.engine.get_kv(i)

    def __len__(self) -> int:
        return self.engine.num_layers


def _is_quantized_engine(engine) -> bool:
    return any(hasattr(engine, n) for n in (
        "get_int8_tensors", "get_int4_tensors", "get_int4_asym_tensors", "get_int4_g32_tensors",
        "get_k8v4_tensors", "get_kivi_tensors", "get_mixed_tensors"))


class INT8CacheWrapperContainer:
    """The model-level HF cache stand-in (src/engine/patch_model.py:134-214): the model
    asks it for the sequence length and the mask sizes, and passes ``self[layer_idx]``
    to each attention layer."""

    def __init__(self, cache_engine, num_layers: int):
        if not _is_quantized_engine(cache_engine):
            raise TypeError(
                "INT8CacheWrapperContainer requires an INT8/INT4 fused cache engine. "
                f"Got {type(cache_engine).__name__}. "
                "If you are using kivi_style or fp16, route through the non-fused decode path.")
        self.engine = cache_engine
        self.num_layers = num_layers
        self._layer_wrappers = [INT8CacheWrapper(cache_engine, i) for i in range(num_layers)]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.engine.get_seq_len()

    def get_query_offset(self, layer_idx: int = 0) -> int:
        """Position of the step's first query token: the cached length (transformers 5.x)."""
        return int(self.engine.get_seq_len())

    @property
    def is_sliding(self):
        return [False] * self.num_layers

    def get_max_cache_shape(self):
        return None

    def __getitem__(self, layer_idx: int) -> INT8CacheWrapper:
        return self._layer_wrappers[layer_idx]

    def __iter__(self):
        return iter(self._layer_wrappers)

    def __len__(self) -> int:
        return self.num_layers

    def to_legacy_cache(self):
        """Dequantized (k, v) per layer (the reference's HF interop; full precision)."""
        return tuple(self.engine.get_kv(i) for i in range(self.num_layers))

    def get_mask_sizes(self, cache_position, layer_idx: int = 0):
        """(kv_length, kv_offset) of the attention of the current step: the cached tokens
        plus the step's query tokens; ``cache_position`` is the step's query length (an
        int, transformers 5.x) or its position tensor (4.x)."""
        cached = int(self.engine.get_seq_len())
        if cache_position is None:
            current = 0
        elif isinstance(cache_position, int):
            current = cache_position
        elif isinstance(cache_position, torch.Tensor):
            current = int(cache_position.shape[0]) if cache_position.ndim else int(cache_position.item())
        else:
            current = int(cache_position)
        return cached + current, 0

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        self.engine.append(layer_idx, key_states, value_states)
        return self.engine.get_kv(layer_idx)


# ---------------------------------------------------------------- RoPE and head metadata


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def _apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """RoPE of q / k [B, H, S, D] with cos / sin [S, R], [B, S, R] or [B, 1|H, S, R]
    (R <= D rotary channels; the rest pass through), in q's dtype
    (src/engine/patch_model.py:223-278)."""
    bsz, _, _, head_dim = q.shape
    cos = cos.to(device=q.device, dtype=q.dtype)
    sin = sin.to(device=q.device, dtype=q.dtype)
    if cos.ndim == 2:
        cos, sin = cos[None], sin[None]
    if cos.ndim == 3:
        cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    elif cos.ndim == 4:
        cos, sin = cos[:, :1], sin[:, :1]
    else:
        raise ValueError(f"Unexpected cos/sin rank {cos.ndim} in _apply_rope; expected 2-4.")
    if cos.shape[0] == 1 and bsz > 1:
        cos = cos.expand(bsz, -1, -1, -1)
        sin = sin.expand(bsz, -1, -1, -1)
    rd = cos.shape[-1]
    if rd > head_dim:
        raise ValueError(f"RoPE dim {rd} > head_dim {head_dim}")

    def rot(x):
        xr = x[..., :rd]
        out = xr * cos + _rotate_half(xr) * sin
        return out if rd == head_dim else torch.cat([out, x[..., rd:]], dim=-1)

    return rot(q), rot(k)


def _get_rope_cos_sin(attn_module, value_states, position_ids, position_embeddings):
    """(cos, sin) from the layer's position_embeddings, else from its rotary_emb
    (src/engine/patch_model.py:499-604); (None, None) when neither is available."""
    if position_embeddings is not None:
        try:
            cos, sin = position_embeddings
            return cos, sin
        except (TypeError, ValueError) as exc:
            warnings.warn(f"_get_rope_cos_sin: position_embeddings unpack failed "
                          f"({type(exc).__name__}: {exc}); falling back to rotary_emb.",
                          RuntimeWarning)
    rotary = getattr(attn_module, "rotary_emb", None)
    if rotary is None or position_ids is None:
        return None, None
    for call in (lambda: rotary(value_states, position_ids),
                 lambda: rotary(value_states, position_ids=position_ids)):
        try:
            out = call()
        except (AttributeError, KeyError, TypeError):
            continue
        if isinstance(out, (tuple, list)) and len(out) == 2:
            return out[0], out[1]
    return None, None


def _infer_heads_from_proj(attn_module, proj_name: str, head_dim: int) -> Optional[int]:
    proj = getattr(attn_module, proj_name, None)
    if proj is None:
        return None
    out = getattr(proj, "out_features", None)
    if out is None and hasattr(proj, "weight"):
        out = int(proj.weight.shape[0])
    if out is None:
        return None
    if int(out) % int(head_dim):
        raise ValueError(f"{proj_name}.out_features={out} is not divisible by head_dim={head_dim}")
    return int(out) // int(head_dim)


def _resolve_attn_shape_meta(attn_module) -> Tuple[int, int, int]:
    """(q_heads, kv_heads, head_dim) of an attention module (src/engine/patch_model.py:607-642)."""
    head_dim = getattr(attn_module, "head_dim", None)
    if head_dim is None:
        raise ValueError("Attention module is missing head_dim.")
    head_dim = int(head_dim)
    q_heads = getattr(attn_module, "_kv_num_attention_heads", None)
    kv_heads = getattr(attn_module, "_kv_num_key_value_heads", None)
    if q_heads is None:
        q_heads = getattr(attn_module, "num_heads", None)
    if kv_heads is None:
        kv_heads = getattr(attn_module, "num_key_value_heads", None)
    if q_heads is None:
        q_heads = _infer_heads_from_proj(attn_module, "q_proj", head_dim)
    if kv_heads is None:
        kv_heads = _infer_heads_from_proj(attn_module, "k_proj", head_dim)
    if q_heads is None or kv_heads is None:
        raise ValueError(
            "Unable to resolve attention head metadata for fused decode. "
            "Expected explicit num_heads/num_key_value_heads or inferable q_proj/k_proj dimensions.")
    q_heads, kv_heads = int(q_heads), int(kv_heads)
    if q_heads <= 0 or kv_heads <= 0:
        raise ValueError(f"Invalid heads: q_heads={q_heads}, kv_heads={kv_heads}")
    if q_heads % kv_heads:
        raise ValueError(f"Invalid GQA mapping for fused decode: q_heads={q_heads}, kv_heads={kv_heads}")
    return q_heads, kv_heads, head_dim


# ---------------------------------------------------------------- the torch decode path


def _materialize_int4_cache_as_int8(k_int4, v_int4, *, head_dim: int, bit_packed: bool):
    """Packed INT4 codes [.., D/2] -> int8 codes in [-8, 7] [.., D]; unpacked caches pass
    through (src/engine/patch_model.py:71-92)."""
    if not bit_packed:
        if k_int4.shape[-1] != head_dim or v_int4.shape[-1] != head_dim:
            raise ValueError(f"Unpacked INT4 cache shape mismatch: k={tuple(k_int4.shape)} "
                             f"v={tuple(v_int4.shape)} head_dim={head_dim}")
        return k_int4, v_int4
    if k_int4.shape[-1] * 2 != head_dim or v_int4.shape[-1] * 2 != head_dim:
        raise ValueError(f"Packed INT4 cache shape mismatch: k={tuple(k_int4.shape)} "
                         f"v={tuple(v_int4.shape)} expected_last_dim={head_dim // 2}")

    def unpack(p):
        u = p.view(torch.uint8).to(torch.int16)
        return (torch.stack(((u >> 4) & 15, u & 15), dim=-1).flatten(-2) - 8).to(torch.int8)

    return unpack(k_int4), unpack(v_int4)


def _attention_fp32(q, k, v, sm_scale):
    """q [B, Hq, D] over dequantized k / v [B, Hkv, S, D] (every row S tokens): GQA heads
    expanded, scores / softmax / weighted sum in fp32, output in q's dtype."""
    rep = q.shape[1] // k.shape[1]
    kf = k.float().repeat_interleave(rep, dim=1)
    vf = v.float().repeat_interleave(rep, dim=1)
    scores = torch.einsum("bhd,bhsd->bhs", q.float(), kf) * sm_scale
    return torch.einsum("bhs,bhsd->bhd", torch.softmax(scores, dim=-1), vf).to(q.dtype)


def _decode_attn_int8_torch_ref(q, k_int8, v_int8, k_scale, v_scale, context_lens, sm_scale):
    """The reference's torch decode attention over INT8 codes with per-(token, group)
    fp16 scales (src/engine/patch_model.py:281-377): codes dequantised as fp16 products,
    GQA heads expanded, scores / softmax / weighted sum in fp32, output in q's dtype, rows
    with an empty context zero.  q [B, Hq, D]; k/v [B, Hkv, S, D]; scales [B, Hkv, S, G]."""
    if q.ndim != 3:
        raise ValueError(f"Expected q [B, H, D], got {q.shape}")
    if k_int8.ndim != 4 or v_int8.ndim != 4:
        raise ValueError(f"Expected k/v [B, H, S, D], got {k_int8.shape} / {v_int8.shape}")
    if k_scale.ndim != 4 or v_scale.ndim != 4:
        raise ValueError(f"Expected k/v scale [B, H, S, G], got {k_scale.shape} / {v_scale.shape}")
    B, Hq, D = q.shape
    _, Hkv, _, Dk = k_int8.shape
    if Dk != D:
        raise ValueError(f"Head dim mismatch: q D={D}, kv D={Dk}")
    if Hq % Hkv:
        raise ValueError(f"GQA unsupported: q_heads={Hq} not divisible by kv_heads={Hkv}")
    G = int(k_scale.shape[-1])
    if G <= 0 or D % G:
        raise ValueError(f"Invalid scale groups: D={D} groups={G}")
    rep = Hq // Hkv
    out = torch.zeros(B, Hq, D, device=q.device, dtype=q.dtype)
    for b in range(B):
        n = int(context_lens[b].item())
        if n <= 0:
            continue

        def deq(codes, scale):
            x = codes[b, :, :n].reshape(Hkv, n, G, D // G).to(torch.float16)
            return (x * scale[b, :, :n].unsqueeze(-1)).reshape(Hkv, n, D).float()

        k = deq(k_int8, k_scale).repeat_interleave(rep, dim=0)
        v = deq(v_int8, v_scale).repeat_interleave(rep, dim=0)
        scores = torch.bmm(k, q[b].float().unsqueeze(-1)).squeeze(-1) * sm_scale  # [Hq, n]
        probs = torch.softmax(scores, dim=-1)
        out[b] = torch.bmm(probs.unsqueeze(1), v).squeeze(1).to(q.dtype)
    return out


# ---------------------------------------------------------------- the fused decode forward


def _layer_inv_tau(engine, layer_idx: int, q_heads: int, device, dtype) -> Optional[torch.Tensor]:
    """The engine's inv_tau[layer] in q's dtype, validated as the reference does
    (src/engine/patch_model.py:711-746); None when temperature is off or absent."""
    inv_tau = getattr(engine, "inv_tau", None)
    if inv_tau is None or not getattr(engine, "use_attn_temperature", True):
        return None
    if layer_idx >= inv_tau.shape[0]:
        raise ValueError(f"inv_tau has {inv_tau.shape[0]} layers but fused decode got layer_idx={layer_idx}.")
    cache = engine.__dict__.setdefault("_hook_tau", {})
    key = (layer_idx, str(device), dtype)
    t = cache.get(key)
    if t is None:
        t = inv_tau[layer_idx].to(device=device, dtype=dtype)
        if t.ndim != 1:
            raise ValueError(f"inv_tau[{layer_idx}] must be a 1D tensor [num_heads], got shape "
                             f"{tuple(t.shape)}. Check calibration file format.")
        if t.shape[0] != q_heads:
            raise ValueError(
                f"inv_tau[{layer_idx}] has {t.shape[0]} elements but q_heads={q_heads}. inv_tau must "
                "be calibrated per query head. If your calibration file uses kv_heads, re-generate "
                "it with per-query-head granularity.")
        t = t.contiguous()
        cache[key] = t
    return t


def _fused_forward_impl(self, hidden_states, cache_wrapper, attention_mask=None, position_ids=None,
                        position_embeddings=None, cache_position=None, return_cache=False, **kwargs):
    """Decode-only attention forward (q_len == 1) over a quantized cache engine
    (src/engine/patch_model.py:645-1008)."""
    if attention_mask is not None:
        warnings.warn(
            "Fused INT8/INT4 decode path received a non-None attention_mask, which will be "
            "silently ignored. The fused kernel handles causality via context lengths and does "
            "not support external masks. If you need padding support, use kv_mode='fp16' or "
            "ensure attention_mask is None for fused decode.", UserWarning, stacklevel=3)
    layer_idx = getattr(cache_wrapper, "layer_idx", getattr(self, "layer_idx", 0))
    bsz, q_len, _ = hidden_states.shape
    if q_len != 1:
        raise ValueError(f"Fused decode expects q_len==1, got {q_len}")
    q_heads, kv_heads, head_dim = _resolve_attn_shape_meta(self)
    engine = cache_wrapper.engine

    q = self.q_proj(hidden_states).view(bsz, 1, q_heads, head_dim).transpose(1, 2)
    k = self.k_proj(hidden_states).view(bsz, 1, kv_heads, head_dim).transpose(1, 2)
    v = self.v_proj(hidden_states).view(bsz, 1, kv_heads, head_dim).transpose(1, 2)
    if getattr(self, "q_norm", None) is not None:
        q = self.q_norm(q)
    if getattr(self, "k_norm", None) is not None:
        k = self.k_norm(k)
    cos, sin = _get_rope_cos_sin(self, v, position_ids, position_embeddings)
    if cos is None or sin is None:
        raise RuntimeError("Failed to obtain RoPE cos/sin for fused decode. "
                           "Check transformers version/model API (position_ids/position_embeddings).")
    q, k = _apply_rope(q, k, cos, sin)
    tau = _layer_inv_tau(engine, layer_idx, q_heads, q.device, q.dtype)

    sm_scale = float(getattr(self, "scaling", 1.0 / math.sqrt(head_dim)))
    decode_impl = getattr(engine, "decode_attn_impl", "triton_fused")
    if hasattr(engine, "record_fused_decode"):
        engine.record_fused_decode(layer_idx, decode_impl)
    q_kernel = q.squeeze(2)  # [B, Hq, D]
    try:
        if decode_impl in _HIP_IMPLS:
            if q_kernel.dtype == torch.float16:
                out = engine.append_decode_attn(layer_idx, q_kernel, k, v, sm_scale=sm_scale, inv_tau=tau)
            else:
                # the reference scales q in its own dtype, then the kernel casts it to fp16
                qs = q_kernel * tau.view(1, -1, 1) if tau is not None else q_kernel
                out = engine.append_decode_attn(layer_idx, qs.to(torch.float16), k, v,
                                                sm_scale=sm_scale).to(q_kernel.dtype)
            if hasattr(engine, "record_triton_kernel_call"):
                engine.record_triton_kernel_call(layer_idx)
        elif decode_impl == "torch_ref" and not (hasattr(engine, "get_int8_tensors") or
                                                 hasattr(engine, "get_int4_tensors")):
            # the KIVI family and the mixed cache: the reference decodes them by handing the
            # dequantized cache to the model's attention (src/engine/generate_loop.py:1357-
            # 1364); here get_kv's fp16 K / V with the same fp32 attention as the INT8 path
            if not hasattr(engine, "get_kv"):
                raise RuntimeError(f"decode_attn_impl='torch_ref' needs a cache with get_kv, got "
                                   f"{type(engine).__name__}")
            qs = q_kernel * tau.view(1, -1, 1) if tau is not None else q_kernel
            engine.append(layer_idx, k, v)
            kd, vd = engine.get_kv(layer_idx)
            out = _attention_fp32(qs, kd, vd, sm_scale)
        elif decode_impl == "torch_ref":
            qs = q_kernel * tau.view(1, -1, 1) if tau is not None else q_kernel
            engine.append(layer_idx, k, v)
            if hasattr(engine, "get_int8_tensors"):
                kq, vq, ks, vs = engine.get_int8_tensors(layer_idx)
            else:
                kq, vq, ks, vs = engine.get_int4_tensors(layer_idx)
                kq, vq = _materialize_int4_cache_as_int8(
                    kq, vq, head_dim=head_dim, bit_packed=bool(getattr(engine, "bit_packed", True)))
            n = int(kq.shape[2])
            ctx = torch.full((bsz,), n, dtype=torch.int32, device=q.device)
            out = _decode_attn_int8_torch_ref(qs, kq, vq, ks.to(torch.float16), vs.to(torch.float16),
                                              ctx, sm_scale)
        else:
            raise ValueError(f"Unknown decode_attn_impl={decode_impl!r}. Use 'triton_fused' (or "
                             "'hip_fused') or 'torch_ref'.")
    except Exception:
        warnings.warn(
            f"ENG-042: Kernel call failed at layer_idx={layer_idx} after cache.append() may have "
            "committed. The cache seq_len may have been incremented without an attention output; "
            "cache state is potentially inconsistent.", RuntimeWarning, stacklevel=3)
        raise

    attn = out.reshape(bsz, 1, q_heads * head_dim).to(hidden_states.dtype)
    attn_output = self.o_proj(attn)
    if os.environ.get("KV_FUSED_DEBUG", "") not in ("", "0") and layer_idx == 0:
        calls = getattr(engine, "_fused_decode_calls", 0) + 1
        engine._fused_decode_calls = calls
        if calls == 1:
            logger.info("Quantized fused decode active (layer=%s q_heads=%s kv_heads=%s seq_len=%s).",
                        layer_idx, q_heads, kv_heads, engine.get_seq_len())
    if return_cache:
        return attn_output, None, cache_wrapper
    return attn_output, None


def apply_int8_fused_patch(model) -> None:
    """Patch the model's attention class for fused quantized decode
    (src/engine/patch_model.py:1011-1226)."""
    try:
        layers = model.model.layers
    except Exception:
        layers = None
    if layers is None:
        raise ValueError("Cannot detect model layers (model.model.layers). "
                         "apply_int8_fused_patch requires a standard HF decoder model.")
    cfg = getattr(model, "config", None)
    cfg_q = getattr(cfg, "num_attention_heads", None)
    cfg_kv = getattr(cfg, "num_key_value_heads", cfg_q)
    for idx, layer in enumerate(layers):
        attn = getattr(layer, "self_attn", None)
        if attn is None:
            continue
        if not hasattr(attn, "layer_idx"):
            attn.layer_idx = idx
        head_dim = getattr(attn, "head_dim", None)
        if head_dim is None:
            continue
        q_heads = cfg_q if cfg_q is not None else _infer_heads_from_proj(attn, "q_proj", int(head_dim))
        kv_heads = cfg_kv if cfg_kv is not None else _infer_heads_from_proj(attn, "k_proj", int(head_dim))
        if kv_heads is None:
            logger.warning("Could not infer kv_heads for layer %d; falling back to q_heads=%s.", idx, q_heads)
            kv_heads = q_heads
        if q_heads is not None:
            attn._kv_num_attention_heads = int(q_heads)
        if kv_heads is not None:
            attn._kv_num_key_value_heads = int(kv_heads)

    AttnClass = layers[0].self_attn.__class__
    if hasattr(AttnClass, "_original_forward"):
        # already patched: never re-save the proxy as the original
        apply_int8_fused_patch._patched_class = AttnClass
        _patched_classes.add(AttnClass)
        logger.info("Skipping re-patch: %s._original_forward already set.", AttnClass.__name__)
        return
    AttnClass._original_forward = AttnClass.forward
    original_sig = inspect.signature(AttnClass._original_forward)
    params = original_sig.parameters
    accepts_var_kw = any(p.kind == inspect.Parameter.VAR_KEYWORD for p in params.values())
    has_past_key_value = "past_key_value" in params
    has_past_key_values = "past_key_values" in params
    has_use_cache = "use_cache" in params

    def _filter_kwargs(kw: dict) -> dict:
        return kw if accepts_var_kw else {k: v for k, v in kw.items() if k in params}

    def forward_proxy(self, hidden_states, attention_mask=None, position_ids=None,
                      past_key_value=None, past_key_values=None, output_attentions=False,
                      use_cache=False, **kwargs):
        if past_key_value is None:
            past_key_value = past_key_values
        cache_wrapper = None
        if isinstance(past_key_value, INT8CacheWrapper):
            cache_wrapper = past_key_value
        elif isinstance(past_key_value, INT8CacheWrapperContainer):
            cache_wrapper = past_key_value[getattr(self, "layer_idx", 0)]
        elif hasattr(past_key_value, "__getitem__") and hasattr(past_key_value, "engine"):
            try:
                cand = past_key_value[getattr(self, "layer_idx", 0)]
                if isinstance(cand, INT8CacheWrapper):
                    cache_wrapper = cand
            except Exception:
                cache_wrapper = None
        if hidden_states is not None and hidden_states.shape[1] == 1 and cache_wrapper is not None:
            if output_attentions:
                warnings.warn(
                    "output_attentions=True was requested but the fused INT8/INT4 decode path does "
                    "not compute attention weights. Attention weights will be None. Use "
                    "decode_attn_impl='torch_ref' or kv_mode='fp16' if you need attention outputs.",
                    UserWarning, stacklevel=2)
            pos_emb = kwargs.pop("position_embeddings", None)
            cache_pos = kwargs.pop("cache_position", None)
            return _fused_forward_impl(self, hidden_states, cache_wrapper, attention_mask=attention_mask,
                                       position_ids=position_ids, position_embeddings=pos_emb,
                                       cache_position=cache_pos,
                                       return_cache=use_cache if has_use_cache else False)
        kw = dict(attention_mask=attention_mask, position_ids=position_ids,
                  output_attentions=output_attentions, use_cache=use_cache, **kwargs)
        kw = _filter_kwargs(kw)
        if past_key_value is not None:
            if has_past_key_value:
                kw["past_key_value"] = past_key_value
            elif has_past_key_values:
                kw["past_key_values"] = past_key_value
        return AttnClass._original_forward(self, hidden_states, **kw)

    AttnClass.forward = forward_proxy
    apply_int8_fused_patch._patched_class = AttnClass
    _patched_classes.add(AttnClass)
    logger.info("Patched %s.forward for fused quantized decode.", AttnClass.__name__)


def _remove_patch_from_class(AttnClass) -> bool:
    if AttnClass is None:
        return False
    original = getattr(AttnClass, "_original_forward", None)
    if original is None:
        logger.warning("remove_int8_fused_patch: %s has no _original_forward; patch may not have "
                       "been applied.", AttnClass.__name__)
        return False
    AttnClass.forward = original
    del AttnClass._original_forward
    _patched_classes.discard(AttnClass)
    if getattr(apply_int8_fused_patch, "_patched_class", None) is AttnClass:
        apply_int8_fused_patch._patched_class = None
    return True


def remove_int8_fused_patch(model=None) -> bool:
    """Restore the original attention forward (src/engine/patch_model.py:1229-1298): the
    model's class, or every patched class when model is None.  True if a patch was removed."""
    if model is not None:
        try:
            AttnClass = model.model.layers[0].self_attn.__class__
        except Exception:
            AttnClass = getattr(apply_int8_fused_patch, "_patched_class", None)
        return _remove_patch_from_class(AttnClass)
    removed = False
    for cls in list(_patched_classes):
        removed |= _remove_patch_from_class(cls)
    legacy = getattr(apply_int8_fused_patch, "_patched_class", None)
    if legacy is not None and legacy not in _patched_classes:
        removed |= _remove_patch_from_class(legacy)
    if not removed:
        logger.warning("remove_int8_fused_patch: no patched class found.")
    return removed
