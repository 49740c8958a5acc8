"""Quantized KV-cache engines whose append runs the HIP quantize-on-append kernel.

:class:`INT8KVCache` and :class:`INT4KVCache` keep the constructor arguments,
methods, attributes, exceptions and warnings of the reference engines:

* ``src/cache/int8_cache.py:29-682``
* ``src/cache/int4_cache.py:32-760``

``append`` quantises on the GPU in one launch for K and V, and the kernel writes
straight into the preallocated buffers.  The codes are bit-exact with the
reference torch quantizers.

Where the layout differs from the reference:

* With a static scale and no adaptive/rescue policy, every token gets the same
  scale.  The engines then keep the effective per-(head, group) scale once.
  ``get_int8_tensors`` / ``get_int4_tensors`` return it as a stride-0 expanded
  view [B, H, S, G] with the values the reference stores per token.
* INT8 scales are kept in fp16.  The INT8 quantizer returns its scale in fp16, so
  the reference's fp32 copy carries the same values.  The kernel boundary's
  ``.to(torch.float16)`` is therefore free.
* Host synchronisation is optional.  With ``check_numerics=True`` (the default)
  ``append`` reads a device status word back, like the reference's
  NaN/Inf/clip checks, and raises/warns the same way.  The decode step
  (``append_decode_attn``) reads the status words of all layers once per step,
  after the step's last layer, instead of once per layer: a NaN / Inf then raises
  ValueError there and every layer of the step goes back to its length before the
  step, so the cache does not advance (``flush_status`` reads them earlier).  With
  ``check_numerics=False`` nothing synchronises.  :class:`KIVIStyleKVCache` reads it
  at prefill only, and on the decode steps its frozen-K range check selects
  (``KV_OOR_CHECK_INTERVAL``, off by default as in the reference).

:class:`FP16KVCache` is the reference's unquantized engine (src/cache/fp16_cache.py).

:class:`INT4AsymKVCache` (asymmetric INT4, static group-32 parameters, optional fp16
K outlier channels) and :class:`K8V4KVCache` (INT8 K, asymmetric INT4 V) hold the
static-group formats of the benchmark configurations 2-4; the reference has no engine
for them.
"""
from __future__ import annotations

import ctypes
import logging
import math
import os
import warnings
from typing import Dict, List, Optional, Tuple

import torch
from torch import Tensor

from . import _capi as C
from .kernels import TILE_BYTES, TILE_TOKENS

logger = logging.getLogger(__name__)

_CLIP_WARN_THRESHOLD = 0.05


def _new_decode_stats() -> Dict[str, object]:
    return {
        "fused_decode_calls": 0,
        "triton_kernel_calls": 0,
        "triton_decode_calls": 0,
        "torch_ref_calls": 0,
        "layer_hits": {},
        "triton_layer_hits": {},
    }


def _static_2d(scale: Tensor, heads: int, groups: int, name: str) -> Tensor:
    """Accept [H, G] (or [1, H, G] / [H, 1, G] / [H, G, 1]) static scales."""
    s = scale
    if s.ndim == 3:
        if s.shape[0] == 1 and s.shape[1] == heads:
            s = s[0]
        elif s.shape[1] == 1 and s.shape[0] == heads:
            s = s[:, 0]
        elif s.shape[2] == 1 and s.shape[0] == heads:
            s = s[..., 0]
    if s.ndim != 2:
        raise NotImplementedError(
            f"{name}: static scale layout {tuple(scale.shape)} is not supported by the HIP "
            "append; use [H, G]")
    if s.shape[0] != heads:
        raise ValueError(
            "_normalize_static_scale: calibration vs model heads mismatch (fail-fast; wrong "
            f"calibration file was loaded).\n  expected heads: {heads}\n  scale heads: {s.shape[0]}")
    if s.shape[1] != groups:
        raise ValueError(f"{name}: static scale has {s.shape[1]} groups, expected {groups}")
    return s


class _EngineBase:
    """Capacity management, stats and bookkeeping shared by the engines."""

    _min_capacity = 256

    def _init_common(self, num_layers, device, max_seq_len, decode_attn_impl, check_numerics):
        if num_layers <= 0:
            raise ValueError(f"num_layers must be > 0, got {num_layers}")
        self.num_layers = num_layers
        self.device = device
        self._dev_type = torch.device(device).type
        self.max_seq_len = int(max_seq_len) if max_seq_len is not None else None
        if self.max_seq_len is not None and self.max_seq_len <= 0:
            raise ValueError(f"max_seq_len must be > 0, got {self.max_seq_len}")
        self.decode_attn_impl = decode_attn_impl
        self.check_numerics = bool(check_numerics)
        self._layer_seq_lens: List[int] = [0] * num_layers
        self._layer_capacity: List[int] = [0] * num_layers
        self._seq_len = 0
        self.decode_stats: Dict[str, object] = _new_decode_stats()
        self._status: Optional[Tensor] = None
        # the decode step's per-layer status rows and the appends not read yet
        self._step_status: Optional[Tensor] = None
        self._step_pending: List[tuple] = []
        self._step_seq_len0 = 0
        # per layer: the LayerStep over the layer's buffers and the fused append's parameter
        # blocks, rebuilt when the buffers are reallocated
        self._steps: List[Optional[object]] = [None] * num_layers
        self._apps: List[Optional[tuple]] = [None] * num_layers

    # -- decode stats (src/cache/int8_cache.py:255-296)
    def _bump_counter(self, key: str, delta: int = 1) -> None:
        self.decode_stats[key] = int(self.decode_stats.get(key, 0)) + int(delta)

    def record_fused_decode(self, layer_id: int, decode_impl: str) -> None:
        self._bump_counter("fused_decode_calls", 1)
        if decode_impl in ("triton_fused", "hip_fused"):
            self._bump_counter("triton_decode_calls", 1)
        elif decode_impl == "torch_ref":
            self._bump_counter("torch_ref_calls", 1)
        hits = self.decode_stats.setdefault("layer_hits", {})
        hits[str(layer_id)] = int(hits.get(str(layer_id), 0)) + 1

    def record_triton_kernel_call(self, layer_id: Optional[int] = None) -> None:
        self._bump_counter("triton_kernel_calls", 1)
        if layer_id is None:
            return
        hits = self.decode_stats.setdefault("triton_layer_hits", {})
        hits[str(layer_id)] = int(hits.get(str(layer_id), 0)) + 1

    def reset_decode_stats(self) -> None:
        self.decode_stats = _new_decode_stats()

    def get_decode_stats(self) -> Dict[str, object]:
        d = self.decode_stats
        return {
            "fused_decode_calls": int(d.get("fused_decode_calls", 0)),
            "triton_kernel_calls": int(d.get("triton_kernel_calls", 0)),
            "torch_ref_calls": int(d.get("torch_ref_calls", 0)),
            "triton_decode_calls": int(d.get("triton_decode_calls", 0)),
            "layer_hits": dict(d.get("layer_hits", {})),
            "triton_layer_hits": dict(d.get("triton_layer_hits", {})),
        }

    def get_seq_len(self) -> int:
        return self._seq_len

    def _new_capacity(self, layer_id: int, target_len: int, capacity: int) -> int:
        if self.max_seq_len is not None and target_len > self.max_seq_len:
            raise ValueError(
                f"target_len {target_len} exceeds max_seq_len {self.max_seq_len} for layer {layer_id}")
        new_cap = max(target_len, self._min_capacity) if capacity == 0 else max(target_len, capacity * 2)
        if self.max_seq_len is not None:
            new_cap = min(new_cap, self.max_seq_len)
            if new_cap < target_len:
                raise ValueError(
                    f"target_len {target_len} exceeds capped capacity {new_cap} for layer {layer_id}")
        return new_cap

    def _validate_kv(self, layer_id: int, k: Tensor, v: Tensor) -> None:
        if layer_id < 0 or layer_id >= self.num_layers:
            raise ValueError(f"layer_id {layer_id} out of range")
        if k.ndim != 4:
            raise ValueError(f"k must be 4D [B,H,S,D], got ndim={k.ndim}")
        if v.ndim != 4:
            raise ValueError(f"v must be 4D [B,H,S,D], got ndim={v.ndim}")
        if k.shape != v.shape:
            raise ValueError(f"k/v shape mismatch: k={tuple(k.shape)} vs v={tuple(v.shape)}")
        if k.device.type != self._dev_type or v.device.type != self._dev_type:
            raise ValueError(
                f"Device mismatch: cache_device={torch.device(self.device)}, k.device={k.device}, "
                f"v.device={v.device}")
        if not k.is_cuda:
            raise ValueError("the HIP cache engines need GPU (ROCm) tensors")
        if k.dtype != torch.float16 or v.dtype != torch.float16:
            raise NotImplementedError(
                f"the HIP append quantizes fp16 K/V (got {k.dtype}/{v.dtype}); the reference "
                "divides in the input dtype, so other dtypes would not give the same codes")
        if k.shape[-1] != 128:
            raise NotImplementedError(f"head_dim must be 128, got {k.shape[-1]}")

    def _status_buf(self, device) -> Tensor:
        if self._status is None or self._status.device != device:
            self._status = torch.zeros(4, dtype=torch.int32, device=device)
        return self._status

    # -- the decode step's status words, read once per step.  ``append`` checks its input
    # as the reference does, with one host read per call; the decode step
    # (``append_decode_attn``) instead writes each layer's status words to a row of a
    # [num_layers, 4] device buffer and reads the whole buffer once, after the step's last
    # layer (layer num_layers - 1) or before a layer is appended a second time.  A NaN / Inf
    # then raises ValueError and every layer appended since the previous read goes back to
    # its length before the step, so the cache does not advance; clip warnings are issued
    # per layer at the same point.
    def _step_status_ptr(self, layer_id: int, device) -> int:
        """Address of layer layer_id's status row for a decode-step append (the pending
        rows are read first if this layer already has one)."""
        buf = self._step_status
        if buf is None or buf.device != device:
            self._flush_step_status()
            buf = self._step_status = torch.zeros(self.num_layers, 4, dtype=torch.int32,
                                                  device=device)
        elif any(e[0] == layer_id for e in self._step_pending):
            self._flush_step_status()
        if not self._step_pending:  # the first append of a step: its length before the step
            self._step_seq_len0 = self._seq_len
        return buf.data_ptr() + 16 * layer_id

    def _defer_status(self, layer_id: int, n_elem: int, kind: str, qrange: str,
                      clip_warn: bool = True) -> None:
        """Records a decode-step append of layer_id (already advanced) whose status row is
        read later; reads every pending row after the step's last layer."""
        self._step_pending.append((layer_id, n_elem, kind, qrange, clip_warn))
        if layer_id == self.num_layers - 1:
            self._flush_step_status()

    def flush_status(self) -> None:
        """Reads the status rows of the decode-step appends not read yet (one host sync):
        raises ValueError, after undoing those appends, if one of them had NaN / Inf input,
        and issues their clip warnings."""
        self._flush_step_status()

    def _flush_step_status(self) -> None:
        pending = self._step_pending
        if not pending:
            return
        self._step_pending = []
        rows = self._step_status.cpu()
        self._step_status.zero_()
        bad = None
        for layer_id, n_elem, kind, qrange, clip_warn in pending:
            st = rows[layer_id].tolist()
            if bad is None and (st[0] & 1 or st[2] & 1):
                bad = (kind, "K" if st[0] & 1 else "V")
            if clip_warn:
                self._clip_warnings(layer_id, n_elem, qrange, st)
        if bad is not None:
            for layer_id, *_ in pending:
                self._layer_seq_lens[layer_id] -= 1
            self._seq_len = self._step_seq_len0
            raise ValueError(f"{bad[0]} append: {bad[1]} input contains NaN or Inf — refusing "
                             "to quantize corrupt data")

    def _discard_step_status(self) -> None:
        self._step_pending = []
        if self._step_status is not None:
            self._step_status.zero_()

    def _read_status(self) -> List[int]:
        """The append kernel's status words (NaN flags and clip counts of K and V), then
        cleared for the next append."""
        st = self._status.cpu().tolist()
        self._status.zero_()
        return st

    def _check_status(self, layer_id: int, n_elem: int, kind: str, qrange: str) -> None:
        st = self._read_status()
        if st[0] & 1:
            raise ValueError(f"{kind} append: K input contains NaN or Inf — refusing to quantize corrupt data")
        if st[2] & 1:
            raise ValueError(f"{kind} append: V input contains NaN or Inf — refusing to quantize corrupt data")
        self._clip_warnings(layer_id, n_elem, qrange, st)

    def _clip_warnings(self, layer_id: int, n_elem: int, qrange: str, st: List[int]) -> None:
        for side, cnt in (("K", st[1]), ("V", st[3])):
            ratio = cnt / max(n_elem, 1)
            if ratio > _CLIP_WARN_THRESHOLD:
                warnings.warn(
                    f"Static {side} scale overflow at layer {layer_id}: {ratio:.1%} of values "
                    f"clipped to {qrange} (threshold={_CLIP_WARN_THRESHOLD:.0%}). The static scale "
                    "may be too small for this input. Consider re-calibrating or enabling "
                    "adaptive_static_scales.", RuntimeWarning)

    def _launch_append(self, pk: C.AppendParams, pv: C.AppendParams, device) -> None:
        C.check(C.lib().kvq_quant_append(ctypes.byref(pk), ctypes.byref(pv),
                                         ctypes.c_void_p(C.stream_handle(device))))


def _dyn_quantile(percentile: float) -> float:
    """kvq_append_params.dyn_quantile of a dynamic quantizer with this clip percentile:
    0 (absmax) at 100 and above, else the quantile level percentile / 100 the reference
    passes to torch.quantile (src/quant/int8_basic.py:78-83, int4_basic.py:84-90)."""
    p = float(percentile)
    if p >= 100.0:
        return 0.0
    if not p > 0.0:
        raise NotImplementedError(f"clip_percentile must be in (0, 100], got {percentile}")
    return p / 100.0


def _fill_append(p: C.AppendParams, fmt: int, x: Tensor, gs: int, codes: Tensor, write_pos: int,
                 status_ptr: Optional[int]) -> None:
    B, H, S, D = x.shape
    p.format = fmt
    p.x = x.data_ptr()
    p.x_stride_b, p.x_stride_h, p.x_stride_s = x.stride(0), x.stride(1), x.stride(2)
    p.batch, p.heads, p.seq_new, p.head_dim, p.group_size = B, H, S, D, gs
    p.codes = codes.data_ptr()
    p.codes_stride_b, p.codes_stride_h, p.codes_stride_t = codes.stride(0), codes.stride(1), codes.stride(2)
    p.write_pos = write_pos
    p.capacity = codes.shape[2]
    p.status = status_ptr


class _SymCacheBase(_EngineBase):
    """Shared logic of the INT8 / INT4 symmetric engines (reference layout)."""

    _fmt = None
    _qrange = ""
    _kind = ""

    def _init_sym(self, num_layers, device, clip_percentile, group_size, dtype, max_seq_len,
                  decode_attn_impl, static_k_scale, static_v_scale, inv_tau, use_attn_temperature,
                  adaptive_static_scales, adaptive_static_margin, adaptive_static_k,
                  adaptive_static_v, check_numerics):
        self._init_common(num_layers, device, max_seq_len, decode_attn_impl, check_numerics)
        if adaptive_static_margin <= 0:
            raise ValueError(f"adaptive_static_margin must be > 0, got {adaptive_static_margin}")
        self.clip_percentile = clip_percentile
        self.group_size = group_size
        self.dtype = dtype
        self.static_k_scale = static_k_scale
        self.static_v_scale = static_v_scale
        self.inv_tau = inv_tau
        self.use_attn_temperature = use_attn_temperature
        self.adaptive_static_scales = adaptive_static_scales
        self.adaptive_static_margin = adaptive_static_margin
        self.adaptive_static_k = adaptive_static_k
        self.adaptive_static_v = adaptive_static_v
        self._k_cache: List[Optional[Tensor]] = [None] * num_layers
        self._v_cache: List[Optional[Tensor]] = [None] * num_layers
        self._k_scale: List[Optional[Tensor]] = [None] * num_layers
        self._v_scale: List[Optional[Tensor]] = [None] * num_layers
        # per layer: True if scales are stored per token, False if one static table
        self._k_tok: List[bool] = [True] * num_layers
        self._v_tok: List[bool] = [True] * num_layers

    # -- subclass hooks
    def _code_dim(self, D: int) -> int:
        raise NotImplementedError

    def _scale_dtype(self) -> torch.dtype:
        raise NotImplementedError

    def _side_is_token(self, side: str) -> bool:
        raise NotImplementedError

    def _effective_static(self, s: Tensor) -> Tensor:
        raise NotImplementedError

    def _policy(self, p: C.AppendParams, side: str) -> None:
        pass

    def _ensure_capacity(self, layer_id, batch, heads, head_dim, num_groups, target_len):
        bufs = [self._k_cache[layer_id], self._v_cache[layer_id],
                self._k_scale[layer_id], self._v_scale[layer_id]]
        non_none = sum(b is not None for b in bufs)
        if non_none not in (0, 4):
            raise RuntimeError(
                f"Inconsistent buffer state for layer {layer_id}: {non_none}/4 buffers are not None "
                "(expected 0 or 4). This may indicate a partial OOM during a prior allocation. "
                "Call release() and retry.")
        cd = self._code_dim(head_dim)
        if non_none == 4:
            kb = self._k_cache[layer_id]
            if kb.shape[0] != batch or kb.shape[1] != heads or kb.shape[3] != cd or \
                    self._k_scale[layer_id].shape[-1] != num_groups:
                raise ValueError(
                    f"Inconsistent KV shape for layer {layer_id}: existing K={tuple(kb.shape)}, "
                    f"incoming=({batch}, {heads}, *, {cd}) with groups={num_groups}")
        capacity = self._layer_capacity[layer_id]
        if non_none == 4 and target_len <= capacity:
            return
        new_cap = self._new_capacity(layer_id, target_len, capacity if non_none else 0)
        old_len = self._layer_seq_lens[layer_id]
        try:
            nk = torch.empty((batch, heads, new_cap, cd), device=self.device, dtype=torch.int8)
            nv = torch.empty((batch, heads, new_cap, cd), device=self.device, dtype=torch.int8)
            nks = self._alloc_scale("k", layer_id, batch, heads, new_cap, num_groups)
            nvs = self._alloc_scale("v", layer_id, batch, heads, new_cap, num_groups)
        except torch.cuda.OutOfMemoryError:
            if non_none == 0:
                self._k_cache[layer_id] = self._v_cache[layer_id] = None
                self._k_scale[layer_id] = self._v_scale[layer_id] = None
                self._layer_capacity[layer_id] = 0
            raise
        if non_none == 4 and old_len > 0:
            nk[:, :, :old_len] = self._k_cache[layer_id][:, :, :old_len]
            nv[:, :, :old_len] = self._v_cache[layer_id][:, :, :old_len]
            if self._k_tok[layer_id]:
                nks[:, :, :old_len] = self._k_scale[layer_id][:, :, :old_len]
            if self._v_tok[layer_id]:
                nvs[:, :, :old_len] = self._v_scale[layer_id][:, :, :old_len]
        self._k_cache[layer_id], self._v_cache[layer_id] = nk, nv
        self._k_scale[layer_id], self._v_scale[layer_id] = nks, nvs
        self._layer_capacity[layer_id] = new_cap
        self._steps[layer_id] = self._apps[layer_id] = None

    def _alloc_scale(self, side, layer_id, batch, heads, cap, groups):
        tok = self._side_is_token(side)
        (self._k_tok if side == "k" else self._v_tok)[layer_id] = tok
        if tok:
            return torch.empty((batch, heads, cap, groups), device=self.device, dtype=self._scale_dtype())
        static = (self.static_k_scale if side == "k" else self.static_v_scale)[layer_id]
        s = _static_2d(static.to(self.device), heads, groups, f"static_{side}_scale")
        return self._effective_static(s).contiguous()

    def _static_for(self, side: str, layer_id: int, heads: int, groups: int) -> Optional[Tensor]:
        st = self.static_k_scale if side == "k" else self.static_v_scale
        if st is None:
            return None
        if layer_id >= len(st):
            raise IndexError(
                f"layer_id {layer_id} exceeds calibration layers {len(st)} for static_{side}_scale")
        s = _static_2d(st[layer_id].to(self.device), heads, groups, f"static_{side}_scale")
        if s.dtype not in (torch.float16, torch.float32):
            s = s.float()
        return s

    def append(self, layer_id: int, k: Tensor, v: Tensor) -> None:
        """Quantize and append KV tensors to the cache (one HIP launch for K and V)."""
        self._validate_kv(layer_id, k, v)
        B, H, S, D = k.shape
        if D % self.group_size:
            raise ValueError(f"head_dim {D} must be divisible by group_size {self.group_size}")
        G = D // self.group_size
        self._pre_append_checks(layer_id)
        sk = self._static_for("k", layer_id, H, G)
        sv = self._static_for("v", layer_id, H, G)
        old_len = self._layer_seq_lens[layer_id]
        target = old_len + S
        self._ensure_capacity(layer_id, B, H, D, G, target)
        if S == 0:
            return
        status = self._status_buf(k.device) if self.check_numerics else None
        pk, pv = self._append_params(layer_id, k, v, old_len, status, sk, sv)
        self._launch_append(pk, pv, k.device)
        if status is not None:
            self._check_status(layer_id, k.numel(), self._kind, self._qrange)
        self._layer_seq_lens[layer_id] = target
        if layer_id == 0:
            self._seq_len = target

    def _append_params(self, layer_id, k, v, old_len, status, sk, sv):
        """kvq_append_params of K and V written at slot old_len (each keeps the tensors it
        points at alive)."""
        pk, pv = C.AppendParams(), C.AppendParams()
        for side, p, x, codes, scale_buf, st, tok in (
                ("k", pk, k, self._k_cache[layer_id], self._k_scale[layer_id], sk, self._k_tok[layer_id]),
                ("v", pv, v, self._v_cache[layer_id], self._v_scale[layer_id], sv, self._v_tok[layer_id])):
            xs = x if x.stride(-1) == 1 else x.contiguous()
            sptr = None
            if status is not None:
                sptr = status.data_ptr() + (0 if side == "k" else 8)
            _fill_append(p, self._fmt, xs, self.group_size, codes, old_len, sptr)
            if st is not None:
                p.static_scale = st.data_ptr()
                p.static_scale_dtype = C.KVQ_DTYPE_F32 if st.dtype == torch.float32 else C.KVQ_DTYPE_F16
                p.static_stride_h, p.static_stride_g = st.stride()
                self._policy(p, side)
            else:
                p.dyn_quantile = _dyn_quantile(self.clip_percentile)
            if tok:
                p.scale_out = scale_buf.data_ptr()
                p.scale_out_dtype = C.KVQ_DTYPE_F32 if scale_buf.dtype == torch.float32 else C.KVQ_DTYPE_F16
                p.so_stride_b, p.so_stride_h, p.so_stride_t, p.so_stride_g = scale_buf.stride()
            # the group rescue over more than 4096 (row, group) scales selects its
            # threshold in a scratch buffer
            scratch = None
            nbytes = int(C.lib().kvq_append_scratch_bytes(ctypes.byref(p)))
            if nbytes:
                scratch = torch.empty(nbytes, dtype=torch.uint8, device=codes.device)
                p.scratch, p.scratch_bytes = scratch.data_ptr(), nbytes
            # keep the (possibly temporary) tensors alive until the launch returns; _keep_fixed
            # is what a reused block must keep (the table and the rescue scratch)
            p._keep_fixed = (st, scratch)
            p._keep = (xs,) + p._keep_fixed
        return pk, pv

    def _pre_append_checks(self, layer_id: int) -> None:
        pass

    # -- decode step: the append + attention of src/engine/patch_model.py:755-957

    def _fused_step_ok(self, D: int, B: Optional[int] = None, H: Optional[int] = None) -> bool:
        """Whether the tiled kernel appends and attends in one launch for this engine's
        format (B, H: the step's batch and KV heads, where the answer depends on them)."""
        return False

    def _step_for(self, layer_id: int, q_heads: int):
        """The layer's LayerStep (kernels.LayerStep) over its whole buffers."""
        kb = self._k_cache[layer_id]
        st = self._steps[layer_id]
        if st is not None and st.key == (q_heads, kb.data_ptr()):
            return st
        from .kernels import LayerStep, kv_view_tok

        B, H, cap = kb.shape[0], kb.shape[1], kb.shape[2]
        kc, vc, ks, vs = self._raw_views(layer_id, cap)
        st = LayerStep(self._fmt, kv_view_tok(kc, ks), self._fmt, kv_view_tok(vc, vs), B, q_heads, H,
                       self.group_size, kb.device, keepalive=(kc, vc, ks, vs))
        st.key = (q_heads, kb.data_ptr())
        self._steps[layer_id] = st
        return st

    def _fused_apps(self, layer_id: int, k: Tensor, v: Tensor, pos: int, status: Optional[int]):
        """The decode step's kvq_append_params of K and V for one new token (built once per
        layer buffers; per call the rows, the slot and the status words (the device address
        of the layer's status row, or None) change)."""
        B, H, S, D = k.shape
        ent = self._apps[layer_id]
        if ent is None or ent[2] != (B, H):
            G = D // self.group_size
            sk = self._static_for("k", layer_id, H, G)
            sv = self._static_for("v", layer_id, H, G)
            pk, pv = self._append_params(layer_id, k, v, pos, None, sk, sv)
            ent = (pk, pv, (B, H))
            self._apps[layer_id] = ent
        pk, pv = ent[0], ent[1]
        sptr = status
        for p, x, off in ((pk, k, 0), (pv, v, 8)):
            if x.stride(-1) != 1:
                x = x.contiguous()
            p.x = x.data_ptr()
            p.x_stride_b, p.x_stride_h, p.x_stride_s = x.stride()[:3]
            p.write_pos = pos
            p.status = None if sptr is None else sptr + off
            p._keep = (x,) + p._keep_fixed
        return pk, pv

    def append_decode_attn(self, layer_id: int, q: Tensor, k: Tensor, v: Tensor,
                           sm_scale: Optional[float] = None,
                           inv_tau: Optional[Tensor] = None) -> Tensor:
        """Decode step of one layer: append the new token (k, v: fp16 [B, H, 1, D]) and attend
        over the whole cache, the new token included (the append + attention of the
        reference's decode step, src/engine/patch_model.py:755-957).  q: fp16 [B, Hq, D];
        inv_tau: optional fp16 [Hq], applied as fp16(q * inv_tau) in the kernel.  Returns
        fp16 [B, Hq, D].  Both run in one HIP launch (kvq_append_decode_attn) with static
        INT8 scales on both sides, or with the tiled kernel's per-token formats (groups of 16
        or more; not the INT4 group rescue, whose threshold spans every row of the append);
        otherwise ``append`` then the decode kernel.
        Either way codes and output are bit-identical to ``append`` followed by
        :func:`kernels.decode_attn_int8` / ``decode_attn_int4`` over the cache's tensors.
        The kernel parameters are kept per layer between calls (no device tensor is created
        besides the output).  With ``check_numerics``, NaN / Inf in k or v raise ValueError
        and the cache does not advance."""
        self._validate_kv(layer_id, k, v)
        B, H, S, D = k.shape
        if S != 1:
            raise ValueError(f"append_decode_attn appends one token per step, got S={S}")
        if q.ndim != 3 or q.dtype != torch.float16 or q.shape[0] != B or q.shape[1] % H:
            raise ValueError(f"q must be fp16 [B, Hq, D] with Hq a multiple of {H}, got "
                             f"{q.dtype} {tuple(q.shape)}")
        if q.stride(-1) != 1:
            q = q.contiguous()
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        if D % self.group_size:
            raise ValueError(f"head_dim {D} must be divisible by group_size {self.group_size}")
        G = D // self.group_size
        self._pre_append_checks(layer_id)
        old = self._layer_seq_lens[layer_id]
        n = old + 1
        self._ensure_capacity(layer_id, B, H, D, G, n)
        status = self._step_status_ptr(layer_id, k.device) if self.check_numerics else None
        # the append's parameter blocks are kept per layer (as ``append`` would build them)
        pk, pv = self._fused_apps(layer_id, k, v, old, status)
        step = self._step_for(layer_id, q.shape[1])
        out = None
        if self._fused_step_ok(D, B, H):
            try:
                out = step.append_attend(q, n, sm_scale, inv_tau, pk, pv)
            except NotImplementedError:
                # the library declined the one-launch step for these buffers (it enqueues
                # nothing then): the two launches below give the same bits
                out = None
        if out is None:
            self._launch_append(pk, pv, k.device)
            out = step.attend(q, n, sm_scale, inv_tau)
        self._layer_seq_lens[layer_id] = n
        if layer_id == 0:
            self._seq_len = n
        if status is not None:
            self._defer_status(layer_id, k.numel(), self._kind, self._qrange)
        return out

    def _raw_views(self, layer_id: int, n: Optional[int] = None):
        if layer_id < 0 or layer_id >= self.num_layers:
            raise ValueError(f"layer_id {layer_id} out of range [0, {self.num_layers})")
        if self._k_cache[layer_id] is None:
            raise ValueError(f"Cache for layer {layer_id} is empty")
        if n is None:
            n = self._layer_seq_lens[layer_id]
        kc = self._k_cache[layer_id][:, :, :n, :]
        vc = self._v_cache[layer_id][:, :, :n, :]
        B, H = kc.shape[0], kc.shape[1]

        def sv(buf, tok):
            if tok:
                return buf[:, :, :n, :]
            return buf[None, :, None, :].expand(B, H, n, buf.shape[-1])

        return kc, vc, sv(self._k_scale[layer_id], self._k_tok[layer_id]), \
            sv(self._v_scale[layer_id], self._v_tok[layer_id])

    def clear(self) -> None:
        self._discard_step_status()
        self._layer_seq_lens = [0] * self.num_layers
        self._seq_len = 0

    def release(self) -> None:
        n = self.num_layers
        self._k_cache, self._v_cache = [None] * n, [None] * n
        self._k_scale, self._v_scale = [None] * n, [None] * n
        self._steps, self._apps = [None] * n, [None] * n
        self._layer_seq_lens = [0] * n
        self._layer_capacity = [0] * n
        self._seq_len = 0

    def get_memory_mb(self) -> float:
        total = 0
        for i in range(self.num_layers):
            for buf in (self._k_cache[i], self._v_cache[i], self._k_scale[i], self._v_scale[i]):
                if buf is not None:
                    total += buf.numel() * buf.element_size()
        return total / (1024 * 1024)

    def to_tuple(self) -> Tuple[Tuple[Tensor, Tensor], ...]:
        out = []
        for i in range(self.num_layers):
            if self._k_cache[i] is None:
                raise ValueError(f"Layer {i} cache is empty")
            out.append(self.get_kv(i))
        return tuple(out)


class INT8KVCache(_SymCacheBase):
    """INT8 symmetric KV cache (src/cache/int8_cache.py:29)."""

    _fmt = C.KVQ_FMT_INT8_SYM
    _qrange = "[-127, 127]"
    _kind = "INT8"

    def __init__(
        self,
        num_layers: int,
        device: str = "cuda",
        clip_percentile: float = 99.9,
        group_size: int = 128,
        dtype: torch.dtype = torch.float16,
        max_seq_len: Optional[int] = None,
        decode_attn_impl: str = "triton_fused",
        static_k_scale: Optional[Tensor] = None,
        static_v_scale: Optional[Tensor] = None,
        inv_tau: Optional[Tensor] = None,
        use_attn_temperature: bool = True,
        adaptive_static_scales: bool = False,
        adaptive_static_margin: float = 1.0,
        adaptive_static_k: bool = True,
        adaptive_static_v: bool = True,
        check_numerics: bool = True,
    ):
        self._init_sym(num_layers, device, clip_percentile, group_size, dtype, max_seq_len,
                       decode_attn_impl, static_k_scale, static_v_scale, inv_tau,
                       use_attn_temperature, adaptive_static_scales, adaptive_static_margin,
                       adaptive_static_k, adaptive_static_v, check_numerics)

    def _code_dim(self, D):
        return D

    def _scale_dtype(self):
        return torch.float16

    def _side_is_token(self, side):
        st = self.static_k_scale if side == "k" else self.static_v_scale
        if st is None:
            return True
        return bool(self.adaptive_static_scales and
                    (self.adaptive_static_k if side == "k" else self.adaptive_static_v))

    def _effective_static(self, s):
        # quantize_symmetric_int8_with_scale: clamp(min=1e-5) then cast to fp16
        return s.clamp(min=1e-5).to(torch.float16)

    def _policy(self, p, side):
        if self._side_is_token(side):
            p.adaptive = 1
            p.adaptive_margin = float(self.adaptive_static_margin)

    def get_int8_tensors(self, layer_id: int) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
        """(k_int8, v_int8, k_scale, v_scale) views [B, H, S, D] / [B, H, S, G] (fp16 scales)."""
        return self._raw_views(layer_id)

    def _fused_step_ok(self, D: int, B: Optional[int] = None, H: Optional[int] = None) -> bool:
        # static tables on both sides (any group size), or per-token scales in groups of 16 or
        # more (the tiled kernel's row formats; its writer runs the append's arithmetic)
        if D != 128 or self.group_size not in (8, 16, 32, 64, 128):
            return False
        return self.group_size >= 16 or not (self._side_is_token("k") or self._side_is_token("v"))

    def get_kv(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        """Dequantize (code * scale in fp32) and return fp16 K/V (int8_cache.py:490-542)."""
        kc, vc, ks, vs = self._raw_views(layer_id)
        if kc.shape[2] == 0:
            logger.warning("get_kv(layer_id=%d) returning zero-length tensors.", layer_id)
        return _deq_sym(kc, ks).to(self.dtype), _deq_sym(vc, vs).to(self.dtype)

    @classmethod
    def from_tuple(cls, past_key_values, device: str = "cuda", clip_percentile: float = 99.9,
                   group_size: int = 128) -> "INT8KVCache":
        cache = cls(num_layers=len(past_key_values), device=device,
                    clip_percentile=clip_percentile, group_size=group_size)
        for i, (k, v) in enumerate(past_key_values):
            cache.append(i, k.to(device), v.to(device))
        return cache

    def __repr__(self) -> str:
        return (f"INT8KVCache(num_layers={self.num_layers}, seq_len={self._seq_len}, "
                f"memory={self.get_memory_mb():.2f}MB)")


class INT4KVCache(_SymCacheBase):
    """INT4 symmetric, bit-packed KV cache (src/cache/int4_cache.py:32)."""

    _fmt = C.KVQ_FMT_INT4_SYM
    _qrange = "[-7, 7]"
    _kind = "INT4"

    def __init__(
        self,
        num_layers: int,
        device: str = "cuda",
        clip_percentile: float = 99.9,
        group_size: int = 32,
        dtype: torch.dtype = torch.float16,
        max_seq_len: Optional[int] = None,
        bit_packed: bool = True,
        decode_attn_impl: str = "triton_fused",
        static_k_scale: Optional[Tensor] = None,
        static_v_scale: Optional[Tensor] = None,
        inv_tau: Optional[Tensor] = None,
        use_attn_temperature: bool = True,
        adaptive_static_scales: bool = False,
        adaptive_static_margin: float = 1.0,
        adaptive_static_k: bool = True,
        adaptive_static_v: bool = True,
        outlier_rescue_ratio: float = 0.0,
        mixed_rescue: bool = False,
        check_numerics: bool = True,
    ):
        if outlier_rescue_ratio < 0.0 or outlier_rescue_ratio > 1.0:
            raise ValueError(f"outlier_rescue_ratio must be in [0, 1], got {outlier_rescue_ratio}")
        self._init_sym(num_layers, device, clip_percentile, group_size, dtype, max_seq_len,
                       decode_attn_impl, static_k_scale, static_v_scale, inv_tau,
                       use_attn_temperature, adaptive_static_scales, adaptive_static_margin,
                       adaptive_static_k, adaptive_static_v, check_numerics)
        # The codes are stored packed either way (the kernels read them so); with
        # bit_packed=False get_int4_tensors returns them unpacked, one int8 code per channel,
        # as the reference's unpacked cache does (src/cache/int4_cache.py:531-537, 623-625).
        self.bit_packed = bool(bit_packed)
        self.outlier_rescue_ratio = float(outlier_rescue_ratio)
        self.mixed_rescue = bool(mixed_rescue)

    def _code_dim(self, D):
        return D // 2

    def _scale_dtype(self):
        return torch.float32

    def _side_is_token(self, side):
        st = self.static_k_scale if side == "k" else self.static_v_scale
        if st is None:
            return True
        adaptive = self.adaptive_static_scales and (
            self.adaptive_static_k if side == "k" else self.adaptive_static_v)
        return bool(adaptive or self.mixed_rescue or self.outlier_rescue_ratio > 0.0)

    def _effective_static(self, s):
        return s.to(torch.float32).clamp(min=1e-5)

    def _fused_step_ok(self, D: int, B: Optional[int] = None, H: Optional[int] = None) -> bool:
        # the tiled kernel's row format (groups of 16 or more) appends in the same launch; the
        # group rescue's threshold (torch.quantile over every (row, group) scale of the append,
        # int4_cache.py:384-390) is found by the decode kernel's writer wave when it lies within
        # its walk from the top: at most 32 rows (B * H), lower rank within 32 of the top
        if D != 128 or self.group_size < 16:
            return False
        rescue = 0.0 < self.outlier_rescue_ratio < 1.0 and (
            self.static_k_scale is not None or self.static_v_scale is not None)
        if not rescue:
            return True
        if B is None or H is None:
            return False
        import numpy as np

        n = B * H * (D // self.group_size)
        q = np.float32(max(0.0, min(1.0, 1.0 - self.outlier_rescue_ratio)))
        lo = int(np.floor(q * np.float32(n - 1)))
        return B * H <= 32 and n - 1 - lo < 32

    def _policy(self, p, side):
        adaptive = self.adaptive_static_scales and (
            self.adaptive_static_k if side == "k" else self.adaptive_static_v)
        p.adaptive = int(bool(adaptive))
        p.adaptive_margin = float(self.adaptive_static_margin)
        p.mixed_rescue = int(self.mixed_rescue)
        r = self.outlier_rescue_ratio
        if r >= 1.0:
            p.rescue_all = 1
        elif r > 0.0:
            p.rescue_quantile = float(max(0.0, min(1.0, 1.0 - r)))

    def _pre_append_checks(self, layer_id):
        missing = [s for s, t in (("K", self.static_k_scale), ("V", self.static_v_scale)) if t is None]
        if missing:
            side = " and ".join(missing)
            if self.outlier_rescue_ratio > 0:
                warnings.warn(
                    f"KVC-031: outlier_rescue_ratio={self.outlier_rescue_ratio} has no effect on "
                    f"{side} at layer {layer_id} because no static {side} scale is provided.",
                    RuntimeWarning)
            if self.mixed_rescue:
                warnings.warn(
                    f"KVC-031: mixed_rescue=True has no effect on {side} at layer {layer_id} "
                    f"because no static {side} scale is provided.", RuntimeWarning)

    def get_int4_tensors(self, layer_id: int) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
        """(k, v, k_scale, v_scale) over the stored tokens, fp32 scales [B,H,S,G]: with
        bit_packed the packed codes [B,H,S,D/2] (views of the cache), else the codes unpacked
        to int8 [B,H,S,D] in [-8, 7] (new tensors, which decode_attn_int4(bit_packed=False)
        takes)."""
        kc, vc, ks, vs = self._raw_views(layer_id)
        if self.bit_packed:
            return kc, vc, ks, vs
        return _unpack(kc), _unpack(vc), ks, vs

    def get_kv(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        kc, vc, ks, vs = self._raw_views(layer_id)
        return (_deq_sym(_unpack(kc), ks).to(self.dtype), _deq_sym(_unpack(vc), vs).to(self.dtype))

    @classmethod
    def from_tuple(cls, past_key_values, device: str = "cuda", clip_percentile: float = 99.9,
                   group_size: int = 32, bit_packed: bool = True) -> "INT4KVCache":
        cache = cls(num_layers=len(past_key_values), device=device, clip_percentile=clip_percentile,
                    group_size=group_size, bit_packed=bit_packed)
        for i, (k, v) in enumerate(past_key_values):
            cache.append(i, k.to(device), v.to(device))
        return cache

    def __repr__(self) -> str:
        return (f"INT4KVCache(num_layers={self.num_layers}, seq_len={self._seq_len}, "
                f"memory={self.get_memory_mb():.2f}MB)")


def _unpack(packed: Tensor) -> Tensor:
    u = packed.view(torch.uint8)
    out = torch.stack([(u >> 4) & 0x0F, u & 0x0F], dim=-1).view(*packed.shape[:-1], packed.shape[-1] * 2)
    return (out.to(torch.int16) - 8).to(torch.int8)


def _deq_sym(q: Tensor, s: Tensor) -> Tensor:
    B, H, S, D = q.shape
    G = s.shape[-1]
    return (q.view(B, H, S, G, D // G).to(s.dtype) * s.unsqueeze(-1)).view(B, H, S, D)


class _StaticG32Cache(_EngineBase):
    """Caches whose every scale is static per (layer, head, group of 32).

    Per layer: K codes [B, H, cap, 64] packed INT4 (asymmetric, byte = hi nibble even
    channel, codes c + 8 with c in [-8, 7]) or [B, H, cap, 128] INT8 (symmetric).  V codes
    are packed asymmetric INT4 kept in the TILE32 layout [B, H, cap / 32, 2048] the decode
    kernels stream (:func:`kernels.tile_v`).  The static tables are [L, H, 4].  With
    ``k_outlier_idx`` (INT4 K only) those 4 K channels per head are also stored verbatim
    in fp16 [B, H, cap, 4] and replace the dequantised codes.  No per-token scale is
    stored: the kernels read the static tables.
    """

    _k_int8 = False

    def __init__(self, num_layers: int, k_scale: Tensor, k_zp: Optional[Tensor], v_scale: Tensor,
                 v_zp: Tensor, device: str = "cuda", max_seq_len: Optional[int] = None,
                 k_outlier_idx: Optional[Tensor] = None, inv_tau: Optional[Tensor] = None,
                 use_attn_temperature: bool = True, decode_attn_impl: str = "hip_fused",
                 check_numerics: bool = False):
        self._init_common(num_layers, device, max_seq_len, decode_attn_impl, check_numerics)
        self.group_size = 32
        for name, t in (("k_scale", k_scale), ("v_scale", v_scale), ("v_zp", v_zp)) + \
                (() if self._k_int8 else (("k_zp", k_zp),)):
            if t is None or t.ndim != 3 or t.shape[0] != num_layers or t.shape[-1] != 4:
                raise ValueError(f"{name} must be [L, H, 4], got "
                                 f"{None if t is None else tuple(t.shape)}")
        # INT8 K keeps the reference's fp16 clamp(min=1e-5) of the static scale
        # (src/quant/int8_basic.py:159); the INT4 tables are fp16 as stored.
        self.k_scale = k_scale.to(device=device, dtype=torch.float16).contiguous()
        self.k_zp = None if self._k_int8 else k_zp.to(device=device, dtype=torch.float16).contiguous()
        self.v_scale = v_scale.to(device=device, dtype=torch.float16).contiguous()
        self.v_zp = v_zp.to(device=device, dtype=torch.float16).contiguous()
        if k_outlier_idx is not None:
            if self._k_int8:
                raise ValueError("k_outlier_idx needs INT4 K")
            oi = k_outlier_idx.detach().cpu()
            if oi.ndim != 3 or oi.shape[0] != num_layers or oi.shape[-1] != 4:
                raise ValueError(f"k_outlier_idx must be [L, H, 4], got {tuple(oi.shape)}")
            if oi.min() < 0 or oi.max() > 127:
                raise ValueError("k_outlier_idx values must lie in [0, 128)")
            if any(len(set(r.tolist())) != 4 for r in oi.reshape(-1, 4)):
                raise ValueError("k_outlier_idx channels must be distinct per head")
        self.k_outlier_idx = (None if k_outlier_idx is None else
                              k_outlier_idx.to(device=device, dtype=torch.int32).contiguous())
        self.inv_tau = inv_tau
        self.use_attn_temperature = use_attn_temperature
        n = num_layers
        self._k: List[Optional[Tensor]] = [None] * n
        self._v: List[Optional[Tensor]] = [None] * n
        self._ko: List[Optional[Tensor]] = [None] * n

    @property
    def v_tiled(self) -> bool:
        """V codes are kept in the TILE32 layout rather than as rows."""
        return True

    def _ensure(self, layer_id, B, H, target):
        cap = self._layer_capacity[layer_id]
        if self._k[layer_id] is not None:
            kb = self._k[layer_id]
            if kb.shape[0] != B or kb.shape[1] != H:
                raise ValueError(f"Inconsistent KV shape for layer {layer_id}")
            if target <= cap:
                return
        new_cap = self._new_capacity(layer_id, target, cap if self._k[layer_id] is not None else 0)
        new_cap = -(-new_cap // TILE_TOKENS) * TILE_TOKENS
        old = self._layer_seq_lens[layer_id]
        nk = torch.empty((B, H, new_cap, 128 if self._k_int8 else 64), dtype=torch.uint8,
                         device=self.device)
        if self.v_tiled:
            nv = torch.empty((B, H, new_cap // TILE_TOKENS, TILE_BYTES), dtype=torch.uint8,
                             device=self.device)
        else:
            nv = torch.empty((B, H, new_cap, 64), dtype=torch.uint8, device=self.device)
        no = (torch.empty((B, H, new_cap, 4), dtype=torch.float16, device=self.device)
              if self.k_outlier_idx is not None else None)
        if self._k[layer_id] is not None and old:
            nk[:, :, :old] = self._k[layer_id][:, :, :old]
            vold = -(-old // TILE_TOKENS) if self.v_tiled else old
            nv[:, :, :vold] = self._v[layer_id][:, :, :vold]
            if no is not None:
                no[:, :, :old] = self._ko[layer_id][:, :, :old]
        self._k[layer_id], self._v[layer_id], self._ko[layer_id] = nk, nv, no
        self._layer_capacity[layer_id] = new_cap
        self._steps[layer_id] = self._apps[layer_id] = None

    def _append_params(self, layer_id: int, k: Tensor, v: Tensor, pos: int, status):
        """kvq_append_params for K and V of this layer written at slot pos, and the
        tensors they point at."""
        pk, pv = C.AppendParams(), C.AppendParams()
        keep = []
        kfmt = C.KVQ_FMT_INT8_SYM if self._k_int8 else C.KVQ_FMT_INT4_ASYM
        for side, p, x, codes, s, z, fmt in (
                ("k", pk, k, self._k[layer_id], self.k_scale, self.k_zp, kfmt),
                ("v", pv, v, self._v[layer_id], self.v_scale, self.v_zp, C.KVQ_FMT_INT4_ASYM)):
            xs = x if x.stride(-1) == 1 else x.contiguous()
            keep.append(xs)
            sptr = None if status is None else status.data_ptr() + (0 if side == "k" else 8)
            _fill_append(p, fmt, xs, 32, codes, pos, sptr)
            if side == "v" and self.v_tiled:
                p.codes_layout = C.KVQ_LAYOUT_TILE32
                p.codes_stride_t = 64
                p.capacity = codes.shape[2] * TILE_TOKENS
            sl = s[layer_id]
            p.static_scale = sl.data_ptr()
            if z is not None:
                p.static_zp = z[layer_id].data_ptr()
            p.static_scale_dtype = C.KVQ_DTYPE_F16
            p.static_stride_h, p.static_stride_g = sl.stride()
            if side == "k" and self.k_outlier_idx is not None:
                oi, oo = self.k_outlier_idx[layer_id], self._ko[layer_id]
                p.n_outlier = oi.shape[-1]
                p.outlier_idx, p.outlier_out = oi.data_ptr(), oo.data_ptr()
                p.oo_stride_b, p.oo_stride_h, p.oo_stride_t = oo.stride(0), oo.stride(1), oo.stride(2)
        return pk, pv, keep

    def append(self, layer_id: int, k: Tensor, v: Tensor) -> None:
        self._validate_kv(layer_id, k, v)
        B, H, S, D = k.shape
        if self.k_scale.shape[1] != H:
            raise ValueError(f"calibration vs model heads mismatch: {self.k_scale.shape[1]} vs {H}")
        old = self._layer_seq_lens[layer_id]
        self._ensure(layer_id, B, H, old + S)
        if S == 0:
            return
        status = self._status_buf(k.device) if self.check_numerics else None
        pk, pv, keep = self._append_params(layer_id, k, v, old, status)
        self._launch_append(pk, pv, k.device)
        if status is not None:
            self._check_status(layer_id, k.numel(), "K8V4" if self._k_int8 else "INT4-asym",
                               "the code range")
        self._layer_seq_lens[layer_id] = old + S
        if layer_id == 0:
            self._seq_len = old + S

    def _k_view(self, layer_id: int, n: int):
        """(format, view) of layer_id's K over its first n tokens for the decode kernels."""
        from .kernels import kv_view_static, kv_view_tok

        kb = self._k[layer_id][:, :, :n]
        if self._k_int8:
            B, H = kb.shape[:2]
            ks = self.k_scale[layer_id].clamp(min=1e-5)[None, :, None, :].expand(B, H, n, 4)
            return C.KVQ_FMT_INT8_SYM, kv_view_tok(kb.view(torch.int8), ks)
        ob = None if self._ko[layer_id] is None else self._ko[layer_id][:, :, :n]
        oi = None if self.k_outlier_idx is None else self.k_outlier_idx[layer_id]
        return C.KVQ_FMT_INT4_ASYM, kv_view_static(kb, self.k_scale[layer_id], self.k_zp[layer_id], oi, ob)

    def _step_for(self, layer_id: int, q_heads: int):
        """The layer's LayerStep (kernels.LayerStep) over its whole buffers."""
        kb = self._k[layer_id]
        st = self._steps[layer_id]
        if st is not None and st.key == (q_heads, kb.data_ptr()):
            return st
        from .kernels import LayerStep, kv_view_static

        B, H, cap = kb.shape[0], kb.shape[1], kb.shape[2]
        kfmt, kview = self._k_view(layer_id, cap)
        vb = self._v[layer_id]
        st = LayerStep(kfmt, kview, C.KVQ_FMT_INT4_ASYM,
                       kv_view_static(vb, self.v_scale[layer_id], self.v_zp[layer_id]),
                       B, q_heads, H, 32, kb.device, keepalive=(vb,))
        st.key = (q_heads, kb.data_ptr())
        self._steps[layer_id] = st
        return st

    def append_decode_attn(self, layer_id: int, q: Tensor, k: Tensor, v: Tensor,
                           sm_scale: Optional[float] = None,
                           inv_tau: Optional[Tensor] = None) -> Tensor:
        """Decode step of one layer in one HIP launch: append the new token (k, v: fp16
        [B, H, 1, 128]) and attend over the layer's whole cache, the new token included.
        Returns fp16 [B, Hq, 128].  Codes and output are bit-identical to ``append`` then
        the decode kernel over the cache's tensors with context lengths ``get_seq_len()``
        (the append + attention of the reference's decode step,
        src/engine/patch_model.py:755-957).  The kernel parameters are kept per layer
        between calls.  With ``check_numerics``, NaN / Inf in k or v raise ValueError and
        the cache does not advance."""
        self._validate_kv(layer_id, k, v)
        B, H, S, D = k.shape
        if S != 1:
            raise ValueError(f"append_decode_attn appends one token per step, got S={S}")
        if self.k_scale.shape[1] != H:
            raise ValueError(f"calibration vs model heads mismatch: {self.k_scale.shape[1]} vs {H}")
        if q.ndim != 3 or q.dtype != torch.float16 or q.shape[0] != B or q.shape[1] % H \
                or q.shape[2] != 128:
            raise ValueError(f"q must be fp16 [B, Hq, 128] with Hq a multiple of {H}, got "
                             f"{q.dtype} {tuple(q.shape)}")
        if q.stride(-1) != 1:
            q = q.contiguous()
        old = self._layer_seq_lens[layer_id]
        self._ensure(layer_id, B, H, old + 1)
        n = old + 1
        if sm_scale is None:
            sm_scale = 1.0 / math.sqrt(D)
        sptr = self._step_status_ptr(layer_id, k.device) if self.check_numerics else None
        ent = self._apps[layer_id]
        if ent is None:
            pk, pv, _ = self._append_params(layer_id, k, v, old, None)
            ent = (pk, pv)
            self._apps[layer_id] = ent
        pk, pv = ent
        for p, x, off in ((pk, k, 0), (pv, v, 8)):
            if x.stride(-1) != 1:
                x = x.contiguous()
            p.x = x.data_ptr()
            p.x_stride_b, p.x_stride_h, p.x_stride_s = x.stride()[:3]
            p.write_pos = old
            p.status = None if sptr is None else sptr + off
            p._keep = (x,)
        out = self._step_for(layer_id, q.shape[1]).append_attend(q, n, sm_scale, inv_tau, pk, pv)
        self._layer_seq_lens[layer_id] = n
        if layer_id == 0:
            self._seq_len = n
        if sptr is not None:
            self._defer_status(layer_id, k.numel(), "K8V4" if self._k_int8 else "INT4-asym",
                               "the code range")
        return out

    def _check_layer(self, layer_id: int) -> int:
        if self._k[layer_id] is None:
            raise ValueError(f"Cache for layer {layer_id} is empty")
        return self._layer_seq_lens[layer_id]

    def clear(self) -> None:
        self._discard_step_status()
        self._layer_seq_lens = [0] * self.num_layers
        self._seq_len = 0

    def release(self) -> None:
        n = self.num_layers
        self._k, self._v, self._ko = [None] * n, [None] * n, [None] * n
        self._steps, self._apps = [None] * n, [None] * n
        self._layer_seq_lens = [0] * n
        self._layer_capacity = [0] * n
        self._seq_len = 0

    def get_memory_mb(self) -> float:
        total = 0
        for bufs in (self._k, self._v, self._ko):
            for b in bufs:
                if b is not None:
                    total += b.numel() * b.element_size()
        return total / (1024 * 1024)


class INT4AsymKVCache(_StaticG32Cache):
    """Asymmetric INT4 K and V with static group-32 scale / zero-point (configs 2 and 3),
    optionally with 4 fp16 outlier K channels per head."""

    def get_int4_g32_tensors(self, layer_id: int):
        """(k_codes [B,H,n,64], v_tiles [B,H,ceil(n/32),2048] (TILE32 layout), k_scale, k_zp,
        v_scale, v_zp, k_outlier_idx, k_outlier_val [B,H,n,4]).  ``untile_v(v_tiles, n)``
        gives V as packed rows."""
        n = self._check_layer(layer_id)
        ko = None if self._ko[layer_id] is None else self._ko[layer_id][:, :, :n]
        oi = None if self.k_outlier_idx is None else self.k_outlier_idx[layer_id]
        vt = self._v[layer_id][:, :, :-(-n // TILE_TOKENS)]
        return (self._k[layer_id][:, :, :n], vt, self.k_scale[layer_id],
                self.k_zp[layer_id], self.v_scale[layer_id], self.v_zp[layer_id], oi, ko)


class K8V4KVCache(_StaticG32Cache):
    """K INT8 symmetric with a static group-32 scale, V asymmetric INT4 with static group-32
    scale / zero-point (config 4).  The reference's closest engine is MixedKVCache
    (src/cache/mixed_kv_cache.py:150-248), whose quantizers are dynamic per token; this
    one uses the static tables of the INT8 path (src/quant/int8_basic.py:111-164) for K."""

    _k_int8 = True

    def __init__(self, num_layers: int, k_scale: Tensor, v_scale: Tensor, v_zp: Tensor,
                 device: str = "cuda", max_seq_len: Optional[int] = None,
                 inv_tau: Optional[Tensor] = None, use_attn_temperature: bool = True,
                 decode_attn_impl: str = "hip_fused", check_numerics: bool = False):
        super().__init__(num_layers, k_scale, None, v_scale, v_zp, device=device,
                         max_seq_len=max_seq_len, inv_tau=inv_tau,
                         use_attn_temperature=use_attn_temperature,
                         decode_attn_impl=decode_attn_impl, check_numerics=check_numerics)

    def get_k8v4_tensors(self, layer_id: int):
        """(k_codes int8 [B,H,n,128], k_scale fp16 [B,H,n,4] (a stride-0 view of the static
        table after the fp16 clamp to 1e-5), v_tiles [B,H,ceil(n/32),2048] (TILE32 layout;
        ``untile_v(v_tiles, n)`` gives packed rows), v_scale, v_zp)."""
        n = self._check_layer(layer_id)
        k = self._k[layer_id][:, :, :n].view(torch.int8)
        B, H = k.shape[:2]
        ks = self.k_scale[layer_id].clamp(min=1e-5)[None, :, None, :].expand(B, H, n, 4)
        vt = self._v[layer_id][:, :, :-(-n // TILE_TOKENS)]
        return k, ks, vt, self.v_scale[layer_id], self.v_zp[layer_id]


_KIVI_BITS = (4, 8, 16)


def _kivi_format(bits: int) -> int:
    return {4: C.KVQ_FMT_INT4_KIVI, 8: C.KVQ_FMT_INT8_KIVI, 16: C.KVQ_FMT_FP16}[bits]


def _kivi_row(bits: int) -> Tuple[int, torch.dtype]:
    """(elements per token row, dtype) of a side's storage: packed nibbles, int8 codes or
    fp16 values."""
    return {4: (64, torch.int8), 8: (128, torch.int8), 16: (128, torch.float16)}[bits]


def _kivi_levels(percentile: float) -> Tuple[float, float]:
    """The two quantile levels of quantize_asymmetric's clipping (src/quant/asymmetric_quant.py:
    97-103): (100 - p) / 100 and p / 100, or (0, 0) for the min / max at p = 100."""
    p = float(percentile)
    if not (50.0 < p <= 100.0):
        raise ValueError(f"percentile must be in (50.0, 100.0], got {percentile}. Values <= 50 invert "
                         "min/max and produce silent errors.")
    if p >= 100.0:
        return 0.0, 0.0
    return max(0.0, min((100.0 - p) / 100.0, 1.0)), max(0.0, min(p / 100.0, 1.0))


def _sorted_quantile(sorted_x: Tensor, q: float, dim: int) -> Tensor:
    """torch.quantile(x, q, dim) from x sorted along dim: the order statistics at floor / ceil
    of fp32(q) * (n - 1) and torch.lerp between them (ATen's quantile, without its input-size
    limit)."""
    import numpy as np

    n = sorted_x.shape[dim]
    rank = np.float32(q) * np.float32(n - 1)
    lo, hi = int(np.floor(rank)), int(np.ceil(rank))
    w = float(np.float32(rank - np.float32(lo)))
    return torch.lerp(sorted_x.select(dim, lo), sorted_x.select(dim, hi), w)


def kivi_channel_params(k: Tensor, bits: int, percentile: float) -> Tuple[Tensor, Tensor]:
    """Per-channel K scale / zero-point over the tokens of a prefill k [B, H, S, D]
    (quantize_asymmetric_per_channel, src/quant/asymmetric_quant.py:24-141, 199-224): the
    range (min / max, or the two quantiles) in fp32, floored at max(1e-5, fp16 tiny x
    (qmax - qmin)), divided by qmax - qmin; z = min - qmin s.  fp32 [B, H, D]."""
    qmin, qmax = (-8, 7) if bits == 4 else (-128, 127)
    lo_q, hi_q = _kivi_levels(percentile)
    kf = k.float()
    if hi_q > 0.0:
        srt = torch.sort(kf, dim=2).values
        t_min, t_max = _sorted_quantile(srt, lo_q, 2), _sorted_quantile(srt, hi_q, 2)
    else:
        t_min, t_max = torch.aminmax(kf, dim=2)
    span = float(qmax - qmin)
    floor = max(1e-5, float(torch.finfo(torch.float16).tiny) * span)
    # IEEE division, as the formula reads and torch computes it on the CPU (a GPU tensor
    # divided by a Python scalar is multiplied by fp32(1 / span) instead)
    rng = (t_max - t_min).clamp(min=floor)
    s = rng / torch.full_like(rng, span)
    return s.contiguous(), (t_min - qmin * s).contiguous()


class _KiviFamily(_EngineBase):
    """Storage and kernels of the KIVI family (src/cache/kivi_style_cache.py:38-900,
    src/cache/role_aware_allocator_cache.py:73-502): per layer a (k_bits, v_bits) pair from
    {4, 8, 16}.  A quantized K side has per-channel asymmetric codes with the scale / zero-point
    frozen at prefill ([B, H, D] fp32); a quantized V side per-token codes ([B, H, T] fp32
    parameters); a 16-bit side keeps fp16 values.  Codes: 4 bits packed [B, H, T, 64] (byte =
    ((c[2i]+8) << 4) | (c[2i+1]+8)), 8 bits int8 [B, H, T, 128].  Every quantized token goes
    through kvq_quant_append (HIP; per-token percentile clipping in the kernel); the prefill's
    per-channel K range is reduced with torch (aminmax, or a sort and torch.lerp for a
    percentile, as torch.quantile does).  Decode attention reads the cache in place through the
    tiled kernel of the layer's pair (kvq_decode_attn), the fp16 residual window (residual_length
    > 0) with it, merged by the kernel's merging work-group.
    """

    _min_capacity = 256

    def _init_kivi(self, num_layers, device, dtype, max_seq_len, bits, k_percentile, v_percentile,
                   inv_tau, use_attn_temperature, residual_length, decode_attn_impl, check_numerics):
        _kivi_levels(k_percentile)
        _kivi_levels(v_percentile)
        self._init_common(num_layers, device, max_seq_len, decode_attn_impl, check_numerics)
        self.dtype = dtype
        self.k_percentile, self.v_percentile = float(k_percentile), float(v_percentile)
        self.residual_length = max(0, int(residual_length))
        if self.residual_length > 65536:
            raise NotImplementedError("residual_length above 65536 is not built (the decode "
                                      "kernel attends the fp16 window in one work-group)")
        # fp16 residual window (kivi_style_cache.py:102-113): per layer a ring of the
        # residual_length most recent decode tokens, _res_len of them valid, the oldest at
        # _res_start once the ring is full
        self._res_k: List[Optional[Tensor]] = [None] * num_layers
        self._res_v: List[Optional[Tensor]] = [None] * num_layers
        self._res_len = [0] * num_layers
        self._res_start = [0] * num_layers
        self.inv_tau = inv_tau
        self.use_attn_temperature = bool(use_attn_temperature)
        self._scale_dtype = torch.float32
        self._bits = [tuple(b) for b in bits]
        n = num_layers
        self._k_cache: List[Optional[Tensor]] = [None] * n
        self._v_cache: List[Optional[Tensor]] = [None] * n
        self._k_scale: List[Optional[Tensor]] = [None] * n
        self._k_zp: List[Optional[Tensor]] = [None] * n
        self._v_scale: List[Optional[Tensor]] = [None] * n
        self._v_zp: List[Optional[Tensor]] = [None] * n
        self._k_scale_initialized = [False] * n
        self._oor_check_interval = int(os.environ.get("KV_OOR_CHECK_INTERVAL", "0"))
        self._oor_step_counter = 0

    def _resolve_bits(self, layer_id: int) -> Tuple[int, int]:
        return self._bits[layer_id]

    def _ensure(self, layer_id: int, B: int, H: int, target: int, device) -> None:
        kb, vb = self._bits[layer_id]
        kc0 = self._k_cache[layer_id]
        if kc0 is not None and (kc0.shape[0] != B or kc0.shape[1] != H):
            raise ValueError(f"Inconsistent KV shape for layer {layer_id}: existing K={tuple(kc0.shape)}, "
                             f"incoming=({B}, {H}, *, 128)")
        cap = self._layer_capacity[layer_id]
        if kc0 is not None and target <= cap:
            return
        new_cap = self._new_capacity(layer_id, target, cap if kc0 is not None else 0)
        new_cap = ((new_cap + TILE_TOKENS - 1) // TILE_TOKENS) * TILE_TOKENS
        old = self._layer_seq_lens[layer_id]
        (kw, kdt), (vw, vdt) = _kivi_row(kb), _kivi_row(vb)
        kc = torch.zeros(B, H, new_cap, kw, dtype=kdt, device=device)
        vc = torch.zeros(B, H, new_cap, vw, dtype=vdt, device=device)
        vs = vz = None
        if vb != 16:
            vs = torch.zeros(B, H, new_cap, dtype=torch.float32, device=device)
            vz = torch.zeros_like(vs)
        if kc0 is not None and old > 0:
            kc[:, :, :old] = kc0[:, :, :old]
            vc[:, :, :old] = self._v_cache[layer_id][:, :, :old]
            if vs is not None:
                vs[:, :, :old] = self._v_scale[layer_id][:, :, :old]
                vz[:, :, :old] = self._v_zp[layer_id][:, :, :old]
        self._k_cache[layer_id], self._v_cache[layer_id] = kc, vc
        self._v_scale[layer_id], self._v_zp[layer_id] = vs, vz
        self._layer_capacity[layer_id] = new_cap
        self._steps[layer_id] = self._apps[layer_id] = None

    def _residual_seq(self) -> int:
        return max(q + r for q, r in zip(self._layer_seq_lens, self._res_len))

    def append(self, layer_id: int, k: Tensor, v: Tensor) -> None:
        """Quantize (or store) and append k, v fp16 [B, H, S, 128] (kivi_style_cache.py:296-617,
        role_aware_allocator_cache.py:311-400).  With residual_length R, a decode token (S = 1
        after the prefill) goes to the fp16 window; once R are held, the oldest is quantized
        into the cache and the new token takes its slot (kivi_style_cache.py:354-404)."""
        self._validate_kv(layer_id, k, v)
        B, H, S, D = k.shape
        R = self.residual_length
        if R > 0 and S == 1 and self._k_scale_initialized[layer_id]:
            if self._res_k[layer_id] is None:
                self._res_k[layer_id] = torch.zeros(B, H, R, D, dtype=torch.float16, device=k.device)
                self._res_v[layer_id] = torch.zeros_like(self._res_k[layer_id])
            rk, rv = self._res_k[layer_id], self._res_v[layer_id]
            if tuple(rk.shape[:2]) != (B, H):
                raise ValueError(f"Inconsistent KV shape for layer {layer_id}: residual window "
                                 f"{tuple(rk.shape)}, incoming {tuple(k.shape)}")
            rlen = self._res_len[layer_id]
            if rlen < R:
                rk[:, :, rlen] = k[:, :, 0]
                rv[:, :, rlen] = v[:, :, 0]
                self._res_len[layer_id] = rlen + 1
                self._seq_len = self._residual_seq()
                return
            slot = self._res_start[layer_id]
            # the oldest token is quantized from its slot (the kernel reads it before the
            # copy of the new token, which follows on the same stream)
            self._append_quantized(layer_id, rk[:, :, slot:slot + 1], rv[:, :, slot:slot + 1])
            rk[:, :, slot] = k[:, :, 0]
            rv[:, :, slot] = v[:, :, 0]
            self._res_start[layer_id] = (slot + 1) % R
            self._seq_len = self._residual_seq()
            return
        self._append_quantized(layer_id, k, v)
        if R > 0:
            self._seq_len = self._residual_seq()

    def _append_quantized(self, layer_id: int, k: Tensor, v: Tensor) -> None:
        B, H, S, D = k.shape
        old = self._layer_seq_lens[layer_id]
        if S == 0:
            return
        kb, vb = self._bits[layer_id]
        self._ensure(layer_id, B, H, old + S, k.device)
        prefill = kb != 16 and not self._k_scale_initialized[layer_id]
        # the frozen-K range check of decode appends runs every KV_OOR_CHECK_INTERVAL steps
        # (0, the default: never), counted on layer 0 (kivi_style_cache.py:143-144, 549-560)
        oor_check = False
        if kb != 16 and not prefill and self._oor_check_interval > 0:
            if layer_id == 0:
                self._oor_step_counter += 1
            oor_check = self._oor_step_counter % self._oor_check_interval == 0
        if prefill:
            if self.check_numerics and not bool(torch.isfinite(k).all()):
                raise ValueError("quantize_asymmetric: input contains NaN or Inf")
            self._k_scale[layer_id], self._k_zp[layer_id] = kivi_channel_params(k, kb, self.k_percentile)
            self._k_scale_initialized[layer_id] = True
        if kb != 16:
            ks = self._k_scale[layer_id]
            if tuple(ks.shape) != (B, H, D):
                raise ValueError(f"Inconsistent decode K scale/zp shape for layer {layer_id}: "
                                 f"expected {(B, H, D)}, got {tuple(ks.shape)}")
        # the status words (NaN flags, K range count) cost a host sync: read at prefill with
        # check_numerics, and on the decode steps the range check selects
        status = self._status_buf(k.device) if (self.check_numerics and prefill) or oor_check else None
        sp = None if status is None else status.data_ptr()
        ksx = k if k.stride(-1) == 1 else k.contiguous()
        vsx = v if v.stride(-1) == 1 else v.contiguous()
        pk = pv = None
        if kb == 16:
            self._k_cache[layer_id][:, :, old:old + S] = ksx
        else:
            pk = C.AppendParams()
            _fill_append(pk, _kivi_format(kb), ksx, 32, self._k_cache[layer_id], old, sp)
            ks, kz = self._k_scale[layer_id], self._k_zp[layer_id]
            pk.static_scale, pk.static_zp = ks.data_ptr(), kz.data_ptr()
            pk.static_scale_dtype = C.KVQ_DTYPE_F32
            pk.static_stride_b, pk.static_stride_h, pk.static_stride_g = ks.stride()
        if vb == 16:
            self._v_cache[layer_id][:, :, old:old + S] = vsx
        else:
            pv = C.AppendParams()
            _fill_append(pv, _kivi_format(vb), vsx, 32, self._v_cache[layer_id], old,
                         None if sp is None else sp + 8)
            vs, vz = self._v_scale[layer_id], self._v_zp[layer_id]
            pv.scale_out, pv.zp_out, pv.scale_out_dtype = vs.data_ptr(), vz.data_ptr(), C.KVQ_DTYPE_F32
            pv.so_stride_b, pv.so_stride_h, pv.so_stride_t = vs.stride()
            pv.dyn_quantile_lo, pv.dyn_quantile = _kivi_levels(self.v_percentile)
        if pk is not None or pv is not None:
            C.check(C.lib().kvq_quant_append(None if pk is None else ctypes.byref(pk),
                                             None if pv is None else ctypes.byref(pv),
                                             ctypes.c_void_p(C.stream_handle(k.device))))
        if status is not None:
            st = self._read_status()
            if st[0] & 1 or st[2] & 1:
                raise ValueError(f"KIVI append: {'K' if st[0] & 1 else 'V'} input contains NaN or Inf "
                                 "— refusing to quantize corrupt data")
            ratio = st[1] / max(k.numel(), 1)
            if oor_check and ratio > _CLIP_WARN_THRESHOLD:
                lo, hi = (-8, 7) if kb == 4 else (-128, 127)
                warnings.warn(
                    f"ENG-041: KIVI decode K clipping at layer {layer_id}: {ratio:.1%} of values exceed "
                    f"prefill-computed scale range [{lo}, {hi}]. Decode token magnitudes may have drifted "
                    "beyond prefill calibration. Attention accuracy may degrade.", RuntimeWarning)
        self._layer_seq_lens[layer_id] = old + S
        self._seq_len = max(self._layer_seq_lens)

    def _check_layer(self, layer_id: int) -> int:
        if layer_id < 0 or layer_id >= self.num_layers:
            raise ValueError(f"layer_id {layer_id} out of range [0, {self.num_layers})")
        if self._k_cache[layer_id] is None:
            raise ValueError(f"Cache for layer {layer_id} is empty")
        n = self._layer_seq_lens[layer_id]
        if n <= 0:
            raise ValueError(f"Cache for layer {layer_id} has no tokens")
        return n

    def get_kivi_tensors(self, layer_id: int):
        """(k_store, v_store, k_scale, k_zp, v_scale, v_zp) over the stored tokens: packed /
        int8 codes or fp16 values, the per-channel K and per-token V parameters (None for a
        16-bit side)."""
        n = self._check_layer(layer_id)
        vs, vz = self._v_scale[layer_id], self._v_zp[layer_id]
        return (self._k_cache[layer_id][:, :, :n], self._v_cache[layer_id][:, :, :n],
                self._k_scale[layer_id], self._k_zp[layer_id],
                None if vs is None else vs[:, :, :n], None if vz is None else vz[:, :, :n])

    def get_kv(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        """Dequantised K, V in self.dtype (kivi_style_cache.py:619-666,
        role_aware_allocator_cache.py:402-440): code x s + z in fp32, then cast."""
        kc, vc, ks, kz, vs, vz = self.get_kivi_tensors(layer_id)
        kb, vb = self._bits[layer_id]
        if kb == 16:
            k = kc.to(self.dtype)
        else:
            kq = _unpack(kc) if kb == 4 else kc
            k = (kq.float() * ks.unsqueeze(2) + kz.unsqueeze(2)).to(self.dtype)
        if vb == 16:
            v = vc.to(self.dtype)
        else:
            vq = _unpack(vc) if vb == 4 else vc
            v = (vq.float() * vs.unsqueeze(-1) + vz.unsqueeze(-1)).to(self.dtype)
        rlen = self._res_len[layer_id]
        if rlen > 0:  # the fp16 window after the quantized tokens, oldest first
            rk, rv = self._residual(layer_id)
            k = torch.cat([k, rk.to(self.dtype)], dim=2)
            v = torch.cat([v, rv.to(self.dtype)], dim=2)
        return k, v

    def _residual(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        """The fp16 window's valid tokens in arrival order [B, H, rlen, 128]."""
        rlen, st = self._res_len[layer_id], self._res_start[layer_id]
        rk, rv = self._res_k[layer_id], self._res_v[layer_id]
        if st:
            rk, rv = torch.roll(rk, -st, dims=2), torch.roll(rv, -st, dims=2)
        return rk[:, :, :rlen], rv[:, :, :rlen]

    def _step_for(self, layer_id: int, q_heads: int):
        """The layer's LayerStep over its whole buffers and its frozen K parameters."""
        kc, ks = self._k_cache[layer_id], self._k_scale[layer_id]
        key = (q_heads, kc.data_ptr(), None if ks is None else ks.data_ptr())
        st = self._steps[layer_id]
        if st is not None and st.key == key:
            return st
        from .kernels import LayerStep, kv_view_fp16, kv_view_kivi

        kb, vb = self._bits[layer_id]
        B, H = kc.shape[0], kc.shape[1]
        vc, vs, vz, kz = self._v_cache[layer_id], self._v_scale[layer_id], self._v_zp[layer_id], \
            self._k_zp[layer_id]
        kview = kv_view_fp16(kc) if kb == 16 else kv_view_kivi(kc, ks, kz, True)
        vview = kv_view_fp16(vc) if vb == 16 else kv_view_kivi(vc, vs, vz, False)
        st = LayerStep(_kivi_format(kb), kview, _kivi_format(vb), vview, B, q_heads, H, 32, kc.device,
                       keepalive=(kc, ks, kz, vc, vs, vz))
        st.key = key
        self._steps[layer_id] = st
        return st

    def _attend(self, layer_id: int, q16: Tensor, sm: float, tau: Optional[Tensor]) -> Tensor:
        st = self._step_for(layer_id, q16.shape[1])
        # the window's slots in ring order: attention does not depend on the token order
        st.set_residual(self._res_k[layer_id], self._res_v[layer_id], self._res_len[layer_id])
        return st.attend(q16, self._layer_seq_lens[layer_id], sm, tau)

    def _layer_tau(self, layer_id: int, q: Tensor) -> Optional[Tensor]:
        """The engine's inv_tau[layer] as fp16 on q's device (converted once per layer)."""
        if not (self.use_attn_temperature and self.inv_tau is not None):
            return None
        cache = self.__dict__.setdefault("_tau16", {})
        t = cache.get(layer_id)
        if t is None or t.device != q.device:
            t = self.inv_tau[layer_id].to(device=q.device, dtype=torch.float16).contiguous()
            cache[layer_id] = t
        return t

    def decode_attn(self, layer_id: int, q: Tensor, sm_scale: Optional[float] = None) -> Tensor:
        """Attention of q [B, Hq, 128] over layer_id's cache (the tiled kernel of the layer's
        (k_bits, v_bits) pair); with use_attn_temperature and inv_tau [L, Hq], q is scaled by
        inv_tau[layer] in fp16."""
        n = self._check_layer(layer_id)
        if q.ndim != 3 or q.shape[-1] != 128:
            raise ValueError(f"q must be [B, Hq, 128], got {tuple(q.shape)}")
        dt = q.dtype
        q16 = q if q.dtype == torch.float16 else q.to(torch.float16)
        if q16.stride(-1) != 1:
            q16 = q16.contiguous()
        sm = 1.0 / math.sqrt(128) if sm_scale is None else sm_scale
        out = self._attend(layer_id, q16, sm, self._layer_tau(layer_id, q))
        self.record_fused_decode(layer_id, "hip_fused")
        return out if dt == torch.float16 else out.to(dt)

    def append_decode_attn(self, layer_id: int, q: Tensor, k: Tensor, v: Tensor,
                           sm_scale: Optional[float] = None,
                           inv_tau: Optional[Tensor] = None) -> Tensor:
        """Decode step of one layer: ``append`` of the new token (k, v [B, H, 1, 128]) then
        the attention of q [B, Hq, 128] over the cache including it.  inv_tau (fp16 [Hq]) is
        applied as given, as in the symmetric engines; None applies none (``decode_attn``
        applies the engine's own).  After the prefill, without a residual window and without
        a K range check due at this step, both run in one HIP launch
        (kvq_append_decode_attn, the append's arithmetic in the decode kernel's writer wave);
        codes, parameters and output are the same bits as the two-launch path."""
        if k.ndim != 4 or k.shape[2] != 1:
            raise ValueError(f"append_decode_attn appends one token per step, got S={k.shape[2]}")
        if q.dtype != torch.float16 or q.stride(-1) != 1:
            q = q.to(torch.float16).contiguous()
        sm = 1.0 / math.sqrt(128) if sm_scale is None else sm_scale
        kb, _ = self._bits[layer_id] if 0 <= layer_id < self.num_layers else (16, 16)
        fused = (self.residual_length == 0 and self._k_cache[layer_id] is not None
                 and (kb == 16 or self._k_scale_initialized[layer_id])
                 and (kb == 16 or self._oor_check_interval <= 0))
        if not fused:
            self.append(layer_id, k, v)
            return self._attend(layer_id, q, sm, inv_tau)
        self._validate_kv(layer_id, k, v)
        B, H = k.shape[0], k.shape[1]
        old = self._layer_seq_lens[layer_id]
        self._ensure(layer_id, B, H, old + 1, k.device)
        ks = self._k_scale[layer_id]
        if kb != 16 and tuple(ks.shape) != (B, H, 128):
            raise ValueError(f"Inconsistent decode K scale/zp shape for layer {layer_id}: "
                             f"expected {(B, H, 128)}, got {tuple(ks.shape)}")
        pk, pv = self._fused_apps(layer_id, k, v, old)
        st = self._step_for(layer_id, q.shape[1])
        st.set_residual(None, None, 0)
        out = st.append_attend(q, old + 1, sm, inv_tau, pk, pv)
        self._layer_seq_lens[layer_id] = old + 1
        self._seq_len = max(self._layer_seq_lens)
        return out

    def _fused_apps(self, layer_id: int, k: Tensor, v: Tensor, pos: int):
        """The fused decode step's kvq_append_params of K and V (one token), kept per layer
        buffers; per call the rows and the slot change.  A quantized side is set up as
        ``append`` sets it up; a 16-bit side is an FP16 append (the row stored as it comes)."""
        kb, vb = self._bits[layer_id]
        kc, vc = self._k_cache[layer_id], self._v_cache[layer_id]
        ks, kz = self._k_scale[layer_id], self._k_zp[layer_id]
        key = (kc.data_ptr(), None if ks is None else ks.data_ptr(), tuple(k.shape[:2]))
        ent = self._apps[layer_id]
        if ent is None or ent[2] != key:
            pk, pv = C.AppendParams(), C.AppendParams()
            for p, x, bits, buf in ((pk, k, kb, kc), (pv, v, vb, vc)):
                _fill_append(p, _kivi_format(bits), x, 32, buf, pos, None)
                if bits == 16:  # byte strides of the fp16 rows
                    p.codes_stride_b, p.codes_stride_h, p.codes_stride_t = (2 * t for t in buf.stride()[:3])
            if kb != 16:
                pk.static_scale, pk.static_zp = ks.data_ptr(), kz.data_ptr()
                pk.static_scale_dtype = C.KVQ_DTYPE_F32
                pk.static_stride_b, pk.static_stride_h, pk.static_stride_g = ks.stride()
            if vb != 16:
                vs, vz = self._v_scale[layer_id], self._v_zp[layer_id]
                pv.scale_out, pv.zp_out, pv.scale_out_dtype = vs.data_ptr(), vz.data_ptr(), C.KVQ_DTYPE_F32
                pv.so_stride_b, pv.so_stride_h, pv.so_stride_t = vs.stride()
                pv.dyn_quantile_lo, pv.dyn_quantile = _kivi_levels(self.v_percentile)
            ent = (pk, pv, key)
            self._apps[layer_id] = ent
        pk, pv = ent[0], ent[1]
        for p, x in ((pk, k), (pv, v)):
            if x.stride(-1) != 1:
                x = x.contiguous()
            p.x = x.data_ptr()
            p.x_stride_b, p.x_stride_h, p.x_stride_s = x.stride()[:3]
            p.write_pos = pos
            p._keep = (x,)
        return pk, pv

    def clear(self) -> None:
        self._discard_step_status()
        self._layer_seq_lens = [0] * self.num_layers
        self._seq_len = 0
        self._steps = [None] * self.num_layers
        self._k_scale_initialized = [False] * self.num_layers
        self._k_scale = [None] * self.num_layers
        self._k_zp = [None] * self.num_layers
        self._res_len = [0] * self.num_layers
        self._res_start = [0] * self.num_layers
        for t in self._res_k + self._res_v:
            if t is not None:
                t.zero_()

    def release(self) -> None:
        n = self.num_layers
        self._k_cache, self._v_cache = [None] * n, [None] * n
        self._v_scale, self._v_zp = [None] * n, [None] * n
        self._steps, self._apps = [None] * n, [None] * n
        self._res_k, self._res_v = [None] * n, [None] * n
        self._layer_capacity = [0] * n
        self.clear()

    def get_memory_mb(self) -> float:
        total = 0
        for lst in (self._k_cache, self._v_cache, self._k_scale, self._k_zp, self._v_scale, self._v_zp):
            total += sum(t.numel() * t.element_size() for t in lst if t is not None)
        return total / (1024 * 1024)

    def to_tuple(self) -> Tuple[Tuple[Tensor, Tensor], ...]:
        """Every layer's dequantised (k, v) (role_aware_allocator_cache.py:477-483)."""
        out = []
        for i in range(self.num_layers):
            if self._layer_seq_lens[i] <= 0:
                raise ValueError(f"Layer {i} cache is empty")
            out.append(self.get_kv(i))
        return tuple(out)


class KIVIStyleKVCache(_KiviFamily):
    """KIVI-style cache (src/cache/kivi_style_cache.py:38-900): every layer quantized with
    quant_bits (4: packed nibbles, 8: int8 codes), K per channel with parameters frozen at
    prefill, V per token, both with optional percentile clipping (k_percentile,
    v_percentile).  See _KiviFamily for the storage and kernels."""

    def __init__(self, num_layers: int, device: str = "cuda", dtype: torch.dtype = torch.float16,
                 max_seq_len: Optional[int] = None, quant_bits: int = 8,
                 k_percentile: float = 100.0, v_percentile: float = 100.0,
                 inv_tau: Optional[Tensor] = None, use_attn_temperature: bool = False,
                 residual_length: int = 0, decode_attn_impl: str = "hip_fused",
                 check_numerics: bool = True):
        if num_layers <= 0:
            raise ValueError(f"num_layers must be > 0, got {num_layers}")
        if quant_bits not in (4, 8):
            raise ValueError(f"quant_bits must be 4 or 8, got {quant_bits}")
        self._init_kivi(num_layers, device, dtype, max_seq_len, [(quant_bits, quant_bits)] * num_layers,
                        k_percentile, v_percentile, inv_tau, use_attn_temperature, residual_length,
                        decode_attn_impl, check_numerics)
        self.quant_bits = int(quant_bits)
        self.bit_packed = self.quant_bits == 4

    def get_int4_asym_tensors(self, layer_id: int):
        """(k_packed, v_packed, k_scale, k_zp, v_scale, v_zp) over the stored tokens, the
        reference's kernel arguments (kivi_style_cache.py:668-700); quant_bits=4 only."""
        if not self.bit_packed:
            raise RuntimeError("get_int4_asym_tensors requires bit_packed=True (quant_bits=4)")
        return self.get_kivi_tensors(layer_id)


class RoleAwareAsymKVCache(KIVIStyleKVCache):
    """RoleAlign's cache (src/cache/role_aware_asym_cache.py:27-76): the KIVI layout with
    calibrated k / v percentiles and inv_tau, tagged with its framework."""

    def __init__(self, num_layers: int, device: str = "cuda", dtype: torch.dtype = torch.float16,
                 max_seq_len: Optional[int] = None, quant_bits: int = 4,
                 k_percentile: float = 100.0, v_percentile: float = 100.0,
                 inv_tau: Optional[Tensor] = None, use_attn_temperature: bool = False,
                 framework: str = "ours_asym", residual_length: int = 0,
                 decode_attn_impl: str = "hip_fused", check_numerics: bool = True):
        super().__init__(num_layers=num_layers, device=device, dtype=dtype, max_seq_len=max_seq_len,
                         quant_bits=quant_bits, k_percentile=k_percentile, v_percentile=v_percentile,
                         inv_tau=inv_tau, use_attn_temperature=use_attn_temperature,
                         residual_length=residual_length, decode_attn_impl=decode_attn_impl,
                         check_numerics=check_numerics)
        self.framework = framework
        self.ba_calibrated = (k_percentile != 100.0) or (v_percentile != 100.0)


def load_per_layer_bits_from_policy(policy_json, *, project_root) -> List[Tuple[int, int]]:
    """Per-layer (k_bits, v_bits) pairs of an allocator policy JSON
    (src/cache/role_aware_allocator_cache.py:36-70): a relative path resolves against
    project_root; the file must hold ``per_layer_bits``, each a pair from {4, 8, 16}."""
    import json
    from pathlib import Path

    path = Path(policy_json)
    if not path.is_absolute():
        path = Path(project_root) / path
    if not path.exists():
        raise FileNotFoundError(f"policy_json={str(policy_json)!r} not found (resolved to {str(path)!r}).")
    with path.open("r", encoding="utf-8") as fh:
        payload = json.load(fh)
    raw = payload.get("per_layer_bits")
    if raw is None:
        raise ValueError(f"policy_json {str(path)!r} missing required key 'per_layer_bits'")
    pairs = []
    for idx, entry in enumerate(raw):
        if not isinstance(entry, (list, tuple)) or len(entry) != 2:
            raise ValueError(f"per_layer_bits[{idx}] must be a 2-tuple/list (k_bits, v_bits), got {entry!r}")
        kb, vb = int(entry[0]), int(entry[1])
        if kb not in _KIVI_BITS or vb not in _KIVI_BITS:
            raise ValueError(f"per_layer_bits[{idx}]=({kb},{vb}) contains unsupported bits; allowed "
                             f"values: {sorted(_KIVI_BITS)}")
        pairs.append((kb, vb))
    return pairs


class RoleAwareAllocatorKVCache(_KiviFamily):
    """The allocator's RoleAlign cache (src/cache/role_aware_allocator_cache.py:73-502): the
    KIVI family with a (k_bits, v_bits) pair from {4, 8, 16} per layer.  See _KiviFamily."""

    def __init__(self, num_layers: int, *, per_layer_bits: List[Tuple[int, int]],
                 device: str = "cuda", dtype: torch.dtype = torch.float16,
                 max_seq_len: Optional[int] = None, k_percentile: float = 100.0,
                 v_percentile: float = 100.0, inv_tau: Optional[Tensor] = None,
                 use_attn_temperature: bool = False, framework: str = "ours_asym_allocator",
                 residual_length: int = 0, decode_attn_impl: str = "torch_ref",
                 check_numerics: bool = True):
        if num_layers <= 0:
            raise ValueError(f"num_layers must be > 0, got {num_layers}")
        if len(per_layer_bits) != num_layers:
            raise ValueError(f"per_layer_bits length {len(per_layer_bits)} must equal num_layers {num_layers}")
        norm = []
        for idx, entry in enumerate(per_layer_bits):
            if not isinstance(entry, (tuple, list)) or len(entry) != 2:
                raise ValueError(f"per_layer_bits[{idx}] must be a 2-tuple/list (k_bits, v_bits), got {entry!r}")
            kb, vb = int(entry[0]), int(entry[1])
            if kb not in _KIVI_BITS or vb not in _KIVI_BITS:
                raise ValueError(f"per_layer_bits[{idx}]=({kb},{vb}) contains unsupported bits; allowed "
                                 f"values: {sorted(_KIVI_BITS)}")
            norm.append((kb, vb))
        if int(residual_length) != 0:
            raise ValueError("RoleAwareAllocatorKVCache currently requires residual_length=0")
        self._init_kivi(num_layers, device, dtype, max_seq_len, norm, k_percentile, v_percentile,
                        inv_tau, use_attn_temperature, 0, decode_attn_impl, check_numerics)
        self.framework = framework
        self.ba_calibrated = (self.k_percentile != 100.0) or (self.v_percentile != 100.0)
        self._per_layer_bits = norm


_MIXED_BITS = {4, 8, 16}


class MixedKVCache(_EngineBase):
    """The reference's K/V mixed-precision cache (src/cache/mixed_kv_cache.py:35-330).  Per
    layer a (k_bits, v_bits) pair (per_layer_bits, or k_bits / v_bits for every layer):

    * K 8: INT8 symmetric per (token, group of k_group_size) with a dynamic percentile-clipped
      scale (src/quant/int8_basic.py:18-108): codes int8 [B, H, cap, 128], fp16 scales
      [B, H, cap, Gk] (the reference keeps the same fp16-valued scales as fp32);
    * K 4: INT4 asymmetric per token (src/quant/asymmetric_quant.py:246-270,
      k_clip_percentile clipping; src/cache/mixed_kv_cache.py:159-162): packed nibbles
      [B, H, cap, 64], fp32 scale / zero-point [B, H, cap] (rows padded to 4 tokens);
    * V 4: INT4 asymmetric per token (v_percentile clipping): packed nibbles [B, H, cap, 64]
      (byte = ((c[2i]+8) << 4) | (c[2i+1]+8); the reference keeps one code per byte), fp32
      scale / zero-point [B, H, cap];
    * V 8: as K 8 with v_group_size and v_percentile;
    * 16 (either side): fp16 values as they come.

    The buffers are preallocated and grow by doubling (the reference concatenates per
    append).  The quantized sides of an append are one kvq_quant_append launch; decode
    attention reads the cache in place through the tiled kernel of the layer's pair, every
    (k_bits, v_bits) pair of {4, 8, 16} (the decode call carries V's group size apart from
    K's, kvq_decode_params.v_group_size).
    """

    _min_capacity = 256
    _BUILT = {(kb, vb) for kb in (4, 8, 16) for vb in (4, 8, 16)}

    def __init__(self, num_layers: int, device: str = "cuda", dtype: torch.dtype = torch.float16,
                 max_seq_len: Optional[int] = None, k_group_size: int = 128,
                 v_group_size: Optional[int] = None, k_clip_percentile: float = 99.9,
                 v_percentile: float = 100.0, k_bits: int = 8, v_bits: int = 4,
                 per_layer_bits: Optional[List[Tuple[int, int]]] = None,
                 decode_attn_impl: str = "torch_ref", check_numerics: bool = True):
        if num_layers <= 0:
            raise ValueError(f"num_layers must be > 0, got {num_layers}")
        if k_bits not in _MIXED_BITS:
            raise ValueError(f"k_bits must be one of {_MIXED_BITS}, got {k_bits}")
        if v_bits not in _MIXED_BITS:
            raise ValueError(f"v_bits must be one of {_MIXED_BITS}, got {v_bits}")
        if per_layer_bits is not None:
            if len(per_layer_bits) != num_layers:
                raise ValueError(f"per_layer_bits length {len(per_layer_bits)} must equal "
                                 f"num_layers {num_layers}")
            for i, entry in enumerate(per_layer_bits):
                if not isinstance(entry, (tuple, list)) or len(entry) != 2:
                    raise ValueError(f"per_layer_bits[{i}] must be a 2-tuple (k_bits, v_bits), "
                                     f"got {entry!r}")
                if entry[0] not in _MIXED_BITS or entry[1] not in _MIXED_BITS:
                    raise ValueError(f"per_layer_bits[{i}]=({entry[0]},{entry[1]}) contains "
                                     f"unsupported bits; allowed values: {_MIXED_BITS}")
            per_layer_bits = [(int(a), int(b)) for a, b in per_layer_bits]
        v_group_size = v_group_size if v_group_size is not None else k_group_size
        bits = per_layer_bits or [(int(k_bits), int(v_bits))] * num_layers
        for kb, vb in bits:
            if (kb, vb) not in self._BUILT:
                raise NotImplementedError(f"MixedKVCache: the ({kb}, {vb}) layer is not built (built: "
                                          f"{sorted(self._BUILT)})")
        for gs in (k_group_size, v_group_size):
            if gs not in (16, 32, 64, 128):
                raise NotImplementedError(f"group sizes must be 16, 32, 64 or 128, got {gs}")
        _dyn_quantile(k_clip_percentile)  # (0, 100]
        if any(kb == 4 for kb, _ in bits):
            _kivi_levels(k_clip_percentile)
        if any(vb == 4 for _, vb in bits):
            _kivi_levels(v_percentile)
        elif any(vb == 8 for _, vb in bits):
            _dyn_quantile(v_percentile)
        self._init_common(num_layers, device, max_seq_len, decode_attn_impl, check_numerics)
        self.dtype = dtype
        self.k_group_size = int(k_group_size)
        self.v_group_size = int(v_group_size)
        self.k_clip_percentile = float(k_clip_percentile)
        self.v_percentile = float(v_percentile)
        self.k_bits, self.v_bits = int(k_bits), int(v_bits)
        self._per_layer_bits = per_layer_bits
        self._bits = bits
        self.inv_tau = None
        self.use_attn_temperature = False
        n = num_layers
        self._k_cache: List[Optional[Tensor]] = [None] * n
        self._k_scale: List[Optional[Tensor]] = [None] * n
        self._k_zp: List[Optional[Tensor]] = [None] * n
        self._v_cache: List[Optional[Tensor]] = [None] * n
        self._v_scale: List[Optional[Tensor]] = [None] * n
        self._v_zp: List[Optional[Tensor]] = [None] * n

    def _resolve_bits(self, layer_id: int) -> Tuple[int, int]:
        """(k_bits, v_bits) of a layer (mixed_kv_cache.py:138-147)."""
        if self._per_layer_bits is not None:
            return self._per_layer_bits[layer_id]
        return self.k_bits, self.v_bits

    def _ensure(self, layer_id: int, B: int, H: int, target: int, device) -> None:
        kc = self._k_cache[layer_id]
        if kc is not None and (kc.shape[0] != B or kc.shape[1] != H):
            raise ValueError(f"Inconsistent KV shape for layer {layer_id}: existing "
                             f"K={tuple(kc.shape)}, incoming=({B}, {H}, *, 128)")
        cap = self._layer_capacity[layer_id]
        if kc is not None and target <= cap:
            return
        kb, vb = self._bits[layer_id]
        new_cap = self._new_capacity(layer_id, target, cap if kc is not None else 0)
        old = self._layer_seq_lens[layer_id]
        # per-token K parameters: rows of a multiple of 4 tokens (the kernel reads 4 tokens'
        # parameters as one 16-byte vector)
        kpitch = (new_cap + 3) // 4 * 4
        new = {
            "k": (torch.empty(B, H, new_cap, 64, dtype=torch.int8, device=device) if kb == 4 else
                  torch.empty(B, H, new_cap, 128, dtype=torch.int8 if kb == 8 else torch.float16,
                              device=device)),
            "ks": (torch.empty(B, H, new_cap, 128 // self.k_group_size, dtype=torch.float16, device=device)
                   if kb == 8 else
                   torch.empty(B, H, kpitch, dtype=torch.float32, device=device)[:, :, :new_cap]
                   if kb == 4 else None),
            "kz": (torch.empty(B, H, kpitch, dtype=torch.float32, device=device)[:, :, :new_cap]
                   if kb == 4 else None),
            "v": torch.empty(B, H, new_cap, 64 if vb == 4 else 128,
                             dtype=torch.float16 if vb == 16 else torch.int8, device=device),
            "vs": (torch.empty(B, H, new_cap, dtype=torch.float32, device=device) if vb == 4 else
                   torch.empty(B, H, new_cap, 128 // self.v_group_size, dtype=torch.float16, device=device)
                   if vb == 8 else None),
            "vz": torch.empty(B, H, new_cap, dtype=torch.float32, device=device) if vb == 4 else None,
        }
        olds = {"k": kc, "ks": self._k_scale[layer_id], "kz": self._k_zp[layer_id],
                "v": self._v_cache[layer_id], "vs": self._v_scale[layer_id], "vz": self._v_zp[layer_id]}
        if kc is not None and old > 0:
            for key, t in new.items():
                if t is not None:
                    t[:, :, :old] = olds[key][:, :, :old]
        self._k_cache[layer_id], self._k_scale[layer_id] = new["k"], new["ks"]
        self._k_zp[layer_id] = new["kz"]
        self._v_cache[layer_id], self._v_scale[layer_id], self._v_zp[layer_id] = new["v"], new["vs"], new["vz"]
        self._layer_capacity[layer_id] = new_cap
        self._steps[layer_id] = self._apps[layer_id] = None

    def _params(self, layer_id: int, k: Tensor, v: Tensor, pos: int, status,
                fp16: bool = False) -> Tuple:
        """kvq_append_params of the quantized sides (K INT8 dynamic, V INT4_KIVI per token or
        INT8 dynamic) writing at slot pos; a 16-bit side gets None, or with fp16 an FP16
        append (the row stored as it comes, for the fused decode step).  The one-token blocks
        of a decode step are kept per layer."""
        S = k.shape[2]
        kb, vb = self._bits[layer_id]
        ents = self._apps[layer_id] if S == 1 else None
        ent = None if ents is None else ents.get(fp16)
        if ent is None:
            pk = pv = None
            if fp16:
                for side, bits, buf in (("k", kb, self._k_cache[layer_id]), ("v", vb, self._v_cache[layer_id])):
                    if bits == 16:
                        pf = C.AppendParams()
                        _fill_append(pf, C.KVQ_FMT_FP16, k if side == "k" else v, 32, buf, pos, None)
                        pf.codes_stride_b, pf.codes_stride_h, pf.codes_stride_t = (2 * t for t in buf.stride()[:3])
                        pf._fp16 = True
                        if side == "k":
                            pk = pf
                        else:
                            pv = pf
            if kb == 8:
                pk = C.AppendParams()
                ks = self._k_scale[layer_id]
                _fill_append(pk, C.KVQ_FMT_INT8_SYM, k, self.k_group_size, self._k_cache[layer_id], pos, None)
                pk.dyn_quantile = _dyn_quantile(self.k_clip_percentile)
                pk.scale_out, pk.scale_out_dtype = ks.data_ptr(), C.KVQ_DTYPE_F16
                pk.so_stride_b, pk.so_stride_h, pk.so_stride_t, pk.so_stride_g = ks.stride()
            elif kb == 4:  # per-token asymmetric, the same arithmetic as a 4-bit V
                pk = C.AppendParams()
                ks, kz = self._k_scale[layer_id], self._k_zp[layer_id]
                _fill_append(pk, C.KVQ_FMT_INT4_KIVI, k, 32, self._k_cache[layer_id], pos, None)
                pk.scale_out, pk.zp_out, pk.scale_out_dtype = ks.data_ptr(), kz.data_ptr(), C.KVQ_DTYPE_F32
                pk.so_stride_b, pk.so_stride_h, pk.so_stride_t = ks.stride()
                pk.dyn_quantile_lo, pk.dyn_quantile = _kivi_levels(self.k_clip_percentile)
            if vb == 4:
                pv = C.AppendParams()
                vc, vs, vz = self._v_cache[layer_id], self._v_scale[layer_id], self._v_zp[layer_id]
                _fill_append(pv, C.KVQ_FMT_INT4_KIVI, v, 32, vc, pos, None)
                pv.scale_out, pv.zp_out, pv.scale_out_dtype = vs.data_ptr(), vz.data_ptr(), C.KVQ_DTYPE_F32
                pv.so_stride_b, pv.so_stride_h, pv.so_stride_t = vs.stride()
                pv.dyn_quantile_lo, pv.dyn_quantile = _kivi_levels(self.v_percentile)
            elif vb == 8:
                pv = C.AppendParams()
                vs = self._v_scale[layer_id]
                _fill_append(pv, C.KVQ_FMT_INT8_SYM, v, self.v_group_size, self._v_cache[layer_id], pos, None)
                pv.dyn_quantile = _dyn_quantile(self.v_percentile)
                pv.scale_out, pv.scale_out_dtype = vs.data_ptr(), C.KVQ_DTYPE_F16
                pv.so_stride_b, pv.so_stride_h, pv.so_stride_t, pv.so_stride_g = vs.stride()
            ent = (pk, pv)
            if S == 1:
                self._apps[layer_id] = {**(ents or {}), fp16: ent}
        pk, pv = ent
        # status: the status words (a tensor), or the address of a decode-step status row
        sptr = status if status is None or isinstance(status, int) else status.data_ptr()
        for p, x, off in ((pk, k, 0), (pv, v, 8)):
            if p is None:
                continue
            p.x = x.data_ptr()
            p.x_stride_b, p.x_stride_h, p.x_stride_s = x.stride()[:3]
            p.seq_new = S
            p.write_pos = pos
            # a 16-bit side is stored as it comes, unchecked (as the two-launch path's copy)
            p.status = None if sptr is None or getattr(p, "_fp16", False) else sptr + off
            p._keep = (x,)
        return pk, pv

    def _append(self, layer_id: int, k: Tensor, v: Tensor) -> int:
        """Quantizes k, v [B, H, S, 128] into the layer at its length; returns the new length."""
        self._validate_kv(layer_id, k, v)
        B, H, S, D = k.shape
        old = self._layer_seq_lens[layer_id]
        if S == 0:
            return old
        if k.stride(-1) != 1:
            k = k.contiguous()
        if v.stride(-1) != 1:
            v = v.contiguous()
        kb, vb = self._bits[layer_id]
        self._ensure(layer_id, B, H, old + S, k.device)
        if kb == 16:
            self._k_cache[layer_id][:, :, old:old + S] = k
        if vb == 16:
            self._v_cache[layer_id][:, :, old:old + S] = v
        if kb != 16 or vb != 16:
            status = self._status_buf(k.device) if self.check_numerics else None
            pk, pv = self._params(layer_id, k, v, old, status)
            C.check(C.lib().kvq_quant_append(None if pk is None else ctypes.byref(pk),
                                             None if pv is None else ctypes.byref(pv),
                                             ctypes.c_void_p(C.stream_handle(k.device))))
            if status is not None:
                st = self._read_status()
                if st[0] & 1 or st[2] & 1:
                    raise ValueError(f"MixedKVCache append: {'K' if st[0] & 1 else 'V'} input contains "
                                     "NaN or Inf — refusing to quantize corrupt data")
        n = old + S
        self._layer_seq_lens[layer_id] = n
        self._seq_len = max(self._layer_seq_lens)
        return n

    def append(self, layer_id: int, k: Tensor, v: Tensor) -> None:
        """Quantize and append k, v fp16 [B, H, S, 128] (mixed_kv_cache.py:191-240)."""
        self._append(layer_id, k, v)

    def _check_layer(self, layer_id: int) -> int:
        if layer_id < 0 or layer_id >= self.num_layers:
            raise ValueError(f"layer_id {layer_id} out of range [0, {self.num_layers})")
        if self._k_cache[layer_id] is None:
            raise ValueError(f"Cache for layer {layer_id} is empty")
        return self._layer_seq_lens[layer_id]

    def get_mixed_tensors(self, layer_id: int):
        """(k_store, k_scale, v_store, v_scale, v_zp) over the stored tokens: K int8 codes
        (fp16 group scales), packed 4-bit codes (fp32 per-token scales; the zero-points are
        ``get_k_zero_points``) or fp16 values, V packed / int8 codes or fp16 values; None
        where a side has no such parameter."""
        n = self._check_layer(layer_id)

        def sl(t):
            return None if t is None else t[:, :, :n]

        return (sl(self._k_cache[layer_id]), sl(self._k_scale[layer_id]), sl(self._v_cache[layer_id]),
                sl(self._v_scale[layer_id]), sl(self._v_zp[layer_id]))

    def get_k_zero_points(self, layer_id: int) -> Optional[Tensor]:
        """fp32 [B, H, S] per-token zero-points of a 4-bit K layer (None otherwise)."""
        n = self._check_layer(layer_id)
        kz = self._k_zp[layer_id]
        return None if kz is None else kz[:, :, :n]

    def get_kv(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        """Dequantised K, V in self.dtype (mixed_kv_cache.py:170-190, 242-254): a symmetric
        side is code x the scale of its group, an asymmetric side code x s + z of its token,
        in fp32, then cast."""
        kc, ks, vc, vs, vz = self.get_mixed_tensors(layer_id)
        kb, vb = self._bits[layer_id]
        if kb == 16:
            k = kc.to(self.dtype)
        elif kb == 8:
            k = _deq_sym(kc, ks.float()).to(self.dtype)
        else:
            kz = self.get_k_zero_points(layer_id)
            k = (_unpack(kc).float() * ks.unsqueeze(-1) + kz.unsqueeze(-1)).to(self.dtype)
        if vb == 16:
            v = vc.to(self.dtype)
        elif vb == 8:
            v = _deq_sym(vc, vs.float()).to(self.dtype)
        else:
            v = (_unpack(vc).float() * vs.unsqueeze(-1) + vz.unsqueeze(-1)).to(self.dtype)
        return k, v

    def _step_for(self, layer_id: int, q_heads: int):
        kc = self._k_cache[layer_id]
        st = self._steps[layer_id]
        if st is not None and st.key == (q_heads, kc.data_ptr()):
            return st
        from .kernels import LayerStep, kv_view_fp16, kv_view_kivi, kv_view_tok

        kb, vb = self._bits[layer_id]
        B, H = kc.shape[0], kc.shape[1]
        ks, vc, vs, vz = self._k_scale[layer_id], self._v_cache[layer_id], self._v_scale[layer_id], \
            self._v_zp[layer_id]
        kz = self._k_zp[layer_id]
        if kb == 8:
            kf, kview = C.KVQ_FMT_INT8_SYM, kv_view_tok(kc, ks)
        elif kb == 4:  # per-token parameters, the layout of a 4-bit V
            kf, kview = C.KVQ_FMT_INT4_KIVI, kv_view_kivi(kc, ks, kz, False)
        else:
            kf, kview = C.KVQ_FMT_FP16, kv_view_fp16(kc)
        if vb == 4:
            vf, vview = C.KVQ_FMT_INT4_KIVI, kv_view_kivi(vc, vs, vz, False)
        elif vb == 8:
            vf, vview = C.KVQ_FMT_INT8_SYM, kv_view_tok(vc, vs)
        else:
            vf, vview = C.KVQ_FMT_FP16, kv_view_fp16(vc)
        # one group size per decode call for K; V's goes apart when both sides have groups
        gs = self.k_group_size if kb == 8 else self.v_group_size if vb == 8 else 32
        st = LayerStep(kf, kview, vf, vview, B, q_heads, H, gs, kc.device,
                       keepalive=(kc, ks, kz, vc, vs, vz))
        if kb == 8 and vb == 8 and self.v_group_size != self.k_group_size:
            st.params.v_group_size = self.v_group_size
        st.key = (q_heads, kc.data_ptr())
        self._steps[layer_id] = st
        return st

    def decode_attn(self, layer_id: int, q: Tensor, sm_scale: Optional[float] = None,
                    inv_tau: Optional[Tensor] = None) -> Tensor:
        """Attention of q [B, Hq, 128] over the layer's cache, read in place (one HIP launch);
        inv_tau (fp16 [Hq]) scales q in fp16 first."""
        n = self._check_layer(layer_id)
        if q.ndim != 3 or q.shape[-1] != 128:
            raise ValueError(f"q must be [B, Hq, 128], got {tuple(q.shape)}")
        dt = q.dtype
        q16 = q if q.dtype == torch.float16 and q.stride(-1) == 1 else q.to(torch.float16).contiguous()
        sm = 1.0 / math.sqrt(128) if sm_scale is None else sm_scale
        out = self._step_for(layer_id, q.shape[1]).attend(q16, n, sm, inv_tau)
        return out if dt == torch.float16 else out.to(dt)

    def append_decode_attn(self, layer_id: int, q: Tensor, k: Tensor, v: Tensor,
                           sm_scale: Optional[float] = None,
                           inv_tau: Optional[Tensor] = None) -> Tensor:
        """Decode step of one layer: the new token (k, v [B, H, 1, 128]) appended, then the
        attention of q [B, Hq, 128] over the cache including it, in one HIP launch
        (kvq_append_decode_attn: the append's arithmetic in the decode kernel's writer wave,
        the same bits as ``append`` then ``decode_attn``).  With check_numerics, NaN / Inf in
        a quantized side raise ValueError afterwards and the cache does not advance."""
        if k.ndim != 4 or k.shape[2] != 1:
            raise ValueError(f"append_decode_attn appends one token per step, got {tuple(k.shape)}")
        if q.dtype != torch.float16 or q.stride(-1) != 1:
            q = q.to(torch.float16).contiguous()
        sm = 1.0 / math.sqrt(128) if sm_scale is None else sm_scale
        self._validate_kv(layer_id, k, v)
        B, H = k.shape[0], k.shape[1]
        if k.stride(-1) != 1:
            k = k.contiguous()
        if v.stride(-1) != 1:
            v = v.contiguous()
        old = self._layer_seq_lens[layer_id]
        self._ensure(layer_id, B, H, old + 1, k.device)
        status = self._step_status_ptr(layer_id, k.device) if self.check_numerics else None
        pk, pv = self._params(layer_id, k, v, old, status, fp16=True)
        out = self._step_for(layer_id, q.shape[1]).append_attend(q, old + 1, sm, inv_tau, pk, pv)
        self._layer_seq_lens[layer_id] = old + 1
        self._seq_len = max(self._layer_seq_lens)
        if status is not None:
            self._defer_status(layer_id, k.numel(), "MixedKVCache", "", clip_warn=False)
        return out

    def clear(self) -> None:
        self._discard_step_status()
        self._layer_seq_lens = [0] * self.num_layers
        self._seq_len = 0

    def release(self) -> None:
        n = self.num_layers
        self._k_cache, self._k_scale, self._k_zp = [None] * n, [None] * n, [None] * n
        self._v_cache, self._v_scale, self._v_zp = [None] * n, [None] * n, [None] * n
        self._steps, self._apps = [None] * n, [None] * n
        self._layer_capacity = [0] * n
        self.clear()

    def get_memory_mb(self) -> float:
        total = 0
        for lst in (self._k_cache, self._k_scale, self._k_zp, self._v_cache, self._v_scale, self._v_zp):
            total += sum(t.numel() * t.element_size() for t in lst if t is not None)
        return total / (1024 * 1024)

    def to_tuple(self) -> Tuple[Tuple[Tensor, Tensor], ...]:
        """Every layer's dequantised (k, v) (mixed_kv_cache.py:311-330)."""
        out = []
        for i in range(self.num_layers):
            if self._k_cache[i] is None:
                raise ValueError(f"Layer {i} cache is empty")
            out.append(self.get_kv(i))
        return tuple(out)

    @classmethod
    def from_tuple(cls, past_key_values, device: str = "cuda", **kwargs) -> "MixedKVCache":
        cache = cls(num_layers=len(past_key_values), device=device, **kwargs)
        for i, (k, v) in enumerate(past_key_values):
            cache.append(i, k.to(device), v.to(device))
        return cache

    def __repr__(self) -> str:
        return (f"MixedKVCache(num_layers={self.num_layers}, k_bits={self.k_bits}, "
                f"v_bits={self.v_bits}, seq_len={self._seq_len}, memory={self.get_memory_mb():.2f}MB)")


class FP16KVCache:
    """The fp16 mode's cache (src/cache/fp16_cache.py:26-366): K / V kept as they come,
    [B, H, capacity, D] per layer, capacity doubling with a copy, ``get_kv`` returning views
    of the stored tokens.  Plain storage: nothing is quantized, so no kernel runs here."""

    _min_capacity = 256

    def __init__(self, num_layers: int, device: str = "cuda", dtype: torch.dtype = torch.float16,
                 max_seq_len: Optional[int] = None):
        if num_layers <= 0:
            raise ValueError(f"num_layers must be > 0, got {num_layers}")
        self.num_layers = num_layers
        self.device = device
        self.dtype = dtype
        self.max_seq_len = int(max_seq_len) if max_seq_len is not None else None
        if self.max_seq_len is not None and self.max_seq_len <= 0:
            raise ValueError(f"max_seq_len must be > 0, got {self.max_seq_len}")
        self._k_cache: List[Optional[Tensor]] = [None] * num_layers
        self._v_cache: List[Optional[Tensor]] = [None] * num_layers
        self._layer_seq_lens: List[int] = [0] * num_layers
        self._layer_capacity: List[int] = [0] * num_layers
        self._seq_len = 0

    def _grow(self, layer_id: int, batch: int, heads: int, head_dim: int, target: int) -> None:
        if self.max_seq_len is not None and target > self.max_seq_len:
            raise ValueError(f"target_len {target} exceeds max_seq_len {self.max_seq_len} for layer {layer_id}")
        kb, cap = self._k_cache[layer_id], self._layer_capacity[layer_id]
        if kb is not None:
            if kb.shape[0] != batch or kb.shape[1] != heads or kb.shape[3] != head_dim:
                raise ValueError(f"Inconsistent KV shape for layer {layer_id}: existing={tuple(kb.shape)}, "
                                 f"incoming=({batch}, {heads}, *, {head_dim})")
            if target <= cap:
                return
        new_cap = max(target, self._min_capacity) if kb is None else max(target, cap * 2)
        if self.max_seq_len is not None:
            new_cap = min(new_cap, self.max_seq_len)
            if new_cap < target:
                raise ValueError(f"target_len {target} exceeds capped capacity {new_cap} for layer {layer_id}")
        nk = torch.empty((batch, heads, new_cap, head_dim), device=self.device, dtype=self.dtype)
        nv = torch.empty_like(nk)
        old = self._layer_seq_lens[layer_id]
        if kb is not None and old:
            nk[:, :, :old] = kb[:, :, :old]
            nv[:, :, :old] = self._v_cache[layer_id][:, :, :old]
        self._k_cache[layer_id], self._v_cache[layer_id] = nk, nv
        self._layer_capacity[layer_id] = new_cap

    def append(self, layer_id: int, k: Tensor, v: Tensor) -> None:
        if layer_id < 0 or layer_id >= self.num_layers:
            raise ValueError(f"layer_id {layer_id} out of range [0, {self.num_layers})")
        if k.shape != v.shape:
            raise ValueError(f"K and V shapes must match. Got K: {k.shape}, V: {v.shape}")
        if k.dim() != 4:
            raise ValueError(f"K/V must be 4D [batch, heads, seq, dim]. Got {k.dim()}D")
        k = k.to(device=self.device, dtype=self.dtype)
        v = v.to(device=self.device, dtype=self.dtype)
        B, H, S, D = k.shape
        old = self._layer_seq_lens[layer_id]
        self._grow(layer_id, B, H, D, old + S)
        self._k_cache[layer_id][:, :, old:old + S] = k
        self._v_cache[layer_id][:, :, old:old + S] = v
        self._layer_seq_lens[layer_id] = old + S
        if layer_id == 0:
            self._seq_len = old + S

    def get_kv(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        if layer_id < 0 or layer_id >= self.num_layers:
            raise ValueError(f"layer_id {layer_id} out of range [0, {self.num_layers})")
        if self._k_cache[layer_id] is None:
            raise ValueError(f"Cache for layer {layer_id} is empty. Call append() first.")
        n = self._layer_seq_lens[layer_id]
        if n == 0:
            logger.warning("get_kv(layer_id=%d) returning zero-length tensors. The cache was cleared "
                           "but buffers are still allocated.", layer_id)
        return self._k_cache[layer_id][:, :, :n], self._v_cache[layer_id][:, :, :n]

    def get_seq_len(self) -> int:
        return self._seq_len

    def clear(self) -> None:
        self._layer_seq_lens = [0] * self.num_layers
        self._seq_len = 0

    def release(self) -> None:
        n = self.num_layers
        self._k_cache, self._v_cache = [None] * n, [None] * n
        self._layer_seq_lens, self._layer_capacity = [0] * n, [0] * n
        self._seq_len = 0

    def get_memory_mb(self) -> float:
        total = sum(t.numel() * t.element_size() for t in self._k_cache + self._v_cache if t is not None)
        return total / (1024 * 1024)

    def to_tuple(self) -> Tuple[Tuple[Tensor, Tensor], ...]:
        out = []
        for i in range(self.num_layers):
            if self._k_cache[i] is None:
                raise ValueError(f"Layer {i} cache is empty")
            out.append(self.get_kv(i))
        return tuple(out)

    @classmethod
    def from_tuple(cls, past_key_values, device: str = "cuda") -> "FP16KVCache":
        cache = cls(num_layers=len(past_key_values), device=device)
        ref = None
        for i, (k, v) in enumerate(past_key_values):
            if k.ndim != 4:
                raise ValueError(f"from_tuple(): layer {i} k must be 4D, got ndim={k.ndim}")
            if v.ndim != 4:
                raise ValueError(f"from_tuple(): layer {i} v must be 4D, got ndim={v.ndim}")
            if tuple(k.shape) != tuple(v.shape):
                raise ValueError(f"from_tuple(): layer {i} k/v shape mismatch: k={tuple(k.shape)} "
                                 f"vs v={tuple(v.shape)}")
            cur = (k.shape[0], k.shape[1], k.shape[3])
            if ref is None:
                ref = cur
            elif cur != ref:
                raise ValueError(f"from_tuple(): cross-layer shape inconsistency at layer {i}: "
                                 f"(batch, heads, head_dim)={cur} vs layer 0={ref}")
            cache.append(i, k, v)
        return cache

    def __repr__(self) -> str:
        return (f"FP16KVCache(num_layers={self.num_layers}, seq_len={self._seq_len}, "
                f"memory={self.get_memory_mb():.2f}MB)")
