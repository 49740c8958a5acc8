"""Decode-attention entry points (q_len == 1) over quantized KV caches.

Drop-in names and signatures of the reference kernels:

* :func:`decode_attn_int8` -- ``src/kernels/triton_decode_attn_int8.py:306-519``
* :func:`decode_attn_int4` -- ``src/kernels/triton_decode_attn_int4.py:62-121``

Both keep the reference's argument names, defaults, validation order, exception
types and zero-context rules.  They run the HIP split-K kernel of libkvq.so.
The INT4 path reads the packed nibbles in place; the reference first unpacks the
whole cache to int8.

Build-native formats with no reference kernel:

* :func:`decode_attn_int4_asym` -- asymmetric INT4 with static per-(head, group-32)
  fp16 scale / zero-point, and optionally 4 fp16 K outlier channels per head.
* :func:`decode_attn_k8v4` -- INT8 K (per-token/group scale) with asymmetric INT4 V.

:class:`DecodePlan` prepares the ctypes parameter block once for fixed buffers.
Repeated launches then cost one C call each, with no host synchronisation.  The
engine and the benchmark use it.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import torch

from . import _capi as C

_BLOCK_SIZES = (32, 64, 128, 256)
HEAD_DIM = 128


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _scale_dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return C.KVQ_DTYPE_F16
    if t.dtype == torch.float32:
        return C.KVQ_DTYPE_F32
    raise ValueError(f"scale dtype must be float16 or float32, got {t.dtype}")


def kv_view_tok(codes: torch.Tensor, scale: torch.Tensor) -> C.KvView:
    """View of codes [B,H,T,Dc] (int8/uint8) with per-(token, group) scale [B,H,T,G]."""
    v = C.KvView()
    v.codes = codes.data_ptr()
    v.stride_b, v.stride_h, v.stride_t = (codes.stride(0), codes.stride(1), codes.stride(2))
    v.scale = scale.data_ptr()
    (v.scale_stride_b, v.scale_stride_h, v.scale_stride_t, v.scale_stride_g) = scale.stride()
    v.scale_dtype = _scale_dtype_code(scale)
    v._keep = (codes, scale)  # the struct holds raw pointers: keep the tensors alive with it
    return v


# ---------------------------------------------------------------- TILE32 layout
#
# Asymmetric INT4 V can be stored in 32-token tiles of 2048 bytes ([B, H, T/32, 2048])
# in which lane L = 16 g + c of the decode kernel finds its PV operand at bytes
# [32 L, 32 L + 32): dword 2 p + k holds packed bytes (4 c + 2 k, 4 c + 2 k + 1) of the
# two tokens a = 0, 1 of k-slot pair p, token r = 16 (p // 2) + 4 g + 2 (p % 2) + a.
TILE_TOKENS = 32
TILE_BYTES = TILE_TOKENS * HEAD_DIM // 2
_TILE_OFF = {}


def _tile32_offsets(device) -> torch.Tensor:
    """int64 [32 * 64]: byte offset within a tile of packed byte bi of tile token r,
    indexed by r * 64 + bi."""
    key = str(device)
    if key not in _TILE_OFF:
        r = torch.arange(TILE_TOKENS).view(-1, 1)
        bi = torch.arange(HEAD_DIM // 2).view(1, -1)
        g, p, a = (r % 16) // 4, 2 * (r // 16) + (r % 4) // 2, r % 2
        c, k, j = bi // 4, (bi // 2) % 2, bi % 2
        off = ((16 * g + c) * 8 + 2 * p + k) * 4 + 2 * a + j
        _TILE_OFF[key] = off.reshape(-1).to(device)
    return _TILE_OFF[key]


def tile_v(rows: torch.Tensor) -> torch.Tensor:
    """Packed codes [B, H, T, 64] -> TILE32 layout [B, H, ceil(T/32), 2048] (zero padded)."""
    B, H, T, Dc = rows.shape
    if Dc != HEAD_DIM // 2:
        raise ValueError(f"packed rows must be [B, H, T, 64], got {tuple(rows.shape)}")
    nt = (T + TILE_TOKENS - 1) // TILE_TOKENS
    src = torch.zeros(B, H, nt * TILE_TOKENS, Dc, dtype=torch.uint8, device=rows.device)
    src[:, :, :T] = rows.view(torch.uint8)
    off = _tile32_offsets(rows.device)
    out = torch.empty(B, H, nt, TILE_BYTES, dtype=torch.uint8, device=rows.device)
    out[..., off] = src.view(B, H, nt, TILE_BYTES)
    return out


def untile_v(tiles: torch.Tensor, tokens: int) -> torch.Tensor:
    """TILE32 layout [B, H, nt, 2048] -> packed codes [B, H, tokens, 64]."""
    B, H, nt, nb = tiles.shape
    if nb != TILE_BYTES or tokens > nt * TILE_TOKENS:
        raise ValueError(f"tiles must be [B, H, nt, {TILE_BYTES}] covering {tokens} tokens")
    rows = tiles.view(torch.uint8)[..., _tile32_offsets(tiles.device)]
    return rows.view(B, H, nt * TILE_TOKENS, HEAD_DIM // 2)[:, :, :tokens]


def is_tiled(codes: torch.Tensor) -> bool:
    return codes.ndim == 4 and codes.shape[-1] == TILE_BYTES


def kv_view_static(
    codes: torch.Tensor,
    scale: torch.Tensor,
    zero_point: torch.Tensor,
    outlier_idx: Optional[torch.Tensor] = None,
    outlier_val: Optional[torch.Tensor] = None,
) -> C.KvView:
    """View of packed asymmetric INT4 codes with static scale/zp [H,G]: rows [B,H,T,D/2],
    or V tiles [B,H,T/32,2048] (TILE32 layout)."""
    v = C.KvView()
    v.codes = codes.data_ptr()
    if is_tiled(codes):
        v.layout = C.KVQ_LAYOUT_TILE32
        v.stride_b, v.stride_h, v.stride_t = codes.stride(0), codes.stride(1), HEAD_DIM // 2
    else:
        v.layout = C.KVQ_LAYOUT_ROWS
        v.stride_b, v.stride_h, v.stride_t = (codes.stride(0), codes.stride(1), codes.stride(2))
    v.scale = scale.data_ptr()
    v.scale_stride_b, v.scale_stride_t = 0, 0
    v.scale_stride_h, v.scale_stride_g = scale.stride()
    v.scale_dtype = C.KVQ_DTYPE_F16
    v.zero_point = zero_point.data_ptr()
    if outlier_idx is not None:
        v.n_outlier = int(outlier_idx.shape[-1])
        v.outlier_idx = outlier_idx.data_ptr()
        v.outlier_val = outlier_val.data_ptr()
        v.outlier_stride_b, v.outlier_stride_h, v.outlier_stride_t = (
            outlier_val.stride(0), outlier_val.stride(1), outlier_val.stride(2))
    v._keep = (codes, scale, zero_point, outlier_idx, outlier_val)
    return v


_WORKSPACES = {}


def _shared_workspace(device, nbytes: int, units: int) -> torch.Tensor:
    """A zero-filled workspace of at least nbytes for the calls of the function-style entry
    points on the current stream of device with ``units`` = batch x kv_heads, kept and
    grown between calls.  Its first units x 128 bytes are the merge counters, which every
    call leaves zero, and the partials follow them: calls with the same units ordered on
    one stream can share it.  Another units count or stream gets its own (a larger count
    would find its counters where partials were written)."""
    key = (str(device), torch.cuda.current_stream(device).cuda_stream, int(units))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


class DecodePlan:
    """A prepared kvq_decode_attn call over fixed tensors.

    Holds references to every tensor it points at and owns its workspace and
    output, so ``launch()`` is a single C call on the current stream.
    """

    def __init__(
        self,
        q: torch.Tensor,
        k_format: int,
        k_view: C.KvView,
        v_format: int,
        v_view: C.KvView,
        context_lens,
        kv_heads: int,
        capacity: int,
        sm_scale: float,
        group_size: int,
        inv_tau: Optional[torch.Tensor] = None,
        out: Optional[torch.Tensor] = None,
        chunk_tokens: int = 0,
        keepalive: tuple = (),
        shared_workspace: bool = False,
    ):
        """context_lens: int32 [B] device tensor (per-row lengths), or an int, the length
        of every row passed by value (no device read of the lengths)."""
        B, Hq, D = q.shape
        self.q = q
        self.context_lens = context_lens
        self.inv_tau = inv_tau
        self.out = torch.empty_like(q) if out is None else out
        # ctypes copies the view structs into the params block by value; keep the view
        # objects (and the tensors they point at) alive for the plan's lifetime
        self._keep = (keepalive, k_view, v_view)
        p = C.DecodeParams()
        p.q = q.data_ptr()
        p.q_stride_b, p.q_stride_h = q.stride(0), q.stride(1)
        p.inv_tau = _ptr(inv_tau)
        p.k_format, p.v_format = k_format, v_format
        p.k, p.v = k_view, v_view
        if isinstance(context_lens, torch.Tensor):
            p.context_lens = context_lens.data_ptr()
        else:
            p.context_lens = None
            p.context_len = int(context_lens)
        p.batch, p.q_heads, p.kv_heads = B, Hq, kv_heads
        p.head_dim, p.group_size = D, group_size
        p.capacity = capacity
        p.sm_scale = float(sm_scale)
        env_chunk = os.environ.get("KVQ_CHUNK_TOKENS")
        p.chunk_tokens = int(env_chunk) if (env_chunk and not chunk_tokens) else int(chunk_tokens)
        L = C.lib()
        nbytes = int(L.kvq_decode_workspace_bytes(ctypes.byref(p)))
        if shared_workspace:
            self.workspace = _shared_workspace(q.device, nbytes, B * kv_heads)
        else:
            # zero-filled once: the workspace holds the merge's arrival counters, which every
            # call leaves zero
            self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=q.device)
        p.workspace = self.workspace.data_ptr()
        p.workspace_bytes = self.workspace.numel()
        p.out = self.out.data_ptr()
        p.out_stride_b, p.out_stride_h = self.out.stride(0), self.out.stride(1)
        self.params = p
        self.chunk_tokens = int(L.kvq_decode_chunk_tokens(ctypes.byref(p)))
        self._pp = ctypes.byref(self.params)
        self.device = q.device

    def launch(self, stream: Optional[int] = None) -> torch.Tensor:
        s = C.stream_handle(self.device) if stream is None else stream
        C.check(C.lib().kvq_decode_attn(self._pp, ctypes.c_void_p(s)))
        return self.out

    def launch_noalloc(self, stream: Optional[int] = None) -> torch.Tensor:
        """The same attention through kvq_decode_attn_noalloc: the split-K workspace is the
        library's fixed per-GPU device array instead of this plan's (bit-identical output;
        calls that may overlap on one GPU race on that array)."""
        s = C.stream_handle(self.device) if stream is None else stream
        C.check(C.lib().kvq_decode_attn_noalloc(self._pp, ctypes.c_void_p(s)))
        return self.out

    def launch_append(self, k_new: C.AppendParams, v_new: C.AppendParams,
                      stream: Optional[int] = None) -> torch.Tensor:
        """One launch: quantize-on-append of the new token described by k_new / v_new
        (which must target this plan's cache buffers) followed by this plan's attention
        (kvq_append_decode_attn).  The caller keeps the tensors k_new / v_new point at
        alive until the launch has run."""
        s = C.stream_handle(self.device) if stream is None else stream
        C.check(C.lib().kvq_append_decode_attn(self._pp, ctypes.byref(k_new), ctypes.byref(v_new),
                                               ctypes.c_void_p(s)))
        return self.out


class LayerStep:
    """The kvq_decode_params block of one cache layer, kept from one decode step to the next.

    The K / V views point at the layer's code and scale buffers (whole capacity); per call
    only q, the output, the context length (passed by value: ``context_lens`` is NULL, every
    row has the same length, as in the reference's decode step,
    src/engine/patch_model.py:799-804) and, for the fused step, the new rows change.  The
    workspace is kept and grows when a call needs more; its merge counters sit at its start,
    so a zero-filled workspace serves every later call.  A call costs one C call plus the
    output allocation: no device tensor is created, filled or read back.
    """

    def __init__(self, k_format: int, k_view: C.KvView, v_format: int, v_view: C.KvView,
                 batch: int, q_heads: int, kv_heads: int, group_size: int, device,
                 keepalive: tuple = ()):
        self._keep = (keepalive, k_view, v_view)
        p = C.DecodeParams()
        p.k_format, p.v_format = k_format, v_format
        p.k, p.v = k_view, v_view
        p.context_lens = None
        p.batch, p.q_heads, p.kv_heads = batch, q_heads, kv_heads
        p.head_dim, p.group_size = HEAD_DIM, group_size
        env_chunk = os.environ.get("KVQ_CHUNK_TOKENS")
        p.chunk_tokens = int(env_chunk) if env_chunk else 0
        self.params = p
        self._pp = ctypes.byref(p)
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device(self.device.type, torch.cuda.current_device())
        self.workspace: Optional[torch.Tensor] = None
        self._tau = None
        # the workspace a call needs depends on the context length only through its 32-token
        # tile count (chunk sizes are multiples of 32 tokens): asked again when that changes
        self._ws_tiles = -1

    def _prepare(self, q: torch.Tensor, n: int, sm_scale: float,
                 inv_tau: Optional[torch.Tensor]) -> torch.Tensor:
        p = self.params
        p.q = q.data_ptr()
        p.q_stride_b, p.q_stride_h = q.stride(0), q.stride(1)
        p.inv_tau = _ptr(inv_tau)
        self._tau = inv_tau
        p.capacity = n
        p.context_len = n
        p.sm_scale = float(sm_scale)
        tiles = (n + 31) >> 5
        if tiles != self._ws_tiles:
            need = int(C.lib().kvq_decode_workspace_bytes(self._pp))
            if self.workspace is None or self.workspace.numel() < need:
                # zero-filled when (re)allocated: the merge counters at its start must be zero
                self.workspace = torch.zeros(max(need, int(need * 1.25)), dtype=torch.uint8,
                                             device=self.device)
                p.workspace = self.workspace.data_ptr()
                p.workspace_bytes = self.workspace.numel()
            self._ws_tiles = tiles
        out = torch.empty_like(q)
        p.out = out.data_ptr()
        p.out_stride_b, p.out_stride_h = out.stride(0), out.stride(1)
        return out

    def set_residual(self, res_k: Optional[torch.Tensor], res_v: Optional[torch.Tensor], n: int) -> None:
        """The fp16 residual window attended with the quantized tokens: the first n tokens of
        res_k / res_v [B, Hkv, R, 128] (fp16, dense rows); n = 0 or None buffers: none."""
        p = self.params
        if res_k is None or n <= 0:
            p.res_k = p.res_v = None
            p.res_stride_b = p.res_stride_h = 0
            p.res_tokens = 0
            return
        p.res_k, p.res_v = res_k.data_ptr(), res_v.data_ptr()
        p.res_stride_b, p.res_stride_h = res_k.stride(0), res_k.stride(1)
        p.res_tokens = int(n)
        self._res = (res_k, res_v)

    def attend(self, q: torch.Tensor, n: int, sm_scale: float,
               inv_tau: Optional[torch.Tensor] = None) -> torch.Tensor:
        """kvq_decode_attn of q [B, Hq, 128] fp16 over the first n tokens of every row."""
        out = self._prepare(q, n, sm_scale, inv_tau)
        C.check(C.lib().kvq_decode_attn(self._pp, ctypes.c_void_p(C.stream_handle(self.device))))
        return out

    def append_attend(self, q: torch.Tensor, n: int, sm_scale: float,
                      inv_tau: Optional[torch.Tensor], k_new: C.AppendParams,
                      v_new: C.AppendParams) -> torch.Tensor:
        """kvq_append_decode_attn: the new token described by k_new / v_new (slot n - 1)
        quantized into the layer's buffers and attention over the first n tokens, one
        launch."""
        out = self._prepare(q, n, sm_scale, inv_tau)
        C.check(C.lib().kvq_append_decode_attn(self._pp, ctypes.byref(k_new), ctypes.byref(v_new),
                                               ctypes.c_void_p(C.stream_handle(self.device))))
        return out


def _bump_debug_stats(debug_stats, layer_idx, block_size):
    # same keys as the reference wrapper (triton_decode_attn_int8.py:474-480),
    # which patch_model.py and the reference tests read
    if isinstance(debug_stats, dict):
        debug_stats["triton_kernel_calls"] = int(debug_stats.get("triton_kernel_calls", 0)) + 1
        debug_stats["triton_block_size"] = int(block_size)
        if layer_idx is not None:
            hits = debug_stats.setdefault("triton_layer_hits", {})
            key = str(layer_idx)
            hits[key] = int(hits.get(key, 0)) + 1


def _resolve_block_size(block_size, max_ctx):
    if block_size is None:
        env = os.environ.get("KV_TRITON_BLOCK_SIZE")
        if env:
            try:
                block_size = int(env)
            except ValueError as exc:
                raise ValueError(f"KV_TRITON_BLOCK_SIZE must be an integer, got {env!r}") from exc
        else:
            block_size = 128 if max_ctx >= 8192 else 64
    if block_size not in _BLOCK_SIZES:
        raise ValueError(f"Unsupported block_size={block_size}. Choose from [32, 64, 128, 256].")
    return block_size


def decode_attn_int8(
    q,
    k_cache,
    v_cache,
    k_scale,
    v_scale,
    context_lens,
    sm_scale=None,
    debug_stats: Optional[dict] = None,
    layer_idx: Optional[int] = None,
    block_size: Optional[int] = None,
):
    """q_len == 1 attention over INT8 K/V with per-(token, group) fp16 scales.

    Same contract as ``decode_attn_int8`` (src/kernels/triton_decode_attn_int8.py:306-519):
    q [B, Hq, D]; k_cache/v_cache int8 [B, Hkv, S, D]; k_scale/v_scale fp16
    [B, Hkv, S, G]; context_lens [B]; returns [B, Hq, D] in q's dtype.  Rows whose
    context length is 0 are zero.  ``block_size`` is validated like the reference,
    but the HIP kernel picks its own split size.
    """
    return _decode_tok(q, k_cache, v_cache, k_scale, v_scale, context_lens, sm_scale,
                       debug_stats, layer_idx, block_size, packed=False, head_dim=None)


def decode_attn_int4(
    q: torch.Tensor,
    k_cache_int4: torch.Tensor,
    v_cache_int4: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    context_lens: torch.Tensor,
    sm_scale: Optional[float] = None,
    *,
    bit_packed: bool = True,
    head_dim: Optional[int] = None,
    debug_stats: Optional[dict] = None,
    layer_idx: Optional[int] = None,
    block_size: Optional[int] = None,
) -> torch.Tensor:
    """q_len == 1 attention over INT4 K/V (src/kernels/triton_decode_attn_int4.py:62-121).

    Packed caches [B, Hkv, S, D/2] (byte = hi nibble even channel, +8 offset) are read
    in place.  Unpacked caches (int8 codes in [-8, 7], [B, Hkv, S, D]) take the INT8
    kernel, exactly as in the reference.
    """
    if q.ndim != 3:
        raise ValueError(f"q must have shape [B, Hq, D], got {tuple(q.shape)}")
    if head_dim is not None:
        d = int(head_dim)
        if d <= 0:
            raise ValueError(f"head_dim must be positive, got {d}")
    else:
        d = q.shape[-1]
    for name, cache in (("k", k_cache_int4), ("v", v_cache_int4)):
        if not bit_packed:
            if cache.shape[-1] != d:
                raise ValueError(
                    f"Unpacked INT4 cache last dim mismatch: got {cache.shape[-1]}, expected {d}")
            if cache.stride(-1) != 1:
                raise ValueError(
                    "Unpacked INT4 cache inner dim must be contiguous (stride=1), "
                    f"got stride={cache.stride(-1)}. Use .contiguous().")
            if cache.dtype != torch.int8:
                raise ValueError(
                    f"Unpacked INT4 cache must be int8, got {cache.dtype}. "
                    "Unpacked INT4 values should be stored as torch.int8.")
        elif cache.shape[-1] * 2 != d:
            raise ValueError(
                f"Packed INT4 cache last dim mismatch: got {cache.shape[-1]}, expected {d // 2}")
    return _decode_tok(q, k_cache_int4, v_cache_int4, k_scale, v_scale, context_lens, sm_scale,
                       debug_stats, layer_idx, block_size, packed=bool(bit_packed), head_dim=d)


def _decode_tok(q, k_cache, v_cache, k_scale, v_scale, context_lens, sm_scale, debug_stats,
                layer_idx, block_size, packed, head_dim):
    if sm_scale is None:
        sm_scale = 1.0 / (q.shape[-1] ** 0.5)
    if q.ndim != 3:
        raise ValueError(f"q must have shape [B, Hq, D], got {tuple(q.shape)}")
    if k_cache.ndim != 4 or v_cache.ndim != 4:
        raise ValueError(
            "k_cache/v_cache must have shape [B, Hkv, S, D], got "
            f"{tuple(k_cache.shape)} / {tuple(v_cache.shape)}")
    if k_scale.ndim != 4 or v_scale.ndim != 4:
        raise ValueError(
            "k_scale/v_scale must have shape [B, Hkv, S, G], got "
            f"{tuple(k_scale.shape)} / {tuple(v_scale.shape)}")
    if context_lens.ndim != 1:
        raise ValueError(f"context_lens must be 1D, got {tuple(context_lens.shape)}")
    if not q.is_cuda:
        raise ValueError("decode_attn_int8 requires GPU (ROCm) tensors.")
    if k_cache.dtype != torch.int8:
        raise ValueError(f"k_cache must be torch.int8, got {k_cache.dtype}")
    if v_cache.dtype != torch.int8:
        raise ValueError(f"v_cache must be torch.int8, got {v_cache.dtype}")
    if k_scale.dtype != torch.float16:
        raise ValueError(
            f"k_scale must be torch.float16 for the fused kernel, got {k_scale.dtype}. "
            "Cast with k_scale.to(torch.float16) before calling.")
    if v_scale.dtype != torch.float16:
        raise ValueError(
            f"v_scale must be torch.float16 for the fused kernel, got {v_scale.dtype}. "
            "Cast with v_scale.to(torch.float16) before calling.")
    if k_cache.stride(-1) != 1:
        raise ValueError(
            f"k_cache inner dim must be contiguous (stride=1), got stride={k_cache.stride(-1)}. "
            "Use .contiguous() before passing to kernel.")
    if v_cache.stride(-1) != 1:
        raise ValueError(
            f"v_cache inner dim must be contiguous (stride=1), got stride={v_cache.stride(-1)}.")
    batch, q_heads, hd = q.shape
    if hd == 0 or (hd & (hd - 1)) != 0:
        raise ValueError(f"HEAD_DIM must be a power of 2, got {hd}.")
    code_dim = hd // 2 if packed else hd
    if k_cache.shape[0] != batch or v_cache.shape[0] != batch:
        raise ValueError(
            f"Batch mismatch: q={batch}, k={k_cache.shape[0]}, v={v_cache.shape[0]}")
    if k_cache.shape[-1] != code_dim or v_cache.shape[-1] != code_dim:
        raise ValueError(
            f"Head dim mismatch: q={hd}, k={k_cache.shape[-1]}, v={v_cache.shape[-1]}")
    if k_cache.shape[:3] != v_cache.shape[:3]:
        raise ValueError(
            f"k/v cache shape mismatch: {tuple(k_cache.shape)} vs {tuple(v_cache.shape)}")
    if k_scale.shape[:3] != k_cache.shape[:3] or v_scale.shape[:3] != v_cache.shape[:3]:
        raise ValueError(
            "Scale and cache shapes mismatch: "
            f"k_scale={tuple(k_scale.shape)}, v_scale={tuple(v_scale.shape)}, "
            f"k={tuple(k_cache.shape)}, v={tuple(v_cache.shape)}")
    if k_scale.shape[-1] != v_scale.shape[-1]:
        raise ValueError(
            f"k_scale/v_scale num_groups mismatch: k={k_scale.shape[-1]} vs v={v_scale.shape[-1]}.")
    if context_lens.shape[0] != batch:
        raise ValueError(
            f"context_lens batch mismatch: expected {batch}, got {context_lens.shape[0]}")
    kv_heads = k_cache.shape[1]
    if q_heads % kv_heads != 0:
        raise ValueError(
            f"GQA head mismatch: q_heads={q_heads} must be a multiple of kv_heads={kv_heads}")
    num_groups = k_scale.shape[-1]
    if num_groups <= 0:
        raise ValueError(f"num_groups must be > 0, got {num_groups}")
    if hd % num_groups != 0:
        raise ValueError(f"head_dim {hd} must be divisible by num_groups {num_groups}")
    group_size = hd // num_groups
    max_seq = int(k_cache.shape[2])
    # the reference validates context lengths on the host (one sync); so does this wrapper
    max_ctx = int(context_lens.max().item()) if context_lens.numel() else 0
    min_ctx = int(context_lens.min().item()) if context_lens.numel() else 0
    if min_ctx < 0:
        raise ValueError(f"context_lens must be >= 0, got min={min_ctx}")
    if max_ctx > max_seq:
        raise ValueError(f"context_lens max ({max_ctx}) exceeds cache seq dim ({max_seq})")
    if max_ctx == 0:
        return torch.zeros_like(q)
    if hd != HEAD_DIM:
        raise NotImplementedError(f"the HIP decode kernel supports head_dim=128, got {hd}")
    block_size = _resolve_block_size(block_size, max_ctx)

    original_dtype = q.dtype
    qk = q if q.dtype == torch.float16 else q.to(torch.float16)
    if qk.stride(-1) != 1:
        qk = qk.contiguous()
    ctx = context_lens if context_lens.dtype == torch.int32 else context_lens.to(torch.int32)
    if ctx.device != q.device:
        ctx = ctx.to(q.device)
    fmt = C.KVQ_FMT_INT4_SYM if packed else C.KVQ_FMT_INT8_SYM
    plan = DecodePlan(
        qk, fmt, kv_view_tok(k_cache, k_scale), fmt, kv_view_tok(v_cache, v_scale),
        ctx, kv_heads, max_seq, sm_scale, group_size,
        keepalive=(k_cache, v_cache, k_scale, v_scale), shared_workspace=True)
    _bump_debug_stats(debug_stats, layer_idx, block_size)
    out = plan.launch()
    if original_dtype != torch.float16:
        out = out.to(original_dtype)
    return out


def kv_view_kivi(codes: torch.Tensor, scale: torch.Tensor, zero_point: torch.Tensor,
                 per_channel: bool) -> C.KvView:
    """View of KIVI-layout packed INT4 rows [B,H,T,64] with fp32 scale / zero-point
    (same strides): per channel [B,H,D] (K) or per token [B,H,T] (V)."""
    v = C.KvView()
    v.codes = codes.data_ptr()
    v.layout = C.KVQ_LAYOUT_ROWS
    v.stride_b, v.stride_h, v.stride_t = codes.stride(0), codes.stride(1), codes.stride(2)
    v.scale = scale.data_ptr()
    v.scale_stride_b, v.scale_stride_h = scale.stride(0), scale.stride(1)
    if per_channel:
        v.scale_stride_t, v.scale_stride_g = 0, scale.stride(2)
    else:
        v.scale_stride_t, v.scale_stride_g = scale.stride(2), 0
    v.scale_dtype = C.KVQ_DTYPE_F32
    v.zero_point = zero_point.data_ptr()
    v._keep = (codes, scale, zero_point)
    return v


def kv_view_fp16(x: torch.Tensor) -> C.KvView:
    """View of fp16 values [B,H,T,128] (a 16-bit side, format KVQ_FMT_FP16): strides in bytes,
    no scale."""
    if x.dtype != torch.float16 or x.stride(-1) != 1:
        raise ValueError(f"fp16 K/V rows must be fp16 with contiguous channels, got {x.dtype}")
    v = C.KvView()
    v.codes = x.data_ptr()
    v.layout = C.KVQ_LAYOUT_ROWS
    v.stride_b, v.stride_h, v.stride_t = 2 * x.stride(0), 2 * x.stride(1), 2 * x.stride(2)
    v.scale = None
    v.scale_dtype = C.KVQ_DTYPE_F16
    v._keep = (x,)
    return v


def _kivi_params(t: torch.Tensor, shape) -> torch.Tensor:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"KIVI scale/zero-point must be {tuple(shape)}, got {tuple(t.shape)}")
    t = t if t.dtype == torch.float32 else t.float()
    return t if t.stride(-1) == 1 else t.contiguous()


def decode_attn_int4_kivi(
    q: torch.Tensor,
    k_cache_packed: torch.Tensor,
    v_cache_packed: torch.Tensor,
    k_scale: torch.Tensor,
    k_zp: torch.Tensor,
    v_scale: torch.Tensor,
    v_zp: torch.Tensor,
    context_lens: torch.Tensor,
    sm_scale: Optional[float] = None,
    block_size: Optional[int] = None,
    *,
    inv_tau: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention over the KIVI layout (src/kernels/triton_decode_attn_int4_asym.py:163-277):
    packed INT4 K/V rows [B, Hkv, S, 64] (byte = ((c[2i]+8) << 4) | (c[2i+1]+8)),
    per-channel K scale / zero-point [B, Hkv, D], per-token V scale / zero-point
    [B, Hkv, S]; value c * s + z.  Parameters are used in fp32 (fp16 ones are widened, as
    the reference does); q is computed in fp16 and the output has q's dtype.  block_size
    is accepted for signature compatibility: the split over the context is chosen by the
    library.  inv_tau (fp16 [Hq]) is an optional per-head query scale.
    """
    if q.ndim != 3 or q.shape[-1] != HEAD_DIM:
        raise ValueError(f"q must be [B, Hq, 128], got {tuple(q.shape)}")
    if k_cache_packed.ndim != 4 or v_cache_packed.ndim != 4:
        raise ValueError(f"cache must be [B, Hkv, S, D//2], got K={tuple(k_cache_packed.shape)} "
                         f"V={tuple(v_cache_packed.shape)}")
    if k_scale.ndim != 3 or k_zp.ndim != 3:
        raise ValueError(f"k_scale/k_zp must be [B, Hkv, D], got {tuple(k_scale.shape)}/{tuple(k_zp.shape)}")
    if v_scale.ndim != 3 or v_zp.ndim != 3:
        raise ValueError(f"v_scale/v_zp must be [B, Hkv, S], got {tuple(v_scale.shape)}/{tuple(v_zp.shape)}")
    if not q.is_cuda:
        raise ValueError("requires GPU (ROCm) tensors")
    B, Hq, D = q.shape
    Hkv, S = k_cache_packed.shape[1], k_cache_packed.shape[2]
    for c in (k_cache_packed, v_cache_packed):
        if tuple(c.shape) != (B, Hkv, S, D // 2) or c.dtype not in (torch.int8, torch.uint8):
            raise ValueError(f"packed codes must be int8/uint8 [{B}, {Hkv}, {S}, 64], got {tuple(c.shape)}")
    if Hq % Hkv:
        raise ValueError(f"q_heads={Hq} not multiple of kv_heads={Hkv}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    _resolve_block_size(block_size, S)
    ks, kz = _kivi_params(k_scale, (B, Hkv, D)), _kivi_params(k_zp, (B, Hkv, D))
    vs, vz = _kivi_params(v_scale, (B, Hkv, S)), _kivi_params(v_zp, (B, Hkv, S))
    kc = k_cache_packed if k_cache_packed.stride(-1) == 1 and k_cache_packed.stride(2) == D // 2 \
        else k_cache_packed.contiguous()
    vc = v_cache_packed if v_cache_packed.stride(-1) == 1 and v_cache_packed.stride(2) == D // 2 \
        else v_cache_packed.contiguous()
    original_dtype = q.dtype
    q16 = q if q.dtype == torch.float16 else q.to(torch.float16)
    plan = DecodePlan(
        q16, C.KVQ_FMT_INT4_KIVI, kv_view_kivi(kc, ks, kz, True),
        C.KVQ_FMT_INT4_KIVI, kv_view_kivi(vc, vs, vz, False),
        _ctx_i32(context_lens, q.device), Hkv, S, sm_scale, 32, inv_tau=inv_tau,
        keepalive=(kc, vc, ks, kz, vs, vz), shared_workspace=True)
    out = plan.launch()
    return out if original_dtype == torch.float16 else out.to(original_dtype)


# the reference's v2 and GQA-tiled kernels compute the same function with other tilings
# (src/kernels/triton_decode_attn_int4_asym_v2.py:186, triton_decode_attn_int4_asym_gqa.py:204)
decode_attn_int4_asym_v2 = decode_attn_int4_kivi
decode_attn_int4_asym_gqa = decode_attn_int4_kivi


def decode_attn_int4_asym(
    q: torch.Tensor,
    k_codes: torch.Tensor,
    v_codes: torch.Tensor,
    k_scale: torch.Tensor,
    k_zp: torch.Tensor,
    v_scale: torch.Tensor,
    v_zp: torch.Tensor,
    context_lens: torch.Tensor,
    sm_scale: Optional[float] = None,
    block_size: Optional[int] = None,
    *,
    inv_tau: Optional[torch.Tensor] = None,
    k_outlier_idx: Optional[torch.Tensor] = None,
    k_outlier_val: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention over the asymmetric INT4 group-32 format (build-native); with
    k_scale of rank 3 ([B, Hkv, D], the reference's signature) the KIVI layout
    (:func:`decode_attn_int4_kivi`).

    k_codes: packed uint8/int8 [B, Hkv, S, 64]; v_codes: the same, or V in the TILE32
    layout [B, Hkv, ceil(S/32), 2048] (:func:`tile_v`); k_scale/k_zp/v_scale/v_zp: fp16
    [Hkv, 4] static parameters; optional k_outlier_idx int32 [Hkv, 4] and
    k_outlier_val fp16 [B, Hkv, S, 4] (K channels stored verbatim).  inv_tau: fp16
    [Hq] per-head query scale, applied as fp16(q * inv_tau) like the reference
    (src/engine/patch_model.py:711-746).
    """
    if k_scale.ndim == 3:
        if k_outlier_idx is not None:
            raise ValueError("outlier channels are not part of the KIVI layout")
        return decode_attn_int4_kivi(q, k_codes, v_codes, k_scale, k_zp, v_scale, v_zp,
                                     context_lens, sm_scale, block_size, inv_tau=inv_tau)
    _check_static_args(q, k_codes, v_codes, (k_scale, k_zp, v_scale, v_zp), context_lens)
    if (k_outlier_idx is None) != (k_outlier_val is None):
        raise ValueError("k_outlier_idx and k_outlier_val must be given together")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    plan = DecodePlan(
        q, C.KVQ_FMT_INT4_ASYM,
        kv_view_static(k_codes, k_scale, k_zp, k_outlier_idx, k_outlier_val),
        C.KVQ_FMT_INT4_ASYM, kv_view_static(v_codes, v_scale, v_zp),
        _ctx_i32(context_lens, q.device), k_codes.shape[1], k_codes.shape[2], sm_scale, 32,
        inv_tau=inv_tau,
        keepalive=(k_codes, v_codes, k_scale, k_zp, v_scale, v_zp, k_outlier_idx, k_outlier_val),
        shared_workspace=True)
    return plan.launch()


def decode_attn_k8v4(
    q: torch.Tensor,
    k_codes: torch.Tensor,
    k_scale: torch.Tensor,
    v_codes: torch.Tensor,
    v_scale: torch.Tensor,
    v_zp: torch.Tensor,
    context_lens: torch.Tensor,
    sm_scale: Optional[float] = None,
    *,
    inv_tau: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """INT8 K (scale [B,Hkv,S,4], may be an expanded static view) + asymmetric INT4 V."""
    if k_codes.dtype != torch.int8 or k_codes.shape[-1] != 128:
        raise ValueError("k_codes must be int8 [B, Hkv, S, 128]")
    if k_scale.ndim != 4 or k_scale.shape[-1] != 4:
        raise ValueError("k_scale must be [B, Hkv, S, 4] (group 32)")
    _check_static_args(q, v_codes, v_codes, (v_scale, v_zp), context_lens)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    plan = DecodePlan(
        q, C.KVQ_FMT_INT8_SYM, kv_view_tok(k_codes, k_scale),
        C.KVQ_FMT_INT4_ASYM, kv_view_static(v_codes, v_scale, v_zp),
        _ctx_i32(context_lens, q.device), k_codes.shape[1], k_codes.shape[2], sm_scale, 32,
        inv_tau=inv_tau, keepalive=(k_codes, k_scale, v_codes, v_scale, v_zp), shared_workspace=True)
    return plan.launch()


def _ctx_i32(context_lens: torch.Tensor, device) -> torch.Tensor:
    c = context_lens if context_lens.dtype == torch.int32 else context_lens.to(torch.int32)
    return c if c.device == device else c.to(device)


def _check_static_args(q, k_codes, v_codes, params, context_lens):
    if q.ndim != 3 or q.dtype != torch.float16 or q.shape[-1] != HEAD_DIM:
        raise ValueError(f"q must be fp16 [B, Hq, 128], got {q.dtype} {tuple(q.shape)}")
    if not q.is_cuda:
        raise ValueError("requires GPU (ROCm) tensors")
    for c in (k_codes, v_codes):
        if c is v_codes and is_tiled(c):
            if c.dtype != torch.uint8 or c.shape[:2] != k_codes.shape[:2] or \
                    c.shape[2] * TILE_TOKENS < k_codes.shape[2] or c.stride(-1) != 1:
                raise ValueError(f"TILE32 V must be uint8 [B, Hkv, >= S/32, {TILE_BYTES}] "
                                 f"contiguous in the last dim, got {tuple(c.shape)}")
            continue
        if c.ndim != 4 or c.shape[-1] != HEAD_DIM // 2 or c.dtype not in (torch.int8, torch.uint8):
            raise ValueError(f"packed codes must be int8/uint8 [B, Hkv, S, 64], got {tuple(c.shape)}")
        if c.stride(-1) != 1:
            raise ValueError("packed codes must be contiguous in the last dim")
    Hkv = k_codes.shape[1]
    for t in params:
        if t.dtype != torch.float16 or tuple(t.shape) != (Hkv, 4):
            raise ValueError(f"static scale/zero-point must be fp16 [{Hkv}, 4], got {t.dtype} {tuple(t.shape)}")
    if context_lens.ndim != 1 or context_lens.shape[0] != q.shape[0]:
        raise ValueError("context_lens must be [B]")
    if q.shape[1] % Hkv:
        raise ValueError("q_heads must be a multiple of kv_heads")
