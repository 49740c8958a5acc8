"""ctypes binding of libkvq.so (declared in include/kvq.h).

PyTorch is imported before the library is opened, so libkvq.so resolves
``libamdhip64.so.7`` to the HIP runtime PyTorch already loaded.  Kernels launched
through this module therefore run on torch's streams and read torch's allocations.

There is deliberately no fallback: if the library is missing or was built for
another ABI, every entry point raises instead of computing something else.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before libkvq.so, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libkvq.so"
ABI_VERSION = 6

KVQ_OK = 0
KVQ_ERR_INVALID = 1
KVQ_ERR_UNSUPPORTED = 2
KVQ_ERR_LAUNCH = 3

KVQ_DTYPE_F16 = 0
KVQ_DTYPE_F32 = 1

KVQ_FMT_INT8_SYM = 1
KVQ_FMT_INT4_SYM = 2
KVQ_FMT_INT4_ASYM = 3
KVQ_FMT_INT4_KIVI = 4
KVQ_FMT_INT8_KIVI = 5
KVQ_FMT_FP16 = 6

KVQ_LAYOUT_ROWS = 0
KVQ_LAYOUT_TILE32 = 1

# size of the device array kvq_decode_attn_noalloc keeps its workspace in
KVQ_NOALLOC_SCRATCH_BYTES = 16 << 20

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p


class KvView(ctypes.Structure):
    _fields_ = [
        ("codes", c_vp),
        ("stride_b", c_i64), ("stride_h", c_i64), ("stride_t", c_i64),
        ("scale", c_vp),
        ("scale_stride_b", c_i64), ("scale_stride_h", c_i64),
        ("scale_stride_t", c_i64), ("scale_stride_g", c_i64),
        ("scale_dtype", c_i32),
        ("n_outlier", c_i32),
        ("zero_point", c_vp),
        ("outlier_idx", c_vp),
        ("outlier_val", c_vp),
        ("outlier_stride_b", c_i64), ("outlier_stride_h", c_i64), ("outlier_stride_t", c_i64),
        ("layout", c_i32), ("reserved", c_i32),
    ]


class DecodeParams(ctypes.Structure):
    _fields_ = [
        ("q", c_vp),
        ("q_stride_b", c_i64), ("q_stride_h", c_i64),
        ("inv_tau", c_vp),
        ("k_format", c_i32), ("v_format", c_i32),
        ("k", KvView), ("v", KvView),
        ("context_lens", c_vp),
        ("batch", c_i32), ("q_heads", c_i32), ("kv_heads", c_i32),
        ("head_dim", c_i32), ("group_size", c_i32),
        ("capacity", c_i64),
        ("sm_scale", c_f32),
        ("chunk_tokens", c_i32),
        ("workspace", c_vp),
        ("workspace_bytes", c_i64),
        ("out", c_vp),
        ("out_stride_b", c_i64), ("out_stride_h", c_i64),
        ("context_len", c_i32), ("v_group_size", c_i32),
        ("res_k", c_vp), ("res_v", c_vp),
        ("res_stride_b", c_i64), ("res_stride_h", c_i64),
        ("res_tokens", c_i32), ("pad1", c_i32),
    ]


class AppendParams(ctypes.Structure):
    _fields_ = [
        ("format", c_i32),
        ("x", c_vp),
        ("x_stride_b", c_i64), ("x_stride_h", c_i64), ("x_stride_s", c_i64),
        ("batch", c_i32), ("heads", c_i32), ("seq_new", c_i32),
        ("head_dim", c_i32), ("group_size", c_i32),
        ("static_scale", c_vp),
        ("static_scale_dtype", c_i32),
        ("static_stride_h", c_i64), ("static_stride_g", c_i64),
        ("static_zp", c_vp),
        ("adaptive", c_i32),
        ("adaptive_margin", c_f32),
        ("mixed_rescue", c_i32),
        ("rescue_quantile", c_f32),
        ("rescue_all", c_i32),
        ("codes", c_vp),
        ("codes_stride_b", c_i64), ("codes_stride_h", c_i64), ("codes_stride_t", c_i64),
        ("scale_out", c_vp),
        ("scale_out_dtype", c_i32),
        ("so_stride_b", c_i64), ("so_stride_h", c_i64), ("so_stride_t", c_i64),
        ("so_stride_g", c_i64),
        ("n_outlier", c_i32),
        ("outlier_idx", c_vp),
        ("outlier_out", c_vp),
        ("oo_stride_b", c_i64), ("oo_stride_h", c_i64), ("oo_stride_t", c_i64),
        ("write_pos", c_i64),
        ("capacity", c_i64),
        ("status", c_vp),
        ("codes_layout", c_i32), ("reserved", c_i32),
        ("scratch", c_vp), ("scratch_bytes", c_i64),
        ("static_stride_b", c_i64), ("zp_out", c_vp),
        ("dyn_quantile", c_f32), ("dyn_quantile_lo", c_f32),
    ]


EXPORTED_SYMBOLS = (
    "kvq_decode_attn",
    "kvq_decode_attn_noalloc",
    "kvq_append_decode_attn",
    "kvq_decode_chunk_tokens",
    "kvq_decode_workspace_bytes",
    "kvq_quant_append",
    "kvq_append_scratch_bytes",
    "kvq_stream_read",
    "kvq_last_error",
    "kvq_abi_version",
)

_lib = None
_lock = threading.Lock()


class KvqError(RuntimeError):
    """A libkvq entry point returned a non-OK status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"libkvq error {code}: {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Open libkvq.so once; raises if it is missing or built for another ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with "
                "`python -m llm_kvcache_quantization_amd.build` (hipcc, gfx950)"
            )
        L = ctypes.CDLL(str(LIB_PATH))
        L.kvq_decode_attn.argtypes = [ctypes.POINTER(DecodeParams), c_vp]
        L.kvq_decode_attn.restype = c_i32
        L.kvq_decode_attn_noalloc.argtypes = [ctypes.POINTER(DecodeParams), c_vp]
        L.kvq_decode_attn_noalloc.restype = c_i32
        L.kvq_decode_chunk_tokens.argtypes = [ctypes.POINTER(DecodeParams)]
        L.kvq_decode_chunk_tokens.restype = c_i32
        L.kvq_decode_workspace_bytes.argtypes = [ctypes.POINTER(DecodeParams)]
        L.kvq_decode_workspace_bytes.restype = c_i64
        L.kvq_quant_append.argtypes = [ctypes.POINTER(AppendParams), ctypes.POINTER(AppendParams), c_vp]
        L.kvq_quant_append.restype = c_i32
        L.kvq_append_scratch_bytes.argtypes = [ctypes.POINTER(AppendParams)]
        L.kvq_append_scratch_bytes.restype = c_i64
        L.kvq_append_decode_attn.argtypes = [ctypes.POINTER(DecodeParams), ctypes.POINTER(AppendParams),
                                             ctypes.POINTER(AppendParams), c_vp]
        L.kvq_append_decode_attn.restype = c_i32
        L.kvq_stream_read.argtypes = [c_vp, c_i64, c_vp, c_i32, c_vp]
        L.kvq_stream_read.restype = c_i32
        L.kvq_last_error.argtypes = []
        L.kvq_last_error.restype = ctypes.c_char_p
        L.kvq_abi_version.argtypes = []
        L.kvq_abi_version.restype = c_i32
        ver = L.kvq_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI {ver}, this package needs {ABI_VERSION}; rebuild it")
        _lib = L
        return _lib


def check(rc: int) -> None:
    if rc != KVQ_OK:
        msg = lib().kvq_last_error().decode(errors="replace")
        if rc in (KVQ_ERR_INVALID,):
            raise ValueError(msg)
        if rc == KVQ_ERR_UNSUPPORTED:
            raise NotImplementedError(msg)
        raise KvqError(rc, msg)


# torch's raw current-stream getter: a few hundred ns, where torch.cuda.current_stream(...)
# builds a Stream object (a few microseconds per decode call)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (as an int)."""
    idx = device.index
    if _raw_stream is not None and idx is not None:
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream
