"""CPU tests of kvq_append_decode_attn's host-side routing for the row formats: the calls
below are refused before any HIP call (so they run without a GPU), with the reason a
caller needs to fall back to kvq_quant_append + kvq_decode_attn.  The buffers are never
touched: the pointers are placeholders."""
import ctypes

import numpy as np
import pytest

from llm_kvcache_quantization_amd import _capi as C

B_FAKE = 0x100000  # 16-byte-aligned placeholder addresses, never dereferenced


def _lib():
    if not C.LIB_PATH.exists():
        pytest.skip("libkvq.so not built (run __graft_entry__.build())")
    return C.lib()


def _view(codes, scale, B, H, T, G):
    """INT4_SYM per-token view: packed rows [B, H, T, 64], fp32 scales [B, H, T, G]."""
    v = C.KvView()
    v.codes = codes
    v.stride_b, v.stride_h, v.stride_t = H * T * 64, T * 64, 64
    v.scale = scale
    v.scale_stride_b, v.scale_stride_h, v.scale_stride_t, v.scale_stride_g = H * T * G, T * G, G, 1
    v.scale_dtype = C.KVQ_DTYPE_F32
    v.layout = C.KVQ_LAYOUT_ROWS
    return v


def _setup(B, H, n_rep=4, T=64, gs=16, ratio=0.01):
    G = 128 // gs
    p = C.DecodeParams()
    p.q = B_FAKE
    p.q_stride_b, p.q_stride_h = H * n_rep * 128, 128
    p.k_format = p.v_format = C.KVQ_FMT_INT4_SYM
    kv = _view(B_FAKE * 2, B_FAKE * 3, B, H, T, G)
    vv = _view(B_FAKE * 4, B_FAKE * 5, B, H, T, G)
    p.k, p.v = kv, vv
    p.batch, p.q_heads, p.kv_heads, p.head_dim, p.group_size = B, H * n_rep, H, 128, gs
    p.capacity = T
    p.context_len = T
    p.sm_scale = 0.088
    p.out = B_FAKE * 6
    p.out_stride_b, p.out_stride_h = H * n_rep * 128, 128
    apps = []
    for view, x in ((kv, B_FAKE * 7), (vv, B_FAKE * 8)):
        a = C.AppendParams()
        a.format = C.KVQ_FMT_INT4_SYM
        a.x = x
        a.x_stride_b, a.x_stride_h, a.x_stride_s = H * 128, 128, 128
        a.batch, a.heads, a.seq_new, a.head_dim, a.group_size = B, H, 1, 128, gs
        a.codes = view.codes
        a.codes_stride_b, a.codes_stride_h, a.codes_stride_t = view.stride_b, view.stride_h, view.stride_t
        a.codes_layout = C.KVQ_LAYOUT_ROWS
        a.write_pos, a.capacity = T - 1, T
        a.static_scale = B_FAKE * 9
        a.static_scale_dtype = C.KVQ_DTYPE_F32
        a.static_stride_h, a.static_stride_g = G, 1
        a.rescue_quantile = float(np.float32(1.0 - ratio))
        a.scale_out = view.scale
        a.scale_out_dtype = C.KVQ_DTYPE_F32
        a.so_stride_b, a.so_stride_h, a.so_stride_t, a.so_stride_g = (
            view.scale_stride_b, view.scale_stride_h, view.scale_stride_t, view.scale_stride_g)
        apps.append(a)
    return p, apps[0], apps[1]


def _call(p, k, v):
    L = _lib()
    rc = L.kvq_append_decode_attn(ctypes.byref(p), ctypes.byref(k), ctypes.byref(v), None)
    return rc, L.kvq_last_error().decode()


def test_group_rescue_beyond_the_writer_is_refused():
    # 64 rows: more than the writer wave prefetches (32)
    rc, msg = _call(*_setup(B=16, H=4))
    assert rc == C.KVQ_ERR_UNSUPPORTED and "beyond the writer" in msg, msg
    # 16 rows at the median: the lower rank lies 64 below the top of 128 scales (gs 16: 8 per row)
    rc, msg = _call(*_setup(B=8, H=2, ratio=0.5))
    assert rc == C.KVQ_ERR_UNSUPPORTED and "beyond the writer" in msg, msg


def test_row_append_must_write_the_buffers_the_decode_reads():
    p, k, v = _setup(B=4, H=2)
    k.scale_out = B_FAKE * 10  # not p.k.scale
    rc, msg = _call(p, k, v)
    assert rc == C.KVQ_ERR_UNSUPPORTED and "scale_out must be the scales" in msg, msg
    p, k, v = _setup(B=4, H=2)
    v.codes = B_FAKE * 11
    rc, msg = _call(p, k, v)
    assert rc == C.KVQ_ERR_UNSUPPORTED and "codes must be the buffer" in msg, msg
    p, k, v = _setup(B=4, H=2)
    k.seq_new = 2
    rc, msg = _call(p, k, v)
    assert rc == C.KVQ_ERR_UNSUPPORTED and "one token" in msg, msg


def test_rescue_limits_match_the_engine_rule():
    """The engine's _fused_step_ok and the library agree on which group rescues fuse: the
    same fp32 rank of torch.quantile's lower order statistic, at most 32 rows."""
    from llm_kvcache_quantization_amd.cache import INT4KVCache

    for B, H, gs, ratio in [(8, 4, 16, 0.01), (16, 2, 32, 0.01), (16, 4, 16, 0.01), (8, 2, 16, 0.5),
                            (4, 2, 128, 0.1), (2, 2, 64, 0.3)]:
        eng = INT4KVCache.__new__(INT4KVCache)
        eng.group_size, eng.outlier_rescue_ratio = gs, ratio
        eng.static_k_scale, eng.static_v_scale = object(), None
        fused = eng._fused_step_ok(128, B, H)
        p, k, v = _setup(B=B, H=H, gs=gs, ratio=ratio)
        k.x = B_FAKE * 7 + 2  # misaligned rows: a call past the rescue rule stops in fill_dev
        rc, msg = _call(p, k, v)
        refused = rc == C.KVQ_ERR_UNSUPPORTED and "beyond the writer" in msg
        passed = rc == C.KVQ_ERR_UNSUPPORTED and "4-byte aligned" in msg
        assert refused or passed, (rc, msg)
        assert fused == passed, (B, H, gs, ratio, rc, msg)
