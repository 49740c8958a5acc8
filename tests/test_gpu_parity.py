"""GPU parity: the HIP kernels of libkvq.so against the CPU oracle.

Quantized codes and scales must be bit-exact.  Attention outputs must be within
max-abs 2e-3 of the dequantise-then-attention oracle with cosine >= 0.9999 (the
tolerance BASELINE.json's north star states for fp16 outputs).
"""
import ctypes
import dataclasses
import math

import pytest
import torch

from oracle import attn as OA
from oracle import quant as OQ

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL = 2e-3
COS_MIN = 0.9999


def _lib():
    import llm_kvcache_quantization_amd as K  # noqa: F401
    from llm_kvcache_quantization_amd import _capi

    _capi.lib()
    return K


def assert_close(out: torch.Tensor, ref: torch.Tensor, tag: str):
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert o.shape == r.shape, (tag, o.shape, r.shape)
    assert torch.isfinite(o).all(), tag
    err = (o - r).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r.flatten(), dim=0).item() \
        if r.abs().max() > 0 else 1.0
    print(f"[{tag}] max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= ATOL and cos >= COS_MIN, (tag, err, cos)


def fp16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of fp16 values at |x| (2^(e - 10) for |x| in [2^e, 2^(e+1)), 2^-24 below 2^-14)."""
    a = x.abs().float().clamp(min=2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def assert_close_ulp(out: torch.Tensor, ref: torch.Tensor, tag: str):
    """assert_close for data whose outputs reach |out| >= 4.  There adjacent fp16 values are
    2^-8 = 3.9e-3 apart, more than the 2e-3 bound: two fp32 computations of the same value
    that differ only in summation order round to neighbouring fp16 values whenever the
    value lies near a rounding boundary.  The bound per element is therefore
    max(2e-3, one fp16 ulp of the oracle's value), which is 2e-3 wherever |out| < 4."""
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert o.shape == r.shape, (tag, o.shape, r.shape)
    assert torch.isfinite(o).all(), tag
    err = (o - r).abs()
    bound = torch.maximum(torch.full_like(r, ATOL), fp16_ulp(r))
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r.flatten(), dim=0).item() \
        if r.abs().max() > 0 else 1.0
    worst = (err - bound).max().item()
    print(f"[{tag}] max_abs={err.max().item():.3e} max|ref|={r.abs().max().item():.2f} "
          f"excess_over_bound={worst:.3e} above_2e-3={(err > ATOL).sum().item()} cos={cos:.7f}",
          flush=True)
    assert worst <= 0 and cos >= COS_MIN, (tag, worst, cos)


def gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- append: bit-exact


@pytest.mark.parametrize("mode", ["static_f16", "static_f32", "adaptive", "dynamic"])
@pytest.mark.parametrize("S,gs", [(1, 32), (37, 16), (5, 128)])
def test_append_int8_bitexact(mode, S, gs):
    K = _lib()
    g = gen(11 + S + gs)
    B, H, D = 3, 2, 128
    G = D // gs
    k = (torch.randn(B, H, S, D, generator=g) * 2).to(torch.float16)
    v = torch.randn(B, H, S, D, generator=g).to(torch.float16)
    k[0, 1, 0, 3] = 40.0  # forces clipping for static scales
    st = (torch.rand(1, H, G, generator=g) * 0.02 + 0.005)
    kw = {}
    if mode == "static_f16":
        sk, sv = st.to(torch.float16), (st * 0.5).to(torch.float16)
    elif mode == "static_f32":
        sk, sv = st, st * 0.5
    elif mode == "adaptive":
        sk, sv = st.to(torch.float16), (st * 0.5).to(torch.float16)
        kw = dict(adaptive_static_scales=True, adaptive_static_margin=1.25)
    else:
        sk = sv = None
        kw = dict(clip_percentile=100.0)
    cache = K.INT8KVCache(1, device=DEV, group_size=gs, static_k_scale=sk, static_v_scale=sv,
                          check_numerics=False, **kw)
    cache.append(0, k.to(DEV), v.to(DEV))
    cache.append(0, k.to(DEV), v.to(DEV))  # second append lands at write_pos = S
    kq, vq, ks, vs = cache.get_int8_tensors(0)
    for x, stt, q_gpu, s_gpu, tag in ((k, sk, kq, ks, "k"), (v, sv, vq, vs, "v")):
        ref_q, ref_s = OQ.int8_cache_quantize(
            x, None if stt is None else stt[0], gs, adaptive=(mode == "adaptive"), margin=1.25)
        for rep in range(2):
            got_q = q_gpu[:, :, rep * S:(rep + 1) * S].cpu()
            got_s = s_gpu[:, :, rep * S:(rep + 1) * S].cpu()
            assert torch.equal(got_q, ref_q), (mode, tag, (got_q != ref_q).sum().item())
            assert torch.equal(got_s.float(), ref_s.float()), (mode, tag)


@pytest.mark.parametrize("mode", ["static", "adaptive", "mixed", "rescue", "rescue_all", "dynamic"])
@pytest.mark.parametrize("S", [1, 9])
def test_append_int4_sym_bitexact(mode, S):
    K = _lib()
    g = gen(21 + S)
    B, H, D, gs = 4, 2, 128, 32
    k = (torch.randn(B, H, S, D, generator=g) * 1.5).to(torch.float16)
    v = torch.randn(B, H, S, D, generator=g).to(torch.float16)
    k[1, 0, 0, 70] = 25.0
    v[2, 1, S - 1, 3] = -30.0
    st = torch.rand(H, D // gs, generator=g) * 0.3 + 0.1
    kw = dict(outlier_rescue_ratio=0.0)
    ref_kw = {}
    sk, sv = st, st * 0.8
    if mode == "adaptive":
        kw.update(adaptive_static_scales=True, adaptive_static_margin=0.9)
        ref_kw = dict(adaptive=True, margin=0.9)
    elif mode == "mixed":
        kw.update(mixed_rescue=True)
        ref_kw = dict(mixed_rescue=True)
    elif mode == "rescue":
        kw.update(outlier_rescue_ratio=0.01)
        ref_kw = dict(outlier_rescue_ratio=0.01)
    elif mode == "rescue_all":
        kw.update(outlier_rescue_ratio=1.0)
        ref_kw = dict(outlier_rescue_ratio=1.0)
    elif mode == "dynamic":
        sk = sv = None
        kw.update(clip_percentile=100.0)
    cache = K.INT4KVCache(1, device=DEV, group_size=gs, static_k_scale=None if sk is None else sk[None],
                          static_v_scale=None if sv is None else sv[None], check_numerics=False, **kw)
    cache.append(0, k.to(DEV), v.to(DEV))
    kp, vp, ks, vs = cache.get_int4_tensors(0)
    for x, stt, p_gpu, s_gpu, tag in ((k, sk, kp, ks, "k"), (v, sv, vp, vs, "v")):
        ref_q, ref_s = OQ.int4_cache_quantize(x, stt, gs, **ref_kw)
        assert torch.equal(p_gpu.cpu(), OQ.pack_int4(ref_q)), (mode, tag)
        assert torch.equal(s_gpu.cpu().float(), ref_s.float()), (mode, tag)


@pytest.mark.parametrize("B,H,S,ratio,ties,gs", [
    (2, 4, 2048, 0.01, False, 32),    # 65,536 scales: the radix-select path
    (1, 2, 600, 0.3, True, 32),       # 4,800 scales, many equal (ties at the threshold)
    (4, 2, 4096, 0.001, False, 32),   # 131,072 scales, a threshold in the far tail
    (2, 2, 256, 0.05, False, 32),     # 4,096 scales: the one-work-group sort path
    (40, 8, 1, 0.01, True, 32),       # 1,280 scales: the one-work-group walk from the top
    (8, 4, 1, 0.01, False, 32),       # a decode step (128 scales): rank counting
    (16, 4, 1, 0.01, True, 32),       # 64 rows, ties
    (8, 4, 1, 0.1, False, 32),        # 13 ranks below the top
    (4, 2, 16, 0.05, True, 32),       # 512 scales, 26 ranks below the top, ties
    (8, 4, 1, 0.01, False, 16),       # config 3's decode step at group 16 (256 scales)
    (3, 3, 1, 0.2, False, 128),       # 9 rows and 9 scales (not a multiple of 4)
    (32, 8, 1, 0.01, True, 32),       # 1,024 scales: the most that are rank-counted
    (2, 2, 7, 0.5, True, 16),         # the median, ties: counted ranks
    (16, 8, 1, 0.3, True, 32),        # 512 scales, 154 ranks below the top: counted ranks
])
def test_append_int4_rescue_large_bitexact(B, H, S, ratio, ties, gs):
    """INT4 group outlier rescue over the dynamic scales of an append: the torch.quantile
    threshold (int4_cache.py:384-390) by the radix select in the scratch buffer (more than
    4096 scales), one work-group's LDS sort or walk from the top (1025-4096), or rank
    counting in every work-group (at most 1024), codes and scales bit-exact."""
    K = _lib()
    from llm_kvcache_quantization_amd import _capi as C

    g = gen(3000 + S)
    D = 128
    k = (torch.randn(B, H, S, D, generator=g) * 1.5).to(torch.float16)
    v = torch.randn(B, H, S, D, generator=g).to(torch.float16)
    if ties:  # few distinct group absmax values
        k = (k * 4).round().div(4).to(torch.float16)
        v = (v * 2).round().div(2).to(torch.float16)
    k[0, 1, min(7, S - 1), 70] = 25.0
    st = torch.rand(H, D // gs, generator=g) * 0.3 + 0.1
    cache = K.INT4KVCache(1, device=DEV, group_size=gs, static_k_scale=st[None],
                          static_v_scale=(st * 0.8)[None], check_numerics=False,
                          outlier_rescue_ratio=ratio)
    p = C.AppendParams()
    p.format, p.batch, p.heads, p.seq_new, p.group_size = C.KVQ_FMT_INT4_SYM, B, H, S, gs
    p.static_scale, p.rescue_quantile = 1, float(torch.tensor(1.0 - ratio, dtype=torch.float32))
    n = B * H * S * (D // gs)
    assert (C.lib().kvq_append_scratch_bytes(ctypes.byref(p)) > 0) == (n > 4096)
    cache.append(0, k.to(DEV), v.to(DEV))
    kp, vp, ks, vs = cache.get_int4_tensors(0)
    for x, stt, p_gpu, s_gpu, tag in ((k, st, kp, ks, "k"), (v, st * 0.8, vp, vs, "v")):
        ref_q, ref_s = OQ.int4_cache_quantize(x, stt, gs, outlier_rescue_ratio=ratio)
        assert torch.equal(s_gpu.cpu().float(), ref_s.float()), (tag, n)
        assert torch.equal(p_gpu.cpu(), OQ.pack_int4(ref_q)), (tag, n)


@pytest.mark.parametrize("outliers", [False, True])
def test_append_asym_bitexact(outliers):
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[3]
    tables = SY.calibrate(cfg, 0)
    g = gen(31)
    k, v = SY.draw_kv(cfg, 0, 3, 19, g)
    oidx = tables.k_outlier_idx if outliers else None
    L = 1
    cache = K.INT4AsymKVCache(L, tables.k_scale[None], tables.k_zp[None], tables.v_scale[None],
                              tables.v_zp[None], device=DEV,
                              k_outlier_idx=None if oidx is None else oidx[None])
    cache.append(0, k[:, :, :7].to(DEV), v[:, :, :7].to(DEV))
    cache.append(0, k[:, :, 7:].to(DEV), v[:, :, 7:].to(DEV))
    kc, vc, *_rest, ko = cache.get_int4_g32_tensors(0)
    ref_k = OQ.pack_int4(OQ.quantize_asymmetric_static(k, tables.k_scale, tables.k_zp)).view(torch.uint8)
    ref_v = OQ.pack_int4(OQ.quantize_asymmetric_static(v, tables.v_scale, tables.v_zp)).view(torch.uint8)
    assert torch.equal(kc.cpu(), ref_k)
    assert vc.shape[-1] == K.kernels.TILE_BYTES  # the engine keeps V in the TILE32 layout
    assert torch.equal(K.untile_v(vc, 19).cpu(), ref_v)  # slots past 19 are unwritten
    if outliers:
        ref_o = torch.stack([k[:, h, :, oidx[h].long()] for h in range(cfg.kv_heads)], dim=1)
        assert torch.equal(ko.cpu(), ref_o)


def test_append_nan_raises_and_does_not_advance():
    K = _lib()
    cache = K.INT8KVCache(1, device=DEV, group_size=32,
                          static_k_scale=torch.full((1, 2, 4), 0.01, dtype=torch.float16),
                          static_v_scale=torch.full((1, 2, 4), 0.01, dtype=torch.float16))
    x = torch.randn(1, 2, 1, 128, dtype=torch.float16, device=DEV)
    cache.append(0, x, x)
    bad = x.clone()
    bad[0, 1, 0, 9] = float("nan")
    with pytest.raises(ValueError):
        cache.append(0, bad, x)
    assert cache.get_seq_len() == 1
    big = x * 100
    with pytest.warns(RuntimeWarning):
        cache.append(0, big, x)


# ---------------------------------------------------------------- decode: tolerance parity


def _rand_int8_case(B, Hq, Hkv, S, G, g):
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
    k = torch.randint(-128, 128, (B, Hkv, S, 128), generator=g, dtype=torch.int8)
    v = torch.randint(-128, 128, (B, Hkv, S, 128), generator=g, dtype=torch.int8)
    ks = (torch.rand(B, Hkv, S, G, generator=g) * 0.01 + 1e-3).to(torch.float16)
    vs = (torch.rand(B, Hkv, S, G, generator=g) * 0.01 + 1e-3).to(torch.float16)
    return q, k, v, ks, vs


@pytest.mark.parametrize("B,Hq,Hkv,S,G,ctx", [
    (1, 12, 2, 4096, 4, [4096]),
    (3, 12, 2, 700, 4, [700, 37, 0]),
    (2, 8, 2, 513, 8, [1, 513]),
    (2, 7, 7, 300, 1, [129, 300]),
    (4, 16, 1, 2048, 2, [2048, 2047, 1000, 31]),
])
def test_decode_int8_parity(B, Hq, Hkv, S, G, ctx):
    K = _lib()
    g = gen(B * 1000 + S)
    q, k, v, ks, vs = _rand_int8_case(B, Hq, Hkv, S, G, g)
    cl = torch.tensor(ctx, dtype=torch.int32)
    sm = 1 / math.sqrt(128)
    ref = OA.decode_attn_int8_torch_ref(q, k, v, ks, vs, cl, sm)
    stats = {}
    out = K.decode_attn_int8(q.to(DEV), k.to(DEV), v.to(DEV), ks.to(DEV), vs.to(DEV), cl.to(DEV),
                             sm_scale=sm, debug_stats=stats, layer_idx=3)
    assert_close(out, ref, f"int8 B{B} Hq{Hq} Hkv{Hkv} S{S} G{G}")
    for b, c in enumerate(ctx):
        if c == 0:
            assert torch.all(out[b] == 0)
    assert stats["triton_kernel_calls"] == 1 and stats["triton_layer_hits"] == {"3": 1}


def test_decode_int8_static_expanded_scales_and_fp32_q():
    K = _lib()
    g = gen(77)
    B, Hq, Hkv, S = 2, 12, 2, 1000
    q, k, v, _, _ = _rand_int8_case(B, Hq, Hkv, S, 4, g)
    st = (torch.rand(Hkv, 4, generator=g) * 0.01 + 1e-3).to(torch.float16)
    ks = st[None, :, None, :].expand(B, Hkv, S, 4)
    cl = torch.tensor([S, 999], dtype=torch.int32)
    ref = OA.decode_attn_int8_torch_ref(q, k, v, ks, ks, cl, 0.1)
    out = K.decode_attn_int8(q.float().to(DEV), k.to(DEV), v.to(DEV), ks.to(DEV), ks.to(DEV),
                             cl.to(DEV), sm_scale=0.1)
    assert out.dtype == torch.float32
    assert_close(out, ref.float(), "int8 static-expanded")


def _static_int8_case(B, Hq, Hkv, S, g, scale_dtype=torch.float16, G=4):
    """Codes and static scales (G groups per head) as INT8KVCache stores them: per-token
    scale views with stride 0 over b and t, which the tiled INT8 kernels serve."""
    q, k, v, _, _ = _rand_int8_case(B, Hq, Hkv, S, G, g)
    sk = (torch.rand(Hkv, G, generator=g) * 0.01 + 1e-3).to(scale_dtype)
    sv = (torch.rand(Hkv, G, generator=g) * 0.02 + 1e-3).to(scale_dtype)
    ks = sk[None, :, None, :].expand(B, Hkv, S, G)
    vs = sv[None, :, None, :].expand(B, Hkv, S, G)
    return q, k, v, ks, vs


@pytest.mark.parametrize("B,Hq,Hkv,S,ctx", [
    (4, 12, 2, 8192, [8192, 8191, 4097, 33]),    # config 1 shape, ragged, partial tiles
    (3, 12, 2, 700, [700, 1, 0]),                 # a single token and an empty row
    (2, 32, 2, 1000, [1000, 999]),                # 16 query heads per kv head (no packing)
    (2, 40, 8, 300, [300, 64]),                   # GQA 5
])
def test_decode_int8_static_tiled(B, Hq, Hkv, S, ctx):
    """Static-scale INT8 K and V (the tiled INT8 kernel) against the oracle."""
    K = _lib()
    g = gen(31 * S + Hq)
    q, k, v, ks, vs = _static_int8_case(B, Hq, Hkv, S, g)
    cl = torch.tensor(ctx, dtype=torch.int32)
    sm = 1 / math.sqrt(128)
    ref = OA.decode_attn_int8_torch_ref(q, k, v, ks, vs, cl, sm)
    out = K.decode_attn_int8(q.to(DEV), k.to(DEV), v.to(DEV), ks.to(DEV), vs.to(DEV), cl.to(DEV),
                             sm_scale=sm)
    assert_close(out, ref, f"int8 static tiled B{B} Hq{Hq} Hkv{Hkv} S{S}")
    for b, c in enumerate(ctx):
        if c == 0:
            assert torch.all(out[b] == 0)


def test_cfg1_every_layer():
    """Configuration 1 (Qwen2.5-1.5B shape, INT8 static g32 tables, B 4, 8k) on each of its 28
    layers: that layer's seeded K / V and calibration tables, the cache built by the HIP
    append (INT8KVCache), then one fused decode step (append of token 8192 + attention) with
    the layer's inverse temperatures.  Codes of the new token bit-exact with the oracle's
    quantizer; outputs of rows 0 and 3 within the bound of the oracle's attention."""
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[1]
    taus = SY.inv_tau(cfg)
    S, B = cfg.context, cfg.batch
    sm = 1 / math.sqrt(128)
    for layer in range(cfg.layers):
        t = SY.calibrate(cfg, layer)
        g = gen(SY.seed_for(1, layer))
        k, v = SY.draw_kv(cfg, layer, B, S, g)
        q = SY.draw_q(cfg, B, g)
        cache = K.INT8KVCache(1, device=DEV, group_size=32, static_k_scale=t.k_scale[None].to(DEV),
                              static_v_scale=t.v_scale[None].to(DEV), check_numerics=False)
        cache.append(0, k[:, :, :S - 1].to(DEV), v[:, :, :S - 1].to(DEV))
        out = cache.append_decode_attn(0, q.to(DEV), k[:, :, S - 1:].to(DEV), v[:, :, S - 1:].to(DEV),
                                       sm, inv_tau=taus[layer].to(DEV))
        kc, vc, ks, vs = [x.cpu() for x in cache.get_int8_tensors(0)]
        rk, _ = OQ.quantize_symmetric_int8_with_scale(k[:, :, S - 1:], t.k_scale, 32)
        rv, _ = OQ.quantize_symmetric_int8_with_scale(v[:, :, S - 1:], t.v_scale, 32)
        assert torch.equal(kc[:, :, S - 1:], rk) and torch.equal(vc[:, :, S - 1:], rv), layer
        rows = [0, 3]
        ref = OA.decode_attn_int8_torch_ref(OA.prescale_q(q[rows], taus[layer]), kc[rows], vc[rows],
                                            ks[rows], vs[rows], torch.full((2,), S, dtype=torch.int32), sm)
        assert_close(out[rows], ref, f"cfg1 layer {layer}")


@pytest.mark.parametrize("G,B,Hq,Hkv,S,ctx", [
    (8, 4, 12, 2, 8192, [8192, 8191, 4097, 33]),   # group 16 (the shipped int8_ours tables)
    (16, 3, 12, 2, 700, [700, 1, 0]),              # group 8
    (2, 2, 28, 4, 1000, [1000, 999]),              # group 64
    (1, 2, 40, 8, 300, [300, 64]),                 # group 128, GQA 5
])
def test_decode_int8_static_tiled_group_sizes(G, B, Hq, Hkv, S, ctx):
    """Static INT8 tables of every group size the engines take (the tiled INT8 kernel reads
    one scale per 8-channel slice) against the oracle, with per-head inverse temperature."""
    K = _lib()
    g = gen(77 * S + G)
    q, k, v, ks, vs = _static_int8_case(B, Hq, Hkv, S, g, G=G)
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    cl = torch.tensor(ctx, dtype=torch.int32)
    sm = 1 / math.sqrt(128)
    ref = OA.decode_attn_int8_torch_ref(OA.prescale_q(q, tau), k, v, ks, vs, cl, sm)
    out = K.decode_attn_int8(OA.prescale_q(q, tau).to(DEV), k.to(DEV), v.to(DEV), ks.to(DEV),
                             vs.to(DEV), cl.to(DEV), sm_scale=sm)
    assert_close(out, ref, f"int8 static tiled G{G} B{B} Hq{Hq} Hkv{Hkv} S{S}")
    for b, c in enumerate(ctx):
        if c == 0:
            assert torch.all(out[b] == 0)


def test_decode_int8_static_tiled_f32_scales_inv_tau_and_splits():
    """fp32 static scales (rounded to fp16 in the kernel, as the reference's fp16 cast),
    per-head inverse temperature, split-size invariance and bit-exact repeats."""
    K = _lib()
    from llm_kvcache_quantization_amd import _capi as C
    from llm_kvcache_quantization_amd.kernels import DecodePlan, kv_view_tok

    g = gen(5150)
    B, Hq, Hkv, S = 2, 12, 2, 5000
    q, k, v, ks, vs = _static_int8_case(B, Hq, Hkv, S, g, torch.float32)
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    cl = torch.tensor([5000, 2222], dtype=torch.int32)
    sm = 1 / math.sqrt(128)
    ref = OA.decode_attn_int8_torch_ref(OA.prescale_q(q, tau), k, v, ks.to(torch.float16),
                                        vs.to(torch.float16), cl, sm)
    d = lambda x: x.to(DEV)
    outs = []
    for chunk in (0, 256, 1024):
        plan = DecodePlan(d(q), C.KVQ_FMT_INT8_SYM, kv_view_tok(d(k), d(ks)), C.KVQ_FMT_INT8_SYM,
                          kv_view_tok(d(v), d(vs)), d(cl), Hkv, S, sm, 32, inv_tau=d(tau),
                          chunk_tokens=chunk)
        a = plan.launch().clone()
        b = plan.launch().clone()
        assert torch.equal(a, b), chunk
        assert_close(a, ref, f"int8 static f32 chunk={chunk}")
        outs.append(a.cpu())


@pytest.mark.parametrize("B,S,ctx", [
    (3, 3000, [3000, 1234, 1]),
    (8, 4096, [4096, 4000, 3001, 2048, 1025, 512, 33, 0]),
])
def test_decode_k8v4_tiled_ragged(B, S, ctx):
    """INT8 K (static) with TILE32 asymmetric INT4 V (the tiled K8/V4 kernel), config 4's
    heads (GQA 5), ragged contexts."""
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[4]
    t = SY.calibrate(cfg, 0)
    g = gen(40 + B)
    k, v = SY.draw_kv(cfg, 0, B, S, g)
    q = SY.draw_q(cfg, B, g)
    tau = SY.inv_tau(cfg)[0]
    k8, ks16 = OQ.quantize_symmetric_int8_with_scale(k, t.k_scale, 32)
    vq = OQ.pack_int4(OQ.quantize_asymmetric_static(v, t.v_scale, t.v_zp))
    cl = torch.tensor(ctx, dtype=torch.int32)
    ref = OA.decode_attn_k8v4_ref(q, k8, ks16, vq, t.v_scale, t.v_zp, cl, 0.0883883, inv_tau=tau)
    # the static table as a stride-0 per-token view (what the tiled kernel serves)
    ks_view = t.k_scale.clamp(min=1e-5).to(torch.float16).to(DEV)[None, :, None, :].expand(
        B, cfg.kv_heads, S, 4)
    assert torch.equal(ks_view.cpu(), ks16)
    out = K.decode_attn_k8v4(q.to(DEV), k8.to(DEV), ks_view, K.tile_v(vq.to(DEV)),
                             t.v_scale.to(DEV), t.v_zp.to(DEV), cl.to(DEV), 0.0883883,
                             inv_tau=tau.to(DEV))
    assert_close(out, ref, f"k8v4 tiled B{B} S{S}")
    for b, c in enumerate(ctx):
        if c == 0:
            assert torch.all(out[b] == 0)


@pytest.mark.parametrize("B,Hq,Hkv,S,ctx", [
    (2, 12, 2, 2048, [2048, 1500]),
    (1, 28, 4, 4096, [4096]),
    (3, 6, 1, 257, [1, 0, 257]),
])
def test_decode_int4_packed_parity(B, Hq, Hkv, S, ctx):
    K = _lib()
    g = gen(S + B)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
    kc = torch.randint(-8, 8, (B, Hkv, S, 128), generator=g, dtype=torch.int8)
    vc = torch.randint(-8, 8, (B, Hkv, S, 128), generator=g, dtype=torch.int8)
    ks = (torch.rand(B, Hkv, S, 4, generator=g) * 0.3 + 0.01).to(torch.float16)
    vs = (torch.rand(B, Hkv, S, 4, generator=g) * 0.3 + 0.01).to(torch.float16)
    kp, vp = OQ.pack_int4(kc), OQ.pack_int4(vc)
    cl = torch.tensor(ctx, dtype=torch.int32)
    ref = OA.decode_attn_int4_torch_ref(q, kp, vp, ks, vs, cl, 0.0883883)
    out = K.decode_attn_int4(q.to(DEV), kp.to(DEV), vp.to(DEV), ks.to(DEV), vs.to(DEV), cl.to(DEV),
                             sm_scale=0.0883883, bit_packed=True, head_dim=128)
    assert_close(out, ref, f"int4 packed B{B} S{S}")
    # unpacked int8 codes take the INT8 kernel, as in the reference wrapper
    out_u = K.decode_attn_int4(q.to(DEV), kc.to(DEV), vc.to(DEV), ks.to(DEV), vs.to(DEV),
                               cl.to(DEV), sm_scale=0.0883883, bit_packed=False)
    assert_close(out_u, ref, f"int4 unpacked B{B} S{S}")


@pytest.mark.parametrize("bits,G,B,Hq,Hkv,S,ctx,static", [
    (8, 8, 3, 12, 2, 700, [700, 37, 0], False),        # groups of 16, an empty row
    (8, 1, 2, 28, 4, 1000, [1000, 999], False),        # groups of 128 (int8_baseline)
    (8, 4, 2, 32, 2, 513, [1, 513], False),            # 16 query heads per kv head
    (4, 8, 4, 12, 2, 8192, [8192, 8191, 4097, 33], False),  # int4_fused: groups of 16, fp32
    (4, 4, 2, 40, 8, 300, [300, 64], False),           # groups of 32 (int4_baseline), GQA 5
    (4, 2, 3, 6, 1, 257, [1, 0, 257], False),          # groups of 64
    (4, 8, 2, 28, 4, 1000, [1000, 555], True),         # a static fp32 table (stride-0 view)
])
def test_decode_per_token_scales_tiled(bits, G, B, Hq, Hkv, S, ctx, static):
    """Per-token scales (INT8 with fp16, packed INT4 with fp32 scales, the engines' dtypes):
    the tiled kernel against the oracle, with per-head inverse temperature.  Scales of the
    tokens past each row's context are NaN, as unwritten cache memory may be."""
    K = _lib()
    g = gen(1000 * bits + 10 * G + S)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
    lo = -127 if bits == 8 else -7
    kc = torch.randint(lo, -lo + 1, (B, Hkv, S, 128), generator=g, dtype=torch.int8)
    vc = torch.randint(lo, -lo + 1, (B, Hkv, S, 128), generator=g, dtype=torch.int8)
    sdt = torch.float16 if bits == 8 else torch.float32
    amp = 0.01 if bits == 8 else 0.3
    if static:
        kt = (torch.rand(Hkv, G, generator=g) * amp + 1e-3).to(sdt)
        vt = (torch.rand(Hkv, G, generator=g) * amp + 1e-3).to(sdt)
        ks = kt[None, :, None, :].expand(B, Hkv, S, G)
        vs = vt[None, :, None, :].expand(B, Hkv, S, G)
    else:
        ks = (torch.rand(B, Hkv, S, G, generator=g) * amp + 1e-3).to(sdt)
        vs = (torch.rand(B, Hkv, S, G, generator=g) * amp + 1e-3).to(sdt)
        for b, c in enumerate(ctx):
            ks[b, :, c:] = float("nan")
            vs[b, :, c:] = float("nan")
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    cl = torch.tensor(ctx, dtype=torch.int32)
    sm = 1 / math.sqrt(128)
    qs = OA.prescale_q(q, tau)
    d = lambda x: x.to(DEV)
    from llm_kvcache_quantization_amd import _capi as C
    from llm_kvcache_quantization_amd.kernels import DecodePlan, kv_view_tok

    if bits == 8:
        ref = OA.decode_attn_int8_torch_ref(qs, kc, vc, ks, vs, cl, sm)
        kx, vx, fmt = kc, vc, C.KVQ_FMT_INT8_SYM
    else:
        kx, vx, fmt = OQ.pack_int4(kc), OQ.pack_int4(vc), C.KVQ_FMT_INT4_SYM
        ref = OA.decode_attn_int4_torch_ref(qs, kx, vx, ks, vs, cl, sm)
    # the engines' call (fp32 INT4 scales are rounded to fp16 in the kernel, as the
    # reference casts them before its kernel)
    if static:  # stride 0 over b and t on the device too
        ksd = kt.to(DEV)[None, :, None, :].expand(B, Hkv, S, G)
        vsd = vt.to(DEV)[None, :, None, :].expand(B, Hkv, S, G)
    else:
        ksd, vsd = d(ks), d(vs)
    plan = DecodePlan(d(q), fmt, kv_view_tok(d(kx), ksd), fmt, kv_view_tok(d(vx), vsd), d(cl),
                      Hkv, S, sm, 128 // G, inv_tau=d(tau))
    out = plan.launch().clone()
    assert torch.equal(out, plan.launch()), "repeated launches differ"
    assert_close(out, ref, f"per-token int{bits} G{G} B{B} Hq{Hq} Hkv{Hkv} S{S} static={static}")
    if not static:
        # the same V scales in rows padded to G + 4 values (not dense): the kernel then gathers
        # the V operands with per-lane loads instead of 16-byte loads through LDS; the
        # operands, and so the bits, are the same
        vpad = torch.full((B, Hkv, S, G + 4), float("nan"), dtype=sdt, device=DEV)
        vpad[..., :G] = vsd
        plan2 = DecodePlan(d(q), fmt, kv_view_tok(d(kx), ksd), fmt, kv_view_tok(d(vx), vpad[..., :G]),
                           d(cl), Hkv, S, sm, 128 // G, inv_tau=d(tau))
        assert torch.equal(plan2.launch(), out), "V gathered through LDS and by dword loads differ"
    if bits == 8 and not static:  # the public entry point takes the same kernel
        pub = K.decode_attn_int8(d(qs), d(kc), d(vc), d(ks), d(vs), d(cl), sm_scale=sm)
        assert_close(pub, ref, f"decode_attn_int8 per-token G{G}")
    for b, c in enumerate(ctx):
        if c == 0:
            assert torch.all(out[b] == 0)


def _asym_case(cfg_idx, B, S, ctx, seed, outliers=True, heads=None):
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[cfg_idx]
    if heads is not None:  # (q heads, kv heads) in place of the configuration's
        cfg = dataclasses.replace(cfg, q_heads=heads[0], kv_heads=heads[1])
    t = SY.calibrate(cfg, 0)
    g = gen(seed)
    k, v = SY.draw_kv(cfg, 0, B, S, g)
    q = SY.draw_q(cfg, B, g)
    tau = SY.inv_tau(cfg)[0]
    kq = OQ.pack_int4(OQ.quantize_asymmetric_static(k, t.k_scale, t.k_zp))
    vq = OQ.pack_int4(OQ.quantize_asymmetric_static(v, t.v_scale, t.v_zp))
    oidx = t.k_outlier_idx if outliers else None
    oval = None
    if outliers:
        oval = torch.stack([k[:, h, :, oidx[h].long()] for h in range(cfg.kv_heads)], dim=1).contiguous()
    cl = torch.tensor(ctx, dtype=torch.int32)
    return cfg, t, q, tau, kq, vq, oidx, oval, cl


@pytest.mark.parametrize("layout", ["rows", "tile32"])
@pytest.mark.parametrize("cfg_idx,B,S,ctx,outliers", [
    (3, 2, 4096, [4096, 3001], True),
    (2, 3, 2048, [2048, 1, 777], True),
    (3, 1, 1000, [1000], False),
    (3, 2, 300, [0, 300], True),
    (3, 2, 45, [45, 33], True),
])
def test_decode_asym_parity(cfg_idx, B, S, ctx, outliers, layout):
    K = _lib()
    cfg, t, q, tau, kq, vq, oidx, oval, cl = _asym_case(cfg_idx, B, S, ctx, 40 + S, outliers)
    sm = 1 / math.sqrt(128)
    ref = OA.decode_attn_asym_ref(q, kq, vq, t.k_scale, t.k_zp, t.v_scale, t.v_zp, cl, sm,
                                  inv_tau=tau, k_outlier_idx=oidx, k_outlier_val=oval)
    d = lambda x: None if x is None else x.to(DEV)
    vd = K.tile_v(vq.to(DEV)) if layout == "tile32" else vq.to(DEV)
    out = K.decode_attn_int4_asym(q.to(DEV), kq.to(DEV), vd, d(t.k_scale), d(t.k_zp),
                                  d(t.v_scale), d(t.v_zp), cl.to(DEV), sm, inv_tau=tau.to(DEV),
                                  k_outlier_idx=d(oidx), k_outlier_val=d(oval))
    assert_close(out, ref, f"asym {layout} cfg{cfg_idx} B{B} S{S} out={outliers}")


def test_decode_k8v4_parity_ragged():
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[4]
    t = SY.calibrate(cfg, 0)
    g = gen(4)
    B, S = 3, 3000
    k, v = SY.draw_kv(cfg, 0, B, S, g)
    q = SY.draw_q(cfg, B, g)
    tau = SY.inv_tau(cfg)[0]
    k8, ks16 = OQ.quantize_symmetric_int8_with_scale(k, t.k_scale, 32)
    vq = OQ.pack_int4(OQ.quantize_asymmetric_static(v, t.v_scale, t.v_zp))
    cl = torch.tensor([3000, 1234, 4097 - 4096], dtype=torch.int32)
    ref = OA.decode_attn_k8v4_ref(q, k8, ks16, vq, t.v_scale, t.v_zp, cl, 0.0883883, inv_tau=tau)
    out = K.decode_attn_k8v4(q.to(DEV), k8.to(DEV), ks16.to(DEV), vq.to(DEV), t.v_scale.to(DEV),
                             t.v_zp.to(DEV), cl.to(DEV), 0.0883883, inv_tau=tau.to(DEV))
    assert_close(out, ref, "k8v4 ragged")


def test_decode_kat_single_token_and_zero_context():
    K = _lib()
    B, H, S = 2, 4, 64
    q = torch.randn(B, H, 128, dtype=torch.float16)
    k = torch.randint(-5, 5, (B, H, S, 128), dtype=torch.int8)
    v = torch.randint(-100, 100, (B, H, S, 128), dtype=torch.int8)
    s = torch.ones(B, H, S, 4, dtype=torch.float16)
    cl = torch.tensor([1, 0], dtype=torch.int32)
    out = K.decode_attn_int8(q.to(DEV), k.to(DEV), v.to(DEV), s.to(DEV), s.to(DEV), cl.to(DEV))
    assert torch.equal(out[0].cpu(), v[0, :, 0].to(torch.float16))  # one token: output = V
    assert torch.all(out[1] == 0)
    allzero = K.decode_attn_int8(q.to(DEV), k.to(DEV), v.to(DEV), s.to(DEV), s.to(DEV),
                                 torch.zeros(2, dtype=torch.int32, device=DEV))
    assert torch.all(allzero == 0)


@pytest.mark.parametrize("layout", ["rows", "tile32"])
def test_decode_split_invariance_and_determinism(layout):
    """Results do not depend on the split size beyond tolerance and repeat bit-exactly."""
    K = _lib()
    from llm_kvcache_quantization_amd import _capi as C
    from llm_kvcache_quantization_amd.kernels import DecodePlan, kv_view_static

    cfg, t, q, tau, kq, vq, oidx, oval, cl = _asym_case(3, 2, 8192, [8192, 5000], 5)
    d = lambda x: x.to(DEV)
    vd = K.tile_v(d(vq)) if layout == "tile32" else d(vq)
    outs = []
    for chunk in (128, 256, 1024, 4096, 8192):
        plan = DecodePlan(d(q), C.KVQ_FMT_INT4_ASYM,
                          kv_view_static(d(kq), d(t.k_scale), d(t.k_zp), d(oidx), d(oval)),
                          C.KVQ_FMT_INT4_ASYM, kv_view_static(vd, d(t.v_scale), d(t.v_zp)),
                          d(cl), cfg.kv_heads, 8192, 1 / math.sqrt(128), 32, inv_tau=d(tau),
                          chunk_tokens=chunk)
        a = plan.launch().clone()
        b = plan.launch().clone()
        assert torch.equal(a, b), chunk
        outs.append(a.cpu())
    for o in outs[1:]:
        assert (o.float() - outs[0].float()).abs().max() <= ATOL


def test_cfg3_full_size_rows():
    """One layer at the headline shape (B=8, Hq=28, Hkv=4, 32768 tokens) built by the HIP
    append kernel; rows 0 and 7 are checked against the oracle."""
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[3]
    t = SY.calibrate(cfg, 0)
    g = torch.Generator(device=DEV).manual_seed(SY.seed_for(3, 0))
    k, v = SY.draw_kv(cfg, 0, cfg.batch, cfg.context, g, device=DEV)
    q = SY.draw_q(cfg, cfg.batch, g, device=DEV)
    tau = SY.inv_tau(cfg)[0].to(DEV)
    cache = K.INT4AsymKVCache(1, t.k_scale[None], t.k_zp[None], t.v_scale[None], t.v_zp[None],
                              device=DEV, k_outlier_idx=t.k_outlier_idx[None])
    cache.append(0, k, v)
    kc, vc, ks, kz, vs, vz, oi, ov = cache.get_int4_g32_tensors(0)
    cl = torch.full((cfg.batch,), cfg.context, dtype=torch.int32, device=DEV)
    out = K.decode_attn_int4_asym(q, kc, vc, ks, kz, vs, vz, cl, 1 / math.sqrt(128), inv_tau=tau,
                                  k_outlier_idx=oi, k_outlier_val=ov)
    for b in (0, cfg.batch - 1):
        sl = slice(b, b + 1)
        kq_ref = OQ.pack_int4(OQ.quantize_asymmetric_static(k[sl].cpu(), t.k_scale, t.k_zp))
        assert torch.equal(kc[sl].cpu(), kq_ref.view(torch.uint8))
        ref = OA.decode_attn_asym_ref(q[sl].cpu(), kc[sl].cpu(), K.untile_v(vc[sl], cfg.context).cpu(),
                                      t.k_scale, t.k_zp, t.v_scale, t.v_zp, cl[sl].cpu(),
                                      1 / math.sqrt(128),
                                      inv_tau=tau.cpu(), k_outlier_idx=t.k_outlier_idx,
                                      k_outlier_val=ov[sl].cpu())
        assert_close(out[sl], ref, f"cfg3 full row {b}")
        vq_ref = OQ.pack_int4(OQ.quantize_asymmetric_static(v[sl].cpu(), t.v_scale, t.v_zp))
        assert torch.equal(K.untile_v(vc[sl], cfg.context).cpu(), vq_ref.view(torch.uint8))


def test_cfg2_full_size_rows():
    """Config 2 at full size (B=16, Hq=12, Hkv=2, 32768 tokens, 4 fp16 K channels) through
    the fused decode step: K, V and outlier-channel codes of rows 0 and 15 bit-exact, their
    outputs against the oracle."""
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[2]
    t = SY.calibrate(cfg, 0)
    g = torch.Generator(device=DEV).manual_seed(SY.seed_for(2, 0))
    S = cfg.context
    k, v = SY.draw_kv(cfg, 0, cfg.batch, S, g, device=DEV)
    q = SY.draw_q(cfg, cfg.batch, g, device=DEV)
    tau = SY.inv_tau(cfg)[0].to(DEV)
    cache = K.INT4AsymKVCache(1, t.k_scale[None], t.k_zp[None], t.v_scale[None], t.v_zp[None],
                              device=DEV, k_outlier_idx=t.k_outlier_idx[None], inv_tau=tau[None])
    cache.append(0, k[:, :, :S - 1].contiguous(), v[:, :, :S - 1].contiguous())
    out = cache.append_decode_attn(0, q, k[:, :, S - 1:], v[:, :, S - 1:], 1 / math.sqrt(128),
                                   inv_tau=tau)
    kc, vc, ks, kz, vs, vz, oi, ov = cache.get_int4_g32_tensors(0)
    cl = torch.full((1,), S, dtype=torch.int32)
    for b in (0, cfg.batch - 1):
        sl = slice(b, b + 1)
        kq_ref = OQ.pack_int4(OQ.quantize_asymmetric_static(k[sl].cpu(), t.k_scale, t.k_zp))
        vq_ref = OQ.pack_int4(OQ.quantize_asymmetric_static(v[sl].cpu(), t.v_scale, t.v_zp))
        vr = K.untile_v(vc[sl], S).cpu()
        assert torch.equal(kc[sl].cpu(), kq_ref.view(torch.uint8)), b
        assert torch.equal(vr, vq_ref.view(torch.uint8)), b
        idx = t.k_outlier_idx.long()
        want_o = torch.stack([k[b, h, :, idx[h]].cpu() for h in range(cfg.kv_heads)])[None]
        assert torch.equal(ov[sl].cpu(), want_o), b
        ref = OA.decode_attn_asym_ref(q[sl].cpu(), kc[sl].cpu(), vr, t.k_scale, t.k_zp, t.v_scale, t.v_zp,
                                      cl, 1 / math.sqrt(128), inv_tau=tau.cpu(),
                                      k_outlier_idx=t.k_outlier_idx, k_outlier_val=ov[sl].cpu())
        assert_close(out[sl], ref, f"cfg2 full row {b}")


def test_cfg4_full_size_rows():
    """Config 4 at full size (B=8, Hq=40, Hkv=8, K INT8 / V INT4 g32) with ragged contexts:
    the seeded draw with rows 0 and 1 set to the distribution's bounds, 65536 and 4096
    tokens (the 65536-token row merges 16 chunks of 4096).  Rows 0, 1 and the longest
    seeded row: codes bit-exact, outputs against the oracle."""
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[4]
    t = SY.calibrate(cfg, 0)
    ctx = SY.context_lengths(cfg)
    ctx[0], ctx[1] = cfg.context, cfg.ragged_min
    S = cfg.context
    g = torch.Generator(device=DEV).manual_seed(SY.seed_for(4, 0))
    k, v = SY.draw_kv(cfg, 0, cfg.batch, S, g, device=DEV)
    q = SY.draw_q(cfg, cfg.batch, g, device=DEV)
    tau = SY.inv_tau(cfg)[0].to(DEV)
    cache = K.K8V4KVCache(1, t.k_scale[None], t.v_scale[None], t.v_zp[None], device=DEV)
    cache.append(0, k, v)
    kc, ks, vt, vs, vz = cache.get_k8v4_tensors(0)
    out = K.decode_attn_k8v4(q, kc, ks, vt, vs, vz, ctx.to(DEV), 1 / math.sqrt(128), inv_tau=tau)
    longest = 2 + int(torch.argmax(ctx[2:]))
    for b in (0, 1, longest):
        n = int(ctx[b])
        sl = slice(b, b + 1)
        k8_ref, ks_ref = OQ.quantize_symmetric_int8_with_scale(k[sl, :, :n].cpu(), t.k_scale, 32)
        vq_ref = OQ.pack_int4(OQ.quantize_asymmetric_static(v[sl, :, :n].cpu(), t.v_scale, t.v_zp))
        assert torch.equal(kc[sl, :, :n].cpu().view(torch.int8), k8_ref), b
        assert torch.equal(ks[sl, :, :n].cpu(), ks_ref), b
        vr = K.untile_v(vt[sl], S)[:, :, :n].cpu()
        assert torch.equal(vr, vq_ref.view(torch.uint8)), b
        ref = OA.decode_attn_k8v4_ref(q[sl].cpu(), k8_ref, ks_ref, vr, t.v_scale, t.v_zp,
                                      torch.tensor([n], dtype=torch.int32), 1 / math.sqrt(128),
                                      inv_tau=tau.cpu())
        assert_close(out[sl], ref, f"cfg4 full row {b} ctx {n}")


@pytest.mark.parametrize("layout", ["rows", "tile32"])
@pytest.mark.parametrize("Hq,Hkv,S,ctx", [(32, 2, 333, [333]), (9, 1, 700, [700, 65]), (8, 1, 96, [96])])
def test_decode_asym_wide_gqa(Hq, Hkv, S, ctx, layout):
    """GQA groups of 8, 9 and 16 query heads per kv head (the tiled kernel packs the
    softmax of groups up to 8 into the MFMA's padding columns; wider groups do not)."""
    K = _lib()
    from llm_kvcache_quantization_amd import calib

    B = len(ctx)
    g = gen(Hq * 1000 + S)
    k = (torch.randn(B, Hkv, S, 128, generator=g) * 1.5).to(torch.float16)
    v = torch.randn(B, Hkv, S, 128, generator=g).to(torch.float16)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
    tau = (0.8 + 0.4 * torch.rand(Hq, generator=g)).to(torch.float16)
    ks, kz = calib.asym_g32_params(k)
    vs, vz = calib.asym_g32_params(v)
    kq = OQ.pack_int4(OQ.quantize_asymmetric_static(k, ks, kz))
    vq = OQ.pack_int4(OQ.quantize_asymmetric_static(v, vs, vz))
    cl = torch.tensor(ctx, dtype=torch.int32)
    sm = 1 / math.sqrt(128)
    ref = OA.decode_attn_asym_ref(q, kq, vq, ks, kz, vs, vz, cl, sm, inv_tau=tau)
    vd = K.tile_v(vq.to(DEV)) if layout == "tile32" else vq.to(DEV)
    out = K.decode_attn_int4_asym(q.to(DEV), kq.to(DEV), vd, ks.to(DEV), kz.to(DEV), vs.to(DEV),
                                  vz.to(DEV), cl.to(DEV), sm, inv_tau=tau.to(DEV))
    assert_close(out, ref, f"asym {layout} Hq{Hq} Hkv{Hkv} S{S}")


def test_tiled_plan_reuse_changing_context():
    """One plan (one workspace) launched repeatedly while context_lens changes in place:
    the number of work-groups that report per (b, kv head) changes between calls, and the
    arrival counters of the single-launch merge must start from zero every time."""
    K = _lib()
    from llm_kvcache_quantization_amd import _capi as C
    from llm_kvcache_quantization_amd.kernels import DecodePlan, kv_view_static

    S = 8192
    cfg, t, q, tau, kq, vq, oidx, oval, cl = _asym_case(3, 2, S, [S, S], 9)
    d = lambda x: x.to(DEV)
    cl_dev = d(cl)
    plan = DecodePlan(d(q), C.KVQ_FMT_INT4_ASYM,
                      kv_view_static(d(kq), d(t.k_scale), d(t.k_zp), d(oidx), d(oval)),
                      C.KVQ_FMT_INT4_ASYM, kv_view_static(K.tile_v(d(vq)), d(t.v_scale), d(t.v_zp)),
                      cl_dev, cfg.kv_heads, S, 1 / math.sqrt(128), 32, inv_tau=d(tau))
    for ctx in ([S, 5000], [100, 7000], [0, 33], [S, S], [4097, 1]):
        cl_dev.copy_(torch.tensor(ctx, dtype=torch.int32))
        out = plan.launch().clone()
        ref = OA.decode_attn_asym_ref(q, kq, vq, t.k_scale, t.k_zp, t.v_scale, t.v_zp,
                                      torch.tensor(ctx, dtype=torch.int32), 1 / math.sqrt(128),
                                      inv_tau=tau, k_outlier_idx=oidx, k_outlier_val=oval)
        assert_close(out, ref, f"plan reuse ctx={ctx}")


# ---------------------------------------------------------------- fused decode step


@pytest.mark.parametrize("cfg_idx,B,S0,steps,outliers", [
    (3, 2, 4095, 3, True),     # the new tokens cross a tile boundary (4095, 4096, 4097)
    (3, 3, 40, 2, True),       # new token's tile is in each wave's first (burst) tiles
    (2, 2, 9000, 2, True),     # GQA 6, the tile read late in the wave's schedule
    (3, 1, 700, 2, False),     # no outlier channels
    (3, 2, 0, 2, True),        # empty cache: the first token is the whole context
])
def test_fused_append_decode_matches_two_calls(cfg_idx, B, S0, steps, outliers):
    """append_decode_attn (one launch) against append + decode_attn_int4_asym (two
    launches) on twin caches: codes, outlier side-band and outputs bit-identical, and the
    output within tolerance of the oracle."""
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[cfg_idx]
    t = SY.calibrate(cfg, 0)
    g = gen(500 + S0)
    k, v = SY.draw_kv(cfg, 0, B, S0 + steps, g)
    qs = [SY.draw_q(cfg, B, g) for _ in range(steps)]
    tau = SY.inv_tau(cfg)[0]
    oi = t.k_outlier_idx[None] if outliers else None
    mk = lambda: K.INT4AsymKVCache(1, t.k_scale[None], t.k_zp[None], t.v_scale[None], t.v_zp[None],
                                   device=DEV, k_outlier_idx=oi)
    two, one = mk(), mk()
    if S0:
        two.append(0, k[:, :, :S0].to(DEV), v[:, :, :S0].to(DEV))
        one.append(0, k[:, :, :S0].to(DEV), v[:, :, :S0].to(DEV))
    sm = 1 / math.sqrt(128)
    for i in range(steps):
        kn, vn = k[:, :, S0 + i:S0 + i + 1].to(DEV), v[:, :, S0 + i:S0 + i + 1].to(DEV)
        q = qs[i].to(DEV)
        two.append(0, kn, vn)
        kc, vc, ks, kz, vs, vz, oidx, ov = two.get_int4_g32_tensors(0)
        n = two.get_seq_len()
        cl = torch.full((B,), n, dtype=torch.int32, device=DEV)
        ref_out = K.decode_attn_int4_asym(q, kc, vc, ks, kz, vs, vz, cl, sm, inv_tau=tau.to(DEV),
                                          k_outlier_idx=oidx, k_outlier_val=ov)
        out = one.append_decode_attn(0, q, kn, vn, sm_scale=sm, inv_tau=tau.to(DEV))
        torch.cuda.synchronize()
        assert one.get_seq_len() == n
        kc1, vc1, _, _, _, _, _, ov1 = one.get_int4_g32_tensors(0)
        assert torch.equal(kc1, kc), f"K codes differ at step {i}"
        assert torch.equal(K.untile_v(vc1, n), K.untile_v(vc, n)), f"V codes differ at step {i}"
        if outliers:
            assert torch.equal(ov1, ov), f"outlier values differ at step {i}"
        assert torch.equal(out, ref_out), f"fused output differs from the two-call path at step {i}"
        ref = OA.decode_attn_asym_ref(qs[i], kc.cpu(), K.untile_v(vc, n).cpu(), t.k_scale, t.k_zp,
                                      t.v_scale, t.v_zp, cl.cpu(), sm, inv_tau=tau,
                                      k_outlier_idx=t.k_outlier_idx if outliers else None,
                                      k_outlier_val=None if ov is None else ov.cpu())
        assert_close(out, ref, f"fused step cfg{cfg_idx} S{n}")


@pytest.mark.parametrize("kind,B,S0,steps,gs", [
    ("int8", 2, 4095, 3, 32),   # config 1 heads; the new tokens cross a tile boundary
    ("int8", 3, 0, 2, 32),      # empty cache: the first token is the whole context
    ("int8", 4, 700, 2, 32),
    ("int8", 2, 4095, 2, 16),   # group 16 (the shipped int8_ours tables)
    ("int8", 3, 31, 2, 8),
    ("int8", 2, 100, 2, 128),
    ("k8v4", 2, 4095, 3, 32),   # config 4 heads (GQA 5), TILE32 V
    ("k8v4", 3, 40, 2, 32),     # the new token's tile is in each wave's first tiles
])
def test_fused_append_decode_int8_matches_two_calls(kind, B, S0, steps, gs):
    """append_decode_attn with INT8 K (one launch) against append + the decode kernel (two
    launches) on twin caches: codes and outputs bit-identical, output within tolerance of
    the oracle."""
    K = _lib()
    from llm_kvcache_quantization_amd import calib as CB
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[1 if kind == "int8" else 4]
    t = SY.calibrate(cfg, 0)
    g = gen(900 + S0 + B + gs)
    k, v = SY.draw_kv(cfg, 0, B, S0 + steps, g)
    qs = [SY.draw_q(cfg, B, g) for _ in range(steps)]
    tau = SY.inv_tau(cfg)[0]
    if kind == "int8":
        if gs != 32:  # tables of this group size from the same calibration sample
            ck, cv = SY.draw_kv(cfg, 0, 1, SY.CALIB_TOKENS, gen(4242))
            t.k_scale, t.v_scale = CB.int8_static_scale(ck, gs), CB.int8_static_scale(cv, gs)
        mk = lambda: K.INT8KVCache(1, device=DEV, group_size=gs, static_k_scale=t.k_scale[None],
                                   static_v_scale=t.v_scale[None], check_numerics=True)
    else:
        mk = lambda: K.K8V4KVCache(1, t.k_scale[None], t.v_scale[None], t.v_zp[None], device=DEV,
                                   check_numerics=True)
    two, one = mk(), mk()
    if kind == "int8":
        assert one._fused_step_ok(128), "static INT8 tables take the one-launch step"
    if S0:
        for c in (two, one):
            c.append(0, k[:, :, :S0].to(DEV), v[:, :, :S0].to(DEV))
    sm = 1 / math.sqrt(128)
    for i in range(steps):
        kn, vn = k[:, :, S0 + i:S0 + i + 1].to(DEV), v[:, :, S0 + i:S0 + i + 1].to(DEV)
        q = qs[i].to(DEV)
        two.append(0, kn, vn)
        n = two.get_seq_len()
        cl = torch.full((B,), n, dtype=torch.int32, device=DEV)
        out = one.append_decode_attn(0, q, kn, vn, sm_scale=sm, inv_tau=tau.to(DEV))
        assert one.get_seq_len() == n
        if kind == "int8":
            k8, v8, ks, vs = two.get_int8_tensors(0)
            ref_out = K.decode_attn_int8(OA.prescale_q(q, tau.to(DEV)), k8, v8, ks, vs, cl, sm_scale=sm)
            k8b, v8b, _, _ = one.get_int8_tensors(0)
            assert torch.equal(k8b, k8) and torch.equal(v8b, v8), f"codes differ at step {i}"
            ref = OA.decode_attn_int8_torch_ref(OA.prescale_q(qs[i], tau), k8.cpu(), v8.cpu(),
                                                ks.cpu(), vs.cpu(), cl.cpu(), sm)
        else:
            k8, ks, vc, vs, vz = two.get_k8v4_tensors(0)
            ref_out = K.decode_attn_k8v4(q, k8, ks, vc, vs, vz, cl, sm, inv_tau=tau.to(DEV))
            k8b, _, vcb, _, _ = one.get_k8v4_tensors(0)
            assert torch.equal(k8b, k8), f"K codes differ at step {i}"
            assert torch.equal(K.untile_v(vcb, n), K.untile_v(vc, n)), f"V codes differ at step {i}"
            ref = OA.decode_attn_k8v4_ref(qs[i], k8.cpu(), ks.cpu(), K.untile_v(vc, n).cpu(),
                                          vs.cpu(), vz.cpu(), cl.cpu(), sm, inv_tau=tau)
        assert torch.equal(out, ref_out), f"fused output differs from the two-call path at step {i}"
        assert_close(out, ref, f"fused {kind} step S{n}")


def test_fused_append_decode_nan_raises_and_does_not_advance():
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[3]
    t = SY.calibrate(cfg, 0)
    g = gen(77)
    k, v = SY.draw_kv(cfg, 0, 2, 65, g)
    q = SY.draw_q(cfg, 2, g).to(DEV)
    cache = K.INT4AsymKVCache(1, t.k_scale[None], t.k_zp[None], t.v_scale[None], t.v_zp[None],
                              device=DEV, k_outlier_idx=t.k_outlier_idx[None], check_numerics=True)
    cache.append(0, k[:, :, :64].to(DEV), v[:, :, :64].to(DEV))
    bad = v[:, :, 64:].clone()
    bad[1, 2, 0, 17] = float("nan")
    with pytest.raises(ValueError, match="NaN or Inf"):
        cache.append_decode_attn(0, q, k[:, :, 64:].to(DEV), bad.to(DEV))
    assert cache.get_seq_len() == 64
    out = cache.append_decode_attn(0, q, k[:, :, 64:].to(DEV), v[:, :, 64:].to(DEV))
    assert cache.get_seq_len() == 65 and torch.isfinite(out.float()).all()


def test_decode_step_status_read_once_per_step_and_rolled_back():
    """check_numerics on the decode step: the status words of all layers are read once,
    after the step's last layer.  A NaN in a middle layer's new token raises there and every
    layer of the step goes back to its length before the step (the reference's "raise and do
    not advance": src/quant/_common.py:13-20 raises before src/cache/int8_cache.py:350-488
    writes); the next step then runs normally."""
    K = _lib()
    from llm_kvcache_quantization_amd import synthetic as SY

    cfg = SY.CONFIGS[3]
    t = SY.calibrate(cfg, 0)
    L = 3
    g = gen(78)
    k, v = SY.draw_kv(cfg, 0, 2, 66, g)
    q = SY.draw_q(cfg, 2, g).to(DEV)
    rep = lambda x: x[None].expand(L, *x.shape).contiguous()
    cache = K.INT4AsymKVCache(L, rep(t.k_scale), rep(t.k_zp), rep(t.v_scale), rep(t.v_zp),
                              device=DEV, k_outlier_idx=rep(t.k_outlier_idx), check_numerics=True)
    for layer in range(L):
        cache.append(layer, k[:, :, :64].to(DEV), v[:, :, :64].to(DEV))
    k1, v1 = k[:, :, 64:65].to(DEV), v[:, :, 64:65].to(DEV)
    bad = v1.clone()
    bad[0, 1, 0, 5] = float("inf")
    cache.append_decode_attn(0, q, k1, v1)
    cache.append_decode_attn(1, q, k1, bad)  # not read yet: no host sync per layer
    assert cache._layer_seq_lens == [65, 65, 64]
    with pytest.raises(ValueError, match="NaN or Inf"):
        cache.append_decode_attn(2, q, k1, v1)
    assert cache._layer_seq_lens == [64, 64, 64] and cache.get_seq_len() == 64
    # the step again with good data, then one more step: every layer matches a fresh cache
    ref = K.INT4AsymKVCache(L, rep(t.k_scale), rep(t.k_zp), rep(t.v_scale), rep(t.v_zp),
                            device=DEV, k_outlier_idx=rep(t.k_outlier_idx), check_numerics=False)
    for layer in range(L):
        ref.append(layer, k[:, :, :64].to(DEV), v[:, :, :64].to(DEV))
    k2, v2 = k[:, :, 65:66].to(DEV), v[:, :, 65:66].to(DEV)
    for kk, vv in ((k1, v1), (k2, v2)):
        for layer in range(L):
            out = cache.append_decode_attn(layer, q, kk, vv)
            ro = ref.append_decode_attn(layer, q, kk, vv)
            assert torch.equal(out, ro), layer
    assert cache._layer_seq_lens == [66, 66, 66] and cache.get_seq_len() == 66
    for layer in range(L):
        assert torch.equal(cache.get_int4_g32_tensors(layer)[0], ref.get_int4_g32_tensors(layer)[0])
    # a partial step read explicitly
    bad2 = k2.clone()
    bad2[1, 0, 0, 0] = float("nan")
    cache.append_decode_attn(0, q, bad2, v2)
    with pytest.raises(ValueError, match="K input contains NaN"):
        cache.flush_status()
    assert cache._layer_seq_lens == [66, 66, 66]


# ---------------------------------------------------------------- KIVI layout


def _kivi_case(B, Hq, Hkv, S, ctx, seed, garbage=True, k_outliers=0):
    """Prefill-style KIVI cache: per-channel K and per-token V parameters from the oracle's
    quantizers over the whole capacity; past each context the V parameters are NaN / inf
    (memory the reference masks) when garbage is set.  V ~ N(0, 1) scaled and shifted per
    token (per-token ranges from about 1 to about 20, |v| up to about 15), as wide as the
    reference's per-token quantizer meets in practice; K ~ N(0, 1) with per-channel widths
    in [0.2, 3.2], and with k_outliers channels per head of range about 100-300 (the
    large-magnitude K channels of Qwen caches)."""
    g = gen(seed)
    D = 128
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    width = torch.rand(1, Hkv, 1, D, generator=g) * 3 + 0.2
    for h in range(Hkv):
        ch = torch.randperm(D, generator=g)[:k_outliers]
        width[0, h, 0, ch] = torch.rand(k_outliers, generator=g) * 33 + 17
    k = torch.randn(B, Hkv, S, D, generator=g) * width
    v = (torch.randn(B, Hkv, S, D, generator=g) * (torch.rand(B, Hkv, S, 1, generator=g) * 2.5 + 0.2)
         + torch.randn(B, Hkv, S, 1, generator=g) * 3.0)
    qk, ks, kz = OQ.quantize_asymmetric_per_channel(k, 4)
    qv, vs, vz = OQ.quantize_asymmetric_per_token(v, 4)
    kp, vp = OQ.pack_int4(qk), OQ.pack_int4(qv)
    ctx_t = torch.tensor(ctx, dtype=torch.int32)
    vs_d, vz_d = vs.clone(), vz.clone()
    if garbage:
        for b, c in enumerate(ctx):
            vs_d[b, :, c:] = float("nan")
            vz_d[b, :, c:] = float("inf")
    return q, kp, vp, ks, kz, vs, vz, vs_d, vz_d, ctx_t


@pytest.mark.parametrize("B,Hq,Hkv,S,ctx,k_outliers", [
    (2, 8, 2, 300, [300, 77], 0),
    (1, 28, 4, 1000, [1000], 0),
    (3, 12, 2, 64, [64, 1, 0], 0),
    (4, 12, 2, 40, [1, 1, 2, 1], 0),
    (1, 16, 1, 4500, [4500], 0),
    (2, 4, 4, 9000, [9000, 5003], 0),
    (1, 9, 1, 33, [33], 0),
    (2, 28, 4, 2000, [2000, 1], 3),
    (1, 12, 2, 5000, [5000], 4),
])
def test_decode_kivi_parity(B, Hq, Hkv, S, ctx, k_outliers):
    K = _lib()
    q, kp, vp, ks, kz, vs, vz, vs_d, vz_d, ctx_t = _kivi_case(B, Hq, Hkv, S, ctx, 31 + S,
                                                              k_outliers=k_outliers)
    ref = OA.decode_attn_kivi_ref(q, kp, vp, ks, kz, vs, vz, ctx_t, 1 / math.sqrt(128))
    d = lambda t: t.to(DEV)  # noqa: E731
    out = K.kernels.decode_attn_int4_asym(d(q), d(kp), d(vp), d(ks), d(kz), d(vs_d), d(vz_d),
                                          d(ctx_t))
    torch.cuda.synchronize()
    assert_close_ulp(out, ref, f"kivi B{B} Hq{Hq} Hkv{Hkv} S{S} kout{k_outliers}")


def test_decode_kivi_inv_tau_bf16_q_and_fp16_params():
    K = _lib()
    B, Hq, Hkv, S, ctx = 2, 8, 2, 700, [700, 390]
    q, kp, vp, ks, kz, vs, vz, vs_d, vz_d, ctx_t = _kivi_case(B, Hq, Hkv, S, ctx, 77, garbage=False)
    g = gen(78)
    tau = (torch.rand(Hq, generator=g) + 0.5).to(torch.float16)
    # fp16 parameters are widened to fp32 (the reference converts them the same way)
    ks16, kz16 = ks.half(), kz.half()
    ref = OA.decode_attn_kivi_ref(q, kp, vp, ks16.float(), kz16.float(), vs, vz, ctx_t, 0.07,
                                  inv_tau=tau)
    d = lambda t: t.to(DEV)  # noqa: E731
    out = K.kernels.decode_attn_int4_kivi(d(q).to(torch.bfloat16), d(kp), d(vp), d(ks16), d(kz16),
                                          d(vs), d(vz), d(ctx_t), 0.07, inv_tau=d(tau))
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    # bf16 q is rounded to fp16 first
    ref16 = OA.decode_attn_kivi_ref(q.to(torch.bfloat16).to(torch.float16), kp, vp, ks16.float(),
                                    kz16.float(), vs, vz, ctx_t, 0.07, inv_tau=tau)
    o, r = out.float().cpu(), ref16.float()
    # the fp16 result rounded to bf16: within 2e-3 plus half a bf16 ulp of the fp16 oracle
    err = (o - r).abs() - r.abs() * 2.0 ** -8
    print(f"[kivi bf16 q] max_excess={err.max().item():.3e}", flush=True)
    assert torch.isfinite(o).all() and (err <= ATOL).all()
    # the bf16 rounding of q moves the result measurably: the fp16-q oracle is a different case
    assert (ref - ref16).abs().max().item() > 0


@pytest.mark.parametrize("B,H,S0,steps", [(2, 2, 37, 3), (1, 4, 300, 1)])
def test_kivi_cache_append_bitexact_and_decode(B, H, S0, steps):
    """KIVIStyleKVCache: prefill + decode appends through kvq_quant_append are bit-exact
    with the oracle's per-channel / per-token quantizers (fp32 parameters included), and the
    cache's decode attention matches the oracle over the stored codes."""
    K = _lib()
    g = gen(500 + S0)
    D = 128
    k0 = (torch.randn(B, H, S0, D, generator=g) * 2).to(torch.float16)
    v0 = torch.randn(B, H, S0, D, generator=g).to(torch.float16)
    cache = K.KIVIStyleKVCache(num_layers=1, device=DEV, quant_bits=4)
    cache.append(0, k0.to(DEV), v0.to(DEV))
    ks_ref_q, ks, kz = OQ.quantize_asymmetric_per_channel(k0, 4)
    ks_codes = [ks_ref_q]
    vq, vs, vz = OQ.quantize_asymmetric_per_token(v0, 4)
    v_codes, v_s, v_z = [vq], [vs], [vz]
    for i in range(steps):
        k1 = (torch.randn(B, H, 1, D, generator=g) * 2.5).to(torch.float16)  # some codes clip
        v1 = torch.randn(B, H, 1, D, generator=g).to(torch.float16)
        cache.append(0, k1.to(DEV), v1.to(DEV))
        ks_codes.append(OQ.kivi_quantize_k_static(k1, ks, kz))
        q1, s1, z1 = OQ.quantize_asymmetric_per_token(v1, 4)
        v_codes.append(q1); v_s.append(s1); v_z.append(z1)
    torch.cuda.synchronize()
    kp, vp, gks, gkz, gvs, gvz = [t.cpu() for t in cache.get_int4_asym_tensors(0)]
    assert cache.get_seq_len() == S0 + steps
    assert torch.equal(gks, ks) and torch.equal(gkz, kz)
    assert torch.equal(gvs, torch.cat(v_s, 2)) and torch.equal(gvz, torch.cat(v_z, 2))
    assert kp.dtype == torch.int8 and vp.dtype == torch.int8
    assert torch.equal(kp, OQ.pack_int4(torch.cat(ks_codes, 2)))
    assert torch.equal(vp, OQ.pack_int4(torch.cat(v_codes, 2)))
    q = torch.randn(B, 4 * H, D, generator=g).to(torch.float16)
    out = cache.decode_attn(0, q.to(DEV))
    torch.cuda.synchronize()
    ctx = torch.full((B,), S0 + steps, dtype=torch.int32)
    ref = OA.decode_attn_kivi_ref(q, kp, vp, gks, gkz, gvs, gvz, ctx, 1 / math.sqrt(D))
    assert_close(out, ref, f"kivi cache B{B} H{H} S{S0}+{steps}")
    k_deq, v_deq = cache.get_kv(0)
    assert k_deq.shape == (B, H, S0 + steps, D)


@pytest.mark.parametrize("B,S,ctx", [
    (10, 16384, [0, 1, 31, 33, 500, 4097, 12000, 16384, 257, 64]),
    (3, 20000, [20000, 19999, 7]),
    (64, 600, [((i * 37) % 600) for i in range(64)]),
])
def test_decode_shared_split_ragged(B, S, ctx):
    """Ragged per-row contexts (a context tensor, 2..64 rows): the tiled kernel shares the
    kv head's work-groups out over the rows by length, empty and one-tile rows included.
    Against the oracle, and two launches bit-identical (the shares depend on the lengths
    only)."""
    K = _lib()
    cfg, t, q, tau, kq, vq, oidx, oval, cl = _asym_case(3, B, S, ctx, 70 + B, True)
    sm = 1 / math.sqrt(128)
    ref = OA.decode_attn_asym_ref(q, kq, vq, t.k_scale, t.k_zp, t.v_scale, t.v_zp, cl, sm,
                                  inv_tau=tau, k_outlier_idx=oidx, k_outlier_val=oval)
    args = (q.to(DEV), kq.to(DEV), K.tile_v(vq.to(DEV)), t.k_scale.to(DEV), t.k_zp.to(DEV),
            t.v_scale.to(DEV), t.v_zp.to(DEV), cl.to(DEV), sm)
    kw = dict(inv_tau=tau.to(DEV), k_outlier_idx=oidx.to(DEV), k_outlier_val=oval.to(DEV))
    out = K.decode_attn_int4_asym(*args, **kw).clone()
    again = K.decode_attn_int4_asym(*args, **kw)
    assert torch.equal(out, again)
    assert_close(out, ref, f"shared split B{B} S{S}")
    for b, c in enumerate(ctx):
        if c == 0:
            assert torch.all(out[b] == 0)


@pytest.mark.parametrize("heads,ctx", [
    ((32, 2), [4000, 90, 2500, 33, 4096, 1200, 700, 3001, 64, 1900]),  # 16 query heads per kv head
    ((4, 4), [4096, 1, 2049, 300, 3999, 1024, 77, 2600]),              # one query head per kv head
    ((20, 2), [4096, 4095, 100, 3000, 31, 2222]),                      # 10: three pairs on some waves
])
def test_decode_shared_split_two_row_merge(heads, ctx):
    """The shared split's merge of work-groups that hold two rows and arrive last for both:
    (row, head) pairs shared out over the 8 waves, two pairs per wave with their loads
    issued together, for query heads per kv head from 1 to 16.  Against the oracle, and two
    launches bit-identical."""
    K = _lib()
    B, S = len(ctx), 4096
    cfg, t, q, tau, kq, vq, oidx, oval, cl = _asym_case(3, B, S, ctx, 90 + heads[0], True, heads)
    sm = 1 / math.sqrt(128)
    ref = OA.decode_attn_asym_ref(q, kq, vq, t.k_scale, t.k_zp, t.v_scale, t.v_zp, cl, sm,
                                  inv_tau=tau, k_outlier_idx=oidx, k_outlier_val=oval)
    args = (q.to(DEV), kq.to(DEV), K.tile_v(vq.to(DEV)), t.k_scale.to(DEV), t.k_zp.to(DEV),
            t.v_scale.to(DEV), t.v_zp.to(DEV), cl.to(DEV), sm)
    kw = dict(inv_tau=tau.to(DEV), k_outlier_idx=oidx.to(DEV), k_outlier_val=oval.to(DEV))
    out = K.decode_attn_int4_asym(*args, **kw).clone()
    again = K.decode_attn_int4_asym(*args, **kw)
    assert torch.equal(out, again)
    assert_close(out, ref, f"two-row merge heads {heads}")

