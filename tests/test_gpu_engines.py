"""GPU tests of the cache engines against the CPU oracle.

* Dynamic quantizers with percentile clipping (the reference engines' default
  clip_percentile=99.9 without static scales): codes and scales bit-exact.
* The calibration tables the reference ships for Qwen2.5-1.5B (group 16; INT8 tables in
  fp16, INT4 tables in fp32 with outlier rescue ratio 0.01; tests/golden/calib_*.json):
  appends bit-exact through prefill (the rescue's radix select) and decode (its LDS sort),
  then decode attention with the tables' inv_tau within max-abs 2e-3 / cosine 0.9999.
* get_kv / to_tuple / from_tuple against the oracle's dequantizers.
* Decode steps through append_decode_attn, whose kernel parameters and workspace are kept
  per layer, across a buffer reallocation, for every engine.
"""
import math
import os
import warnings

import pytest
import torch

from oracle import attn as OA
from oracle import quant as OQ

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL = 2e-3
COS_MIN = 0.9999
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _k():
    import llm_kvcache_quantization_amd as K
    from llm_kvcache_quantization_amd import _capi

    _capi.lib()
    return K


def gen(seed):
    return torch.Generator().manual_seed(seed)


def assert_close(out, ref, tag):
    o, r = out.detach().float().cpu(), ref.detach().float().cpu()
    assert o.shape == r.shape, (tag, o.shape, r.shape)
    assert torch.isfinite(o).all(), tag
    err = (o - r).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r.flatten(), dim=0).item()
    print(f"[{tag}] max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= ATOL and cos >= COS_MIN, (tag, err, cos)


def fp16_ulp(x):
    a = x.abs().float().clamp(min=2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def assert_close_ulp(out, ref, tag):
    """assert_close for outputs that reach |out| >= 4, where neighbouring fp16 values are
    more than 2e-3 apart (2^-8 at [4, 8), 2^-7 at [8, 16)): two fp32 computations of one
    value that differ only in summation order may round to neighbouring fp16 values there.
    Per element the bound is max(2e-3, one fp16 ulp of the oracle's value)."""
    o, r = out.detach().float().cpu(), ref.detach().float().cpu()
    assert o.shape == r.shape and torch.isfinite(o).all(), tag
    err = (o - r).abs()
    worst = (err - torch.maximum(torch.full_like(r, ATOL), fp16_ulp(r))).max().item()
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r.flatten(), dim=0).item()
    print(f"[{tag}] max_abs={err.max().item():.3e} max|ref|={r.abs().max().item():.2f} "
          f"above_2e-3={(err > ATOL).sum().item()} excess={worst:.3e} cos={cos:.7f}", flush=True)
    assert worst <= 0 and cos >= COS_MIN, (tag, worst, cos)


def _kv(B, H, S, g, scale=1.0, outliers=True):
    k = torch.randn(B, H, S, 128, generator=g) * scale
    v = torch.randn(B, H, S, 128, generator=g) * scale
    if outliers:
        k[..., 5] *= 12.0
        k[..., 77] *= -9.0
    return k.to(torch.float16), v.to(torch.float16)


# ---------------------------------------------------------------- percentile dynamic scales


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("percentile,gs,ties", [
    (99.9, 128, False), (99.5, 16, False), (99.0, 32, False), (99.9, 64, False), (100.0, 32, False),
    (99.9, 128, True),   # equal values at the top of the groups
    (90.0, 128, False),  # ranks far from the top (the rank-count path)
    (97.0, 64, True),
])
def test_dynamic_percentile_append_bitexact(bits, percentile, gs, ties):
    K = _k()
    print(f"[case] bits={bits} p={percentile} gs={gs} ties={ties}", flush=True)
    g = gen(int(percentile * 10) + gs + bits + ties)
    B, H = 2, 2
    k0, v0 = _kv(B, H, 37, g)
    k1, v1 = _kv(B, H, 1, g)
    if ties:  # few distinct magnitudes, so the largest ones repeat within a group
        k0, v0, k1, v1 = [(x * 2).round().div(2).to(torch.float16) for x in (k0, v0, k1, v1)]
    Cache = K.INT8KVCache if bits == 8 else K.INT4KVCache
    cache = Cache(1, device=DEV, clip_percentile=percentile, group_size=gs)
    cache.append(0, k0.to(DEV), v0.to(DEV))
    cache.append(0, k1.to(DEV), v1.to(DEV))
    torch.cuda.synchronize()
    k, v = torch.cat([k0, k1], 2), torch.cat([v0, v1], 2)
    if bits == 8:
        kc, vc, ks, vs = [t.cpu() for t in cache.get_int8_tensors(0)]
        rk, rks = OQ.quantize_symmetric_int8(k, percentile, gs)
        rv, rvs = OQ.quantize_symmetric_int8(v, percentile, gs)
    else:
        kc, vc, ks, vs = [t.cpu() for t in cache.get_int4_tensors(0)]
        kc, vc = OQ.unpack_int4(kc), OQ.unpack_int4(vc)
        rk, rks = OQ.quantize_symmetric_int4(k, percentile, gs)
        rv, rvs = OQ.quantize_symmetric_int4(v, percentile, gs)
    assert torch.equal(kc, rk) and torch.equal(vc, rv)
    assert torch.equal(ks.float(), rks.float()) and torch.equal(vs.float(), rvs.float())


# ---------------------------------------------------------------- the shipped tables


def _shipped(bits):
    from llm_kvcache_quantization_amd.calib import load_calibration_json

    return load_calibration_json(os.path.join(GOLDEN, f"calib_qwen25_1p5b_int{bits}.json"), quant_bits=bits)


def _table_scaled(t_scale, B, S, g, qmax, spread):
    """K or V [B, Hkv, S, 128] fp16 whose groups span about +-qmax * scale / spread."""
    H, G = t_scale.shape
    gs = 128 // G
    width = (t_scale.float() * qmax / spread).repeat_interleave(gs, dim=-1)  # [H, 128]
    return (torch.randn(B, H, S, 128, generator=g) * width[None, :, None, :]).to(torch.float16)


@pytest.mark.parametrize("layer", [0, 13, 27])
def test_shipped_int8_tables(layer):
    """kv_mode int8_ours with the reference's own table: static fp16 k/v scales, group 16,
    clip_percentile 99.5, inv_tau [28, 12]."""
    K = _k()
    t = _shipped(8)
    assert t.group_size == 16 and t.k_scale.dtype == torch.float16 and tuple(t.k_scale.shape) == (28, 2, 8)
    g = gen(100 + layer)
    B, S0, steps, Hq = 2, 300, 3, 12
    cache = K.INT8KVCache(28, device=DEV, clip_percentile=99.5, group_size=t.group_size,
                          static_k_scale=t.k_scale.to(DEV), static_v_scale=t.v_scale.to(DEV),
                          inv_tau=t.inv_tau.to(DEV))
    k0 = _table_scaled(t.k_scale[layer], B, S0, g, 127, 3.0)
    v0 = _table_scaled(t.v_scale[layer], B, S0, g, 127, 3.0)
    cache.append(layer, k0.to(DEV), v0.to(DEV))
    ks_all, vs_all = [k0], [v0]
    tau16 = t.inv_tau[layer].to(torch.float16)
    for i in range(steps):
        k1 = _table_scaled(t.k_scale[layer], B, 1, g, 127, 3.0)
        v1 = _table_scaled(t.v_scale[layer], B, 1, g, 127, 3.0)
        q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
        out = cache.append_decode_attn(layer, q.to(DEV), k1.to(DEV), v1.to(DEV), inv_tau=tau16.to(DEV))
        ks_all.append(k1)
        vs_all.append(v1)
        torch.cuda.synchronize()
        kc, vc, ks, vs = [x.cpu() for x in cache.get_int8_tensors(layer)]
        rk, rks = OQ.int8_cache_quantize(torch.cat(ks_all, 2), t.k_scale[layer], 16)
        rv, rvs = OQ.int8_cache_quantize(torch.cat(vs_all, 2), t.v_scale[layer], 16)
        assert torch.equal(kc, rk) and torch.equal(vc, rv)
        assert torch.equal(ks, rks) and torch.equal(vs, rvs)
        n = S0 + i + 1
        ref = OA.decode_attn_int8_torch_ref(OA.prescale_q(q, tau16), rk, rv, rks, rvs,
                                            torch.full((B,), n), 1 / math.sqrt(128))
        assert_close_ulp(out, ref, f"shipped int8 layer {layer} S{n}")


@pytest.mark.parametrize("layer", [0, 27])
def test_shipped_int4_tables_with_rescue(layer):
    """kv_mode int4_fused with the reference's own table: static fp32 scales, group 16,
    int4_outlier_ratio 0.01 (per-token fp32 scales; the prefill's rescue threshold over
    2 x 2 x 300 x 8 = 9600 group scales comes from the radix select, the decode steps' from
    the in-launch sort)."""
    K = _k()
    t = _shipped(4)
    assert t.group_size == 16 and t.k_scale.dtype == torch.float32 and t.outlier_ratio == 0.01
    g = gen(200 + layer)
    B, S0, steps, Hq = 2, 300, 2, 12
    cache = K.INT4KVCache(28, device=DEV, clip_percentile=99.0, group_size=t.group_size,
                          static_k_scale=t.k_scale.to(DEV), static_v_scale=t.v_scale.to(DEV),
                          inv_tau=t.inv_tau.to(DEV), outlier_rescue_ratio=t.outlier_ratio,
                          mixed_rescue=t.mixed_rescue)
    k0 = _table_scaled(t.k_scale[layer], B, S0, g, 7, 2.0)
    v0 = _table_scaled(t.v_scale[layer], B, S0, g, 7, 2.0)
    cache.append(layer, k0.to(DEV), v0.to(DEV))
    rk0, rks0 = OQ.int4_cache_quantize(k0, t.k_scale[layer], 16, outlier_rescue_ratio=0.01)
    rv0, rvs0 = OQ.int4_cache_quantize(v0, t.v_scale[layer], 16, outlier_rescue_ratio=0.01)
    codes_k, codes_v, sk, sv = [rk0], [rv0], [rks0], [rvs0]
    tau16 = t.inv_tau[layer].to(torch.float16)
    for i in range(steps):
        k1 = _table_scaled(t.k_scale[layer], B, 1, g, 7, 2.0)
        v1 = _table_scaled(t.v_scale[layer], B, 1, g, 7, 2.0)
        q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
        out = cache.append_decode_attn(layer, q.to(DEV), k1.to(DEV), v1.to(DEV), inv_tau=tau16.to(DEV))
        a, b = OQ.int4_cache_quantize(k1, t.k_scale[layer], 16, outlier_rescue_ratio=0.01)
        c, d = OQ.int4_cache_quantize(v1, t.v_scale[layer], 16, outlier_rescue_ratio=0.01)
        codes_k.append(a); sk.append(b); codes_v.append(c); sv.append(d)
        torch.cuda.synchronize()
        kp, vp, ks, vs = [x.cpu() for x in cache.get_int4_tensors(layer)]
        rk, rv = torch.cat(codes_k, 2), torch.cat(codes_v, 2)
        rks, rvs = torch.cat(sk, 2), torch.cat(sv, 2)
        assert torch.equal(kp, OQ.pack_int4(rk)) and torch.equal(vp, OQ.pack_int4(rv))
        assert torch.equal(ks, rks) and torch.equal(vs, rvs)
        n = S0 + i + 1
        # the reference casts the fp32 scales to fp16 at the kernel boundary
        ref = OA.decode_attn_int8_torch_ref(OA.prescale_q(q, tau16), rk, rv, rks.half(), rvs.half(),
                                            torch.full((B,), n), 1 / math.sqrt(128))
        assert_close_ulp(out, ref, f"shipped int4 layer {layer} S{n}")


# ---------------------------------------------------------------- get_kv / to_tuple / from_tuple


@pytest.mark.parametrize("bits", [8, 4])
def test_get_kv_to_tuple_from_tuple(bits):
    K = _k()
    g = gen(300 + bits)
    B, H, S, L = 2, 2, 40, 2
    Cache = K.INT8KVCache if bits == 8 else K.INT4KVCache
    gs = 32
    st = torch.rand(L, H, 128 // gs, generator=g) * (0.03 if bits == 8 else 0.5) + 0.01
    st = st.to(torch.float16) if bits == 8 else st
    static = Cache(L, device=DEV, group_size=gs, static_k_scale=st.to(DEV), static_v_scale=st.to(DEV))
    dynamic = Cache(L, device=DEV, group_size=gs, clip_percentile=99.9)
    past = []
    for layer in range(L):
        k, v = _kv(B, H, S, g)
        past.append((k.to(DEV), v.to(DEV)))
        static.append(layer, k.to(DEV), v.to(DEV))
        dynamic.append(layer, k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    for cache in (static, dynamic):
        for layer in range(L):
            get = cache.get_int8_tensors if bits == 8 else cache.get_int4_tensors
            kc, vc, ks, vs = [x.cpu() for x in get(layer)]
            if bits == 4:
                kc, vc = OQ.unpack_int4(kc), OQ.unpack_int4(vc)
            k_deq, v_deq = cache.get_kv(layer)
            assert k_deq.dtype == torch.float16
            assert torch.equal(k_deq.cpu(), OQ.cache_get_kv(kc, ks))
            assert torch.equal(v_deq.cpu(), OQ.cache_get_kv(vc, vs))
        tup = cache.to_tuple()
        assert len(tup) == L and all(torch.equal(a, b) for (a, _), (b, _) in
                                     zip(tup, [cache.get_kv(i) for i in range(L)]))
    # from_tuple quantizes with the reference's defaults (dynamic, clip_percentile 99.9)
    rebuilt = Cache.from_tuple(tuple(past), device=DEV)
    for layer in range(L):
        k, v = past[layer]
        get = rebuilt.get_int8_tensors if bits == 8 else rebuilt.get_int4_tensors
        kc, vc, ks, vs = [x.cpu() for x in get(layer)]
        if bits == 8:
            rk, rks = OQ.quantize_symmetric_int8(k.cpu(), 99.9, 128)
        else:
            kc = OQ.unpack_int4(kc)
            rk, rks = OQ.quantize_symmetric_int4(k.cpu(), 99.9, 32)
        assert torch.equal(kc, rk) and torch.equal(ks.float(), rks.float())
    with pytest.raises(ValueError):
        Cache(1, device=DEV).to_tuple()


# ---------------------------------------------------------------- cached decode steps


def _engine(K, kind, L, H, g):
    from llm_kvcache_quantization_amd import synthetic as SY  # noqa: F401

    if kind == "int8_g32":
        st = (torch.rand(L, H, 4, generator=g) * 0.03 + 0.01).to(torch.float16)
        return K.INT8KVCache(L, device=DEV, group_size=32, static_k_scale=st.to(DEV),
                             static_v_scale=st.to(DEV), check_numerics=False)
    if kind == "int8_g16":
        st = (torch.rand(L, H, 8, generator=g) * 0.03 + 0.01).to(torch.float16)
        return K.INT8KVCache(L, device=DEV, group_size=16, static_k_scale=st.to(DEV),
                             static_v_scale=st.to(DEV))
    if kind == "int4_rescue":
        st = torch.rand(L, H, 4, generator=g) * 0.4 + 0.2
        return K.INT4KVCache(L, device=DEV, group_size=32, static_k_scale=st.to(DEV),
                             static_v_scale=st.to(DEV), outlier_rescue_ratio=0.1)
    if kind == "asym":
        s = (torch.rand(L, H, 4, generator=g) * 0.3 + 0.4).to(torch.float16)
        z = (torch.randn(L, H, 4, generator=g) * 0.1).to(torch.float16)
        oi = torch.stack([torch.stack([torch.randperm(128, generator=g)[:4].sort().values
                                       for _ in range(H)]) for _ in range(L)]).to(torch.int32)
        return K.INT4AsymKVCache(L, s, z, s, z, device=DEV, k_outlier_idx=oi)
    if kind == "k8v4":
        ks = (torch.rand(L, H, 4, generator=g) * 0.03 + 0.01).to(torch.float16)
        s = (torch.rand(L, H, 4, generator=g) * 0.3 + 0.4).to(torch.float16)
        z = (torch.randn(L, H, 4, generator=g) * 0.1).to(torch.float16)
        return K.K8V4KVCache(L, ks, s, z, device=DEV)
    if kind == "kivi":
        return K.KIVIStyleKVCache(L, device=DEV, quant_bits=4)
    if kind == "mixed":
        return K.MixedKVCache(L, device=DEV, k_group_size=32)
    raise ValueError(kind)


def _reference_out(K, kind, cache, layer, q, tau, n):
    ctx = torch.full((q.shape[0],), n, dtype=torch.int32)
    sm = 1 / math.sqrt(128)
    if kind.startswith("int8"):
        kc, vc, ks, vs = [x.cpu() for x in cache.get_int8_tensors(layer)]
        return OA.decode_attn_int8_torch_ref(OA.prescale_q(q, tau), kc, vc, ks, vs, ctx, sm)
    if kind == "int4_rescue":
        kp, vp, ks, vs = [x.cpu() for x in cache.get_int4_tensors(layer)]
        return OA.decode_attn_int4_torch_ref(OA.prescale_q(q, tau), kp, vp, ks.half(), vs.half(), ctx, sm)
    if kind == "asym":
        kc, vt, ks, kz, vs, vz, oi, ov = cache.get_int4_g32_tensors(layer)
        vr = K.untile_v(vt, n)
        return OA.decode_attn_asym_ref(q, kc.cpu(), vr.cpu(), ks.cpu(), kz.cpu(), vs.cpu(), vz.cpu(),
                                       ctx, sm, inv_tau=tau, k_outlier_idx=oi.cpu(), k_outlier_val=ov.cpu())
    if kind == "k8v4":
        kc, ks, vt, vs, vz = cache.get_k8v4_tensors(layer)
        return OA.decode_attn_k8v4_ref(q, kc.cpu(), ks.cpu(), K.untile_v(vt, n).cpu(), vs.cpu(),
                                       vz.cpu(), ctx, sm, inv_tau=tau)
    if kind == "mixed":
        kc, ks, vp, vs, vz = [x.cpu() for x in cache.get_mixed_tensors(layer)]
        return OA.decode_attn_mixed_ref(q, kc, ks, OQ.unpack_int4(vp), vs, vz, ctx, sm, inv_tau=tau)
    kp, vp, ks, kz, vs, vz = [x.cpu() for x in cache.get_int4_asym_tensors(layer)]
    return OA.decode_attn_kivi_ref(q, kp, vp, ks, kz, vs, vz, ctx, sm, inv_tau=tau)


@pytest.mark.parametrize("kind", ["int8_g32", "int8_g16", "int4_rescue", "asym", "k8v4", "kivi",
                                  "mixed"])
def test_cached_decode_steps_across_growth(kind):
    """A prefill of 250 tokens, then 12 decode steps through append_decode_attn on two
    layers: the first capacity (256) is outgrown at step 7, so the cached kernel parameters
    are rebuilt over the new buffers; every step matches the oracle over the cache's own
    tensors."""
    K = _k()
    print(f"[case] {kind}", flush=True)
    g = gen(400 + len(kind))
    B, H, Hq, L, S0, steps = 2, 2, 14, 2, 250, 12
    cache = _engine(K, kind, L, H, g)
    for layer in range(L):
        k, v = _kv(B, H, S0, g, outliers=kind != "int8_g32")
        cache.append(layer, k.to(DEV), v.to(DEV))
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    for i in range(steps):
        for layer in range(L):
            k1, v1 = _kv(B, H, 1, g, outliers=kind != "int8_g32")
            q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
            out = cache.append_decode_attn(layer, q.to(DEV), k1.to(DEV), v1.to(DEV), inv_tau=tau.to(DEV))
            torch.cuda.synchronize()
            n = S0 + i + 1
            assert cache.get_seq_len() == n or layer == 1
            if i in (0, 5, 6, 7, steps - 1):
                ref = _reference_out(K, kind, cache, layer, q, tau, n)
                assert_close(out, ref, f"{kind} layer {layer} S{n}")


def test_kivi_decode_range_check(monkeypatch):
    """KV_OOR_CHECK_INTERVAL selects the decode steps whose K is checked against the
    prefill's frozen per-channel range (src/cache/kivi_style_cache.py:549-560); the count
    is of the unrounded quotient (x - z) / s, so a token at 7.3 steps above the zero point
    (stored as code 7) counts.  With the default interval (0) no check runs."""
    K = _k()
    B, H = 1, 2
    base = torch.tensor([-1.0, 1.0]).repeat(8)[:, None].expand(16, 128)      # min -1, max 1
    k0 = base.expand(B, H, 16, 128).to(torch.float16).contiguous()
    v0 = torch.randn(B, H, 16, 128, generator=gen(77)).to(torch.float16)
    s = 2.0 / 15.0
    x = -1.0 + 15.3 * s                                                      # (x - z) / s = 7.3
    k1 = torch.full((B, H, 1, 128), x, dtype=torch.float16)
    v1 = torch.randn(B, H, 1, 128, generator=gen(78)).to(torch.float16)
    for interval, expect in (("0", False), ("1", True)):
        monkeypatch.setenv("KV_OOR_CHECK_INTERVAL", interval)
        cache = K.KIVIStyleKVCache(num_layers=1, device=DEV, quant_bits=4)
        cache.append(0, k0.to(DEV), v0.to(DEV))
        with warnings.catch_warnings(record=True) as rec:
            warnings.simplefilter("always")
            cache.append(0, k1.to(DEV), v1.to(DEV))
        hits = [r for r in rec if "ENG-041" in str(r.message)]
        assert bool(hits) == expect, (interval, [str(r.message) for r in rec])
        kp = cache.get_int4_asym_tensors(0)[0][0, 0, 16].view(torch.uint8).cpu()
        assert torch.all(kp == 0xFF)                                          # codes 7, 7 stored


# ---------------------------------------------------------------- MixedKVCache


@pytest.mark.parametrize("k_gs,pct,S0,Hq", [(128, 99.9, 37, 12), (32, 99.9, 300, 14), (16, 99.0, 5, 8),
                                            (64, 100.0, 1, 4)])
def test_mixed_cache_append_bitexact_and_decode(k_gs, pct, S0, Hq):
    """MixedKVCache (K INT8 with a dynamic percentile-clipped scale per token and group, V
    INT4 asymmetric per token): prefill and decode appends bit-exact with the oracle's
    quantize_symmetric_int8 / quantize_asymmetric_per_token (codes, fp16 K scales, fp32 V
    scale and zero-point), decode attention within max-abs 2e-3 / cosine 0.9999 of the
    dequantise-then-attention oracle (including a one-token context), get_kv exactly the
    reference's dequantisation."""
    K = _k()
    print(f"[case] mixed gs={k_gs} p={pct} S0={S0} Hq={Hq}", flush=True)
    g = gen(600 + k_gs + S0)
    B, H, steps = 2, 2, 3
    cache = K.MixedKVCache(1, device=DEV, k_group_size=k_gs, k_clip_percentile=pct)
    ks_, vs_ = [], []
    k0, v0 = _kv(B, H, S0, g)
    v0 = (v0.float() * torch.rand(B, H, S0, 1, generator=g) * 6 + torch.randn(B, H, S0, 1, generator=g) * 3)
    v0 = v0.to(torch.float16)
    cache.append(0, k0.to(DEV), v0.to(DEV))
    ks_.append(k0); vs_.append(v0)
    for _ in range(steps):
        k1, v1 = _kv(B, H, 1, g)
        cache.append(0, k1.to(DEV), v1.to(DEV))
        ks_.append(k1); vs_.append(v1)
    torch.cuda.synchronize()
    n = S0 + steps
    assert cache.get_seq_len() == n
    kc, ksc, vp, vsc, vz = [x.cpu() for x in cache.get_mixed_tensors(0)]
    rk, rks, rv, rvs, rvz = [], [], [], [], []
    for k, v in zip(ks_, vs_):  # the reference quantizes each append on its own
        a, b_ = OQ.quantize_symmetric_int8(k, pct, k_gs)
        c, d, e = OQ.quantize_asymmetric_per_token(v, 4, 100.0)
        rk.append(a); rks.append(b_); rv.append(c); rvs.append(d); rvz.append(e)
    assert torch.equal(kc, torch.cat(rk, 2))
    assert torch.equal(ksc.float(), torch.cat(rks, 2).float())
    assert torch.equal(vp, OQ.pack_int4(torch.cat(rv, 2)))
    assert torch.equal(vsc, torch.cat(rvs, 2)) and torch.equal(vz, torch.cat(rvz, 2))
    k_deq, v_deq = cache.get_kv(0)
    assert torch.equal(k_deq.cpu(), OQ.dequantize_symmetric(kc, ksc.float()).to(torch.float16))
    assert torch.equal(v_deq.cpu(), OQ.dequantize_kivi(OQ.unpack_int4(vp), vsc, vz, False).to(torch.float16))
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
    out = cache.decode_attn(0, q.to(DEV), inv_tau=tau.to(DEV))
    torch.cuda.synchronize()
    ref = OA.decode_attn_mixed_ref(q, kc, ksc, OQ.unpack_int4(vp), vsc, vz, torch.full((B,), n), 1 / math.sqrt(128),
                                   inv_tau=tau)
    assert_close_ulp(out, ref, f"mixed gs{k_gs} S{n}")


def test_int4_engine_unpacked_view():
    """INT4KVCache(bit_packed=False) (src/cache/int4_cache.py:55, 531-537, 623-625): the same
    codes as the packed engine, returned unpacked by get_int4_tensors (int8 codes in [-7, 7],
    [B, H, S, D]), which decode_attn_int4(bit_packed=False) takes; the decode step gives the
    packed engine's bits."""
    K = _k()
    g = gen(410)
    B, H, Hq, S = 2, 2, 12, 90
    st = torch.rand(1, H, 4, generator=g) * 0.5 + 0.05
    caches = [K.INT4KVCache(1, device=DEV, group_size=32, static_k_scale=st.to(DEV), static_v_scale=st.to(DEV),
                            bit_packed=bp, check_numerics=False) for bp in (True, False)]
    k, v = _kv(B, H, S + 1, g)
    for c in caches:
        c.append(0, k[:, :, :S].to(DEV), v[:, :, :S].to(DEV))
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16).to(DEV)
    outs = [c.append_decode_attn(0, q, k[:, :, S:].to(DEV), v[:, :, S:].to(DEV)) for c in caches]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    kp, vp, ks, vs = caches[0].get_int4_tensors(0)
    ku, vu, ks2, vs2 = caches[1].get_int4_tensors(0)
    assert ku.dtype == torch.int8 and ku.shape == (B, H, S + 1, 128) and caches[1].bit_packed is False
    assert torch.equal(ku.cpu(), OQ.unpack_int4(kp.cpu())) and torch.equal(vu.cpu(), OQ.unpack_int4(vp.cpu()))
    assert int(ku.abs().max()) <= 7 and torch.equal(ks, ks2) and torch.equal(vs, vs2)
    ctx = torch.full((B,), S + 1, dtype=torch.int32, device=DEV)
    # the kernel wrappers take fp16 scales, as the reference's (the hook casts the engines' fp32)
    ks16, vs16 = ks.half(), vs.half()
    a = K.decode_attn_int4(q, kp, vp, ks16, vs16, ctx, 1 / math.sqrt(128), bit_packed=True)
    b = K.decode_attn_int4(q, ku, vu, ks2.half(), vs2.half(), ctx, 1 / math.sqrt(128), bit_packed=False)
    torch.cuda.synchronize()
    ref = OA.decode_attn_int4_torch_ref(q.cpu(), kp.cpu(), vp.cpu(), ks16.cpu(), vs16.cpu(), ctx.cpu(),
                                        1 / math.sqrt(128))
    assert_close_ulp(a, ref, "int4 packed")
    assert_close_ulp(b, ref, "int4 unpacked")
    assert torch.equal(caches[0].get_kv(0)[0], caches[1].get_kv(0)[0])
