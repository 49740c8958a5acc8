"""GPU tests of the KIVI family and the mixed bit pairs against the CPU oracle.

* KIVIStyleKVCache with quant_bits 8 (the reference's default) and 4, with and without
  percentile clipping (k_percentile over the prefill's tokens per channel, v_percentile over
  each token's channels in the append kernel): codes, scales and zero-points bit-exact with
  the oracle's quantize_asymmetric_* (torch.quantile semantics), decode attention within
  max-abs 2e-3 (or one fp16 ulp where |out| >= 4) and cosine 0.9999.
* RoleAwareAllocatorKVCache with every (k_bits, v_bits) pair from {4, 8, 16} on its own layer.
* MixedKVCache pairs (8, 8), (8, 16), (16, 4), (16, 16) and V percentile clipping.
"""
import math

import pytest
import torch

from oracle import attn as OA
from oracle import quant as OQ

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL = 2e-3
COS_MIN = 0.9999


def _k():
    import llm_kvcache_quantization_amd as K
    from llm_kvcache_quantization_amd import _capi

    _capi.lib()
    return K


def gen(seed):
    return torch.Generator().manual_seed(seed)


def fp16_ulp(x):
    a = x.abs().float().clamp(min=2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


def assert_close_ulp(out, ref, tag):
    """max-abs 2e-3, or one fp16 ulp of the oracle's value where that is larger (|out| >= 4:
    neighbouring fp16 values are more than 2e-3 apart there), and cosine >= 0.9999."""
    o, r = out.detach().float().cpu(), ref.detach().float().cpu()
    assert o.shape == r.shape and torch.isfinite(o).all(), tag
    err = (o - r).abs()
    worst = (err - torch.maximum(torch.full_like(r, ATOL), fp16_ulp(r))).max().item()
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r.flatten(), dim=0).item()
    print(f"[{tag}] max_abs={err.max().item():.3e} max|ref|={r.abs().max().item():.2f} "
          f"excess={worst:.3e} cos={cos:.7f}", flush=True)
    assert worst <= 0 and cos >= COS_MIN, (tag, worst, cos)


def _kv(B, H, S, g, ties=False):
    k = torch.randn(B, H, S, 128, generator=g) * 1.5
    k[..., 3] *= 15.0
    k[..., 90] = k[..., 90] * 8.0 + 4.0
    v = torch.randn(B, H, S, 128, generator=g) * (torch.rand(B, H, S, 1, generator=g) * 3 + 0.2)
    v = v + torch.randn(B, H, S, 1, generator=g)
    if ties:
        k, v = (k * 2).round() / 2, (v * 2).round() / 2
    return k.to(torch.float16), v.to(torch.float16)


def _store(codes, bits):
    return OQ.pack_int4(codes) if bits == 4 else codes


def _ref_layer(kb, vb, k_list, v_list, kp, vp):
    """The oracle's stored K / V sides of a KIVI-family layer appended in the pieces k_list /
    v_list (the first is the prefill): (k_store, k_s, k_z, v_store, v_s, v_z)."""
    k_all = torch.cat(k_list, 2)
    if kb == 16:
        ks_ = kz_ = None
        k_store = k_all
    else:
        q0, ks_, kz_ = OQ.quantize_asymmetric_per_channel(k_list[0], kb, kp)
        codes = [q0] + [OQ.kivi_quantize_k_static(k, ks_, kz_, kb) for k in k_list[1:]]
        k_store = _store(torch.cat(codes, 2), kb)
    if vb == 16:
        v_store, vs_, vz_ = torch.cat(v_list, 2), None, None
    else:
        parts = [OQ.quantize_asymmetric_per_token(v, vb, vp) for v in v_list]
        v_store = _store(torch.cat([p[0] for p in parts], 2), vb)
        vs_, vz_ = torch.cat([p[1] for p in parts], 2), torch.cat([p[2] for p in parts], 2)
    return k_store, ks_, kz_, v_store, vs_, vz_


def _check_codes(cache, layer, kb, vb, k_list, v_list, kp, vp, tag):
    kc, vc, ks, kz, vs, vz = [None if t is None else t.cpu() for t in cache.get_kivi_tensors(layer)]
    rk, rks, rkz, rv, rvs, rvz = _ref_layer(kb, vb, k_list, v_list, kp, vp)
    assert torch.equal(kc, rk), f"{tag} K codes"
    assert torch.equal(vc, rv), f"{tag} V codes"
    if kb != 16:
        assert torch.equal(ks, rks) and torch.equal(kz, rkz), f"{tag} K params"
    if vb != 16:
        assert torch.equal(vs, rvs) and torch.equal(vz, rvz), f"{tag} V params"
    return kc, vc, ks, kz, vs, vz


def _check_layer(K, cache, layer, kb, vb, k_list, v_list, kp, vp, g, Hq, tag):
    kc, vc, ks, kz, vs, vz = _check_codes(cache, layer, kb, vb, k_list, v_list, kp, vp, tag)
    B = kc.shape[0]
    n = kc.shape[2]
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
    out = cache.decode_attn(layer, q.to(DEV))
    torch.cuda.synchronize()
    ref = OA.decode_attn_kivi_family_ref(q, kc, kb, ks, kz, vc, vb, vs, vz, torch.full((B,), n),
                                         1 / math.sqrt(128))
    assert_close_ulp(out, ref, tag)
    k_deq, v_deq = cache.get_kv(layer)
    assert torch.equal(k_deq.cpu(), OA.dequant_kivi_side(kc, kb, ks, kz, True).to(torch.float16))
    assert torch.equal(v_deq.cpu(), OA.dequant_kivi_side(vc, vb, vs, vz, False).to(torch.float16))


@pytest.mark.parametrize("bits,kp,vp,ties", [
    (8, 100.0, 100.0, False), (4, 100.0, 100.0, False),
    (8, 99.5, 99.9, False), (4, 99.5, 99.9, False), (4, 99.0, 97.0, True), (8, 100.0, 99.9, True),
])
def test_kivi_cache_bits_and_percentiles(bits, kp, vp, ties):
    K = _k()
    print(f"[case] kivi bits={bits} kp={kp} vp={vp} ties={ties}", flush=True)
    g = gen(700 + bits + int(kp * 10) + int(vp) + ties)
    B, H, S0, steps = 2, 2, 300, 4
    cache = K.KIVIStyleKVCache(1, device=DEV, quant_bits=bits, k_percentile=kp, v_percentile=vp)
    k0, v0 = _kv(B, H, S0, g, ties)
    cache.append(0, k0.to(DEV), v0.to(DEV))
    ks_, vs_ = [k0], [v0]
    for _ in range(steps):
        k1, v1 = _kv(B, H, 1, g, ties)
        cache.append(0, k1.to(DEV), v1.to(DEV))
        ks_.append(k1)
        vs_.append(v1)
    torch.cuda.synchronize()
    assert cache.get_seq_len() == S0 + steps
    _check_layer(K, cache, 0, bits, bits, ks_, vs_, kp, vp, g, 14, f"kivi{bits} kp{kp} vp{vp}")


PAIRS = [(4, 4), (8, 8), (4, 8), (8, 4), (16, 4), (4, 16), (16, 16), (8, 16), (16, 8)]


def test_allocator_every_bit_pair():
    """RoleAwareAllocatorKVCache with each (k_bits, v_bits) pair on its own layer, prefill and
    decode steps through append_decode_attn (the cached kernel parameters and growth past the
    first capacity), clipping percentiles 99.9 / 99.5."""
    K = _k()
    g = gen(811)
    L, B, H, Hq, S0, steps = len(PAIRS), 2, 2, 8, 250, 9
    cache = K.RoleAwareAllocatorKVCache(L, per_layer_bits=PAIRS, device=DEV, k_percentile=99.9,
                                        v_percentile=99.5)
    hist = []
    for layer in range(L):
        k0, v0 = _kv(B, H, S0, g)
        cache.append(layer, k0.to(DEV), v0.to(DEV))
        hist.append(([k0], [v0]))
    for i in range(steps):
        for layer, (kb, vb) in enumerate(PAIRS):
            k1, v1 = _kv(B, H, 1, g)
            q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
            out = cache.append_decode_attn(layer, q.to(DEV), k1.to(DEV), v1.to(DEV))
            hist[layer][0].append(k1)
            hist[layer][1].append(v1)
            if i in (0, steps - 1):
                torch.cuda.synchronize()
                kc, vc, ks, kz, vs, vz = [None if t is None else t.cpu() for t in cache.get_kivi_tensors(layer)]
                n = S0 + i + 1
                ref = OA.decode_attn_kivi_family_ref(q, kc, kb, ks, kz, vc, vb, vs, vz, torch.full((B,), n),
                                                     1 / math.sqrt(128))
                assert_close_ulp(out, ref, f"alloc ({kb},{vb}) S{n}")
    torch.cuda.synchronize()
    for layer, (kb, vb) in enumerate(PAIRS):
        _check_layer(K, cache, layer, kb, vb, hist[layer][0], hist[layer][1], 99.9, 99.5, g, Hq,
                     f"alloc ({kb},{vb}) final")
    assert len(cache.to_tuple()) == L


@pytest.mark.parametrize("kb,vb,gs,vgs,vp,kp", [
    (8, 8, 32, 32, 99.9, 99.9), (8, 16, 64, 64, 100.0, 99.9), (16, 4, 128, 128, 99.9, 99.9),
    (16, 16, 128, 128, 100.0, 99.9), (8, 4, 128, 128, 99.9, 99.9),
    # K at 4 bits (asymmetric per token, k_clip_percentile), fp16 K with INT8 V, and INT8 K and
    # V with their own group sizes
    (4, 4, 128, 128, 99.9, 99.9), (4, 8, 128, 32, 100.0, 99.0), (4, 16, 128, 128, 99.9, 100.0),
    (16, 8, 128, 16, 99.9, 99.9), (8, 8, 128, 32, 99.9, 99.5), (8, 8, 16, 64, 100.0, 99.9)])
def test_mixed_cache_bit_pairs(kb, vb, gs, vgs, vp, kp):
    K = _k()
    print(f"[case] mixed ({kb},{vb}) gs={gs} vgs={vgs} vp={vp} kp={kp}", flush=True)
    g = gen(900 + kb + vb + gs + vgs)
    B, H, Hq, S0, steps = 2, 2, 10, 70, 3
    cache = K.MixedKVCache(1, device=DEV, k_group_size=gs, v_group_size=vgs, k_bits=kb, v_bits=vb,
                           v_percentile=vp, k_clip_percentile=kp)
    ks_, vs_ = [], []
    k0, v0 = _kv(B, H, S0, g)
    cache.append(0, k0.to(DEV), v0.to(DEV))
    ks_.append(k0)
    vs_.append(v0)
    for _ in range(steps):
        k1, v1 = _kv(B, H, 1, g)
        cache.append(0, k1.to(DEV), v1.to(DEV))
        ks_.append(k1)
        vs_.append(v1)
    torch.cuda.synchronize()
    kc, ksc, vc, vsc, vz = [None if t is None else t.cpu() for t in cache.get_mixed_tensors(0)]
    kz = None
    if kb == 8:
        parts = [OQ.quantize_symmetric_int8(k, kp, gs) for k in ks_]
        assert torch.equal(kc, torch.cat([p[0] for p in parts], 2))
        assert torch.equal(ksc.float(), torch.cat([p[1] for p in parts], 2).float())
    elif kb == 4:
        kz = cache.get_k_zero_points(0).cpu()
        parts = [OQ.quantize_asymmetric_per_token(k, 4, kp) for k in ks_]
        assert torch.equal(kc, OQ.pack_int4(torch.cat([p[0] for p in parts], 2)))
        assert torch.equal(ksc, torch.cat([p[1] for p in parts], 2)) and torch.equal(kz, torch.cat([p[2] for p in parts], 2))
    else:
        assert torch.equal(kc, torch.cat(ks_, 2))
    if vb == 4:
        parts = [OQ.quantize_asymmetric_per_token(v, 4, vp) for v in vs_]
        assert torch.equal(vc, OQ.pack_int4(torch.cat([p[0] for p in parts], 2)))
        assert torch.equal(vsc, torch.cat([p[1] for p in parts], 2)) and torch.equal(vz, torch.cat([p[2] for p in parts], 2))
    elif vb == 8:
        parts = [OQ.quantize_symmetric_int8(v, vp, vgs) for v in vs_]
        assert torch.equal(vc, torch.cat([p[0] for p in parts], 2))
        assert torch.equal(vsc.float(), torch.cat([p[1] for p in parts], 2).float())
    else:
        assert torch.equal(vc, torch.cat(vs_, 2))
    n = S0 + steps
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
    out = cache.decode_attn(0, q.to(DEV), inv_tau=tau.to(DEV))
    torch.cuda.synchronize()
    ref = OA.decode_attn_mixed_bits_ref(q, kc, kb, ksc, vc, vb, vsc, vz, torch.full((B,), n),
                                        1 / math.sqrt(128), inv_tau=tau, k_zp=kz)
    assert_close_ulp(out, ref, f"mixed ({kb},{vb})")
    k_deq, v_deq = cache.get_kv(0)
    assert k_deq.shape == (B, H, n, 128) and v_deq.shape == (B, H, n, 128)


def test_fp16_pair_partial_tile_ignores_stale_rows():
    """A 16-bit V side reads whole 32-token tiles: rows past the context in the last tile may
    hold any fp16 bits (inf / NaN here) and must not reach the output."""
    K = _k()
    g = gen(950)
    cache = K.RoleAwareAllocatorKVCache(1, per_layer_bits=[(16, 16)], device=DEV)
    k0, v0 = _kv(1, 2, 40, g)
    cache.append(0, k0.to(DEV), v0.to(DEV))
    cache._v_cache[0][:, :, 40:64] = float("inf")
    cache._k_cache[0][:, :, 40:64] = float("nan")
    q = torch.randn(1, 4, 128, generator=g).to(torch.float16)
    out = cache.decode_attn(0, q.to(DEV))
    torch.cuda.synchronize()
    ref = OA.decode_attn_kivi_family_ref(q, k0, 16, None, None, v0, 16, None, None, torch.tensor([40]),
                                         1 / math.sqrt(128))
    assert_close_ulp(out, ref, "fp16 stale tail")


@pytest.mark.parametrize("bits,R,extra", [(4, 32, 5), (8, 16, 40), (4, 128, 0), (4, 4200, 3)])
def test_kivi_residual_window(bits, R, extra):
    """residual_length R (src/cache/kivi_style_cache.py:102-113, 354-404): after the prefill,
    decode tokens fill an fp16 window of R; each later token evicts the oldest into the
    quantized cache.  Codes bit-exact with the oracle over the evicted tokens, get_kv the
    dequantized cache followed by the window in arrival order, decode attention over both
    within the bound; the window alone (an empty quantized context) through the C ABI."""
    K = _k()
    print(f"[case] residual bits={bits} R={R} extra={extra}", flush=True)
    g = gen(1200 + bits + R + extra)
    B, H, Hq, S0 = 2, 2, 12, 70
    cache = K.KIVIStyleKVCache(1, device=DEV, quant_bits=bits, residual_length=R, v_percentile=99.9)
    k0, v0 = _kv(B, H, S0, g)
    cache.append(0, k0.to(DEV), v0.to(DEV))
    dec_k, dec_v = [], []
    for _ in range(R + extra):
        k1, v1 = _kv(B, H, 1, g)
        cache.append(0, k1.to(DEV), v1.to(DEV))
        dec_k.append(k1)
        dec_v.append(v1)
    torch.cuda.synchronize()
    assert cache.get_seq_len() == S0 + R + extra
    assert cache._layer_seq_lens[0] == S0 + extra and cache._res_len[0] == R
    kc, vc, ks, kz, vs, vz = _check_codes(cache, 0, bits, bits, [k0] + dec_k[:extra], [v0] + dec_v[:extra],
                                          100.0, 99.9, f"residual{bits} quantized part")
    k_all, v_all = cache.get_kv(0)
    win_k, win_v = torch.cat(dec_k[extra:], 2), torch.cat(dec_v[extra:], 2)
    assert torch.equal(k_all[:, :, S0 + extra:].cpu(), win_k) and torch.equal(v_all[:, :, S0 + extra:].cpu(), win_v)
    kd = torch.cat([OA.dequant_kivi_side(kc, bits, ks, kz, True), win_k.float()], 2)
    vd = torch.cat([OA.dequant_kivi_side(vc, bits, vs, vz, False), win_v.float()], 2)
    q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
    out = cache.decode_attn(0, q.to(DEV))
    torch.cuda.synchronize()
    ref = OA.attention_fp32(q, kd, vd, torch.full((B,), kd.shape[2]), 1 / math.sqrt(128))
    assert_close_ulp(out, ref, f"residual{bits} R{R} decode")
    # the window alone: a quantized context of 0 tokens
    st = cache._step_for(0, Hq)
    st.set_residual(cache._res_k[0], cache._res_v[0], R)
    out0 = st.attend(q.to(DEV), 0, 1 / math.sqrt(128))
    torch.cuda.synchronize()
    rk, rv = cache._res_k[0].cpu(), cache._res_v[0].cpu()
    ref0 = OA.attention_fp32(q, rk.float(), rv.float(), torch.full((B,), R), 1 / math.sqrt(128))
    assert_close_ulp(out0, ref0, f"residual{bits} R{R} window only")
