"""Pins of the KIVI-layout oracle (oracle/quant.py quantize_asymmetric*, dequantize_kivi,
oracle/attn.py decode_attn_kivi_ref).

The checks restate the reference's own tests of src/quant/asymmetric_quant.py
(tests/test_asymmetric_quant.py:112-282: manual min/max semantics, round trips, constant and
shifted data) and add what the arithmetic fixes: the minimum and maximum of each reduced
slice land on codes qmin and qmax, every in-range element is within s/2 of its
reconstruction, the parameters reduce over the right axis, and the attention matches an
independent float64 brute force that unpacks the nibbles with integer arithmetic.
"""
import math

import numpy as np
import torch

from oracle import attn as OA
from oracle import quant as OQ


def test_manual_min_max_semantics_both_axes():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 2, 8, 16, generator=g)
    for fn, dim in ((OQ.quantize_asymmetric_per_channel, 2), (OQ.quantize_asymmetric_per_token, 3)):
        for bits, qmin, span in ((8, -128, 255.0), (4, -8, 15.0)):
            _, s, z = fn(x, quant_bits=bits)
            mn, mx = x.amin(dim=dim), x.amax(dim=dim)
            floor = max(1e-5, float(torch.finfo(torch.float16).tiny) * span)
            es = (mx - mn).clamp(min=floor) / span
            assert torch.equal(s, es)
            assert torch.equal(z, mn - qmin * es)


def test_extremes_map_to_code_range_and_error_bound():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 40, 128, generator=g) * 3 + 1
    q, s, z = OQ.quantize_asymmetric_per_token(x, 4)
    assert q.dtype == torch.int8 and q.min() >= -8 and q.max() <= 7
    # per token: the argmin is code -8, the argmax code 7
    imin, imax = x.argmin(dim=-1, keepdim=True), x.argmax(dim=-1, keepdim=True)
    assert (q.gather(-1, imin) == -8).all() and (q.gather(-1, imax) == 7).all()
    xh = OQ.dequantize_kivi(q, s, z, per_channel=False)
    assert ((x - xh).abs() <= s.unsqueeze(-1) * 0.5 * (1 + 1e-5) + 1e-6).all()
    qk, sk, zk = OQ.quantize_asymmetric_per_channel(x, 4)
    assert sk.shape == (2, 3, 128)
    jmin, jmax = x.argmin(dim=2, keepdim=True), x.argmax(dim=2, keepdim=True)
    assert (qk.gather(2, jmin) == -8).all() and (qk.gather(2, jmax) == 7).all()
    xk = OQ.dequantize_kivi(qk, sk, zk, per_channel=True)
    assert ((x - xk).abs() <= sk.unsqueeze(2) * 0.5 * (1 + 1e-5) + 1e-6).all()
    # decode-time K with the frozen parameters reproduces the prefill codes
    assert torch.equal(OQ.kivi_quantize_k_static(x, sk, zk), qk)


def test_constant_zero_and_shifted_data():
    x0 = torch.zeros(1, 2, 4, 8)
    q, s, z = OQ.quantize_asymmetric_per_token(x0, 8)
    assert OQ.dequantize_kivi(q, s, z, False).abs().max().item() < 1e-4
    xc = torch.full((1, 2, 4, 8), 3.14)
    q, s, z = OQ.quantize_asymmetric_per_token(xc, 4)
    assert (q == -8).all()  # (x - (x + 8 s)) / s = -8
    assert (OQ.dequantize_kivi(q, s, z, False) - xc).abs().max().item() < 0.1
    g = torch.Generator().manual_seed(9)
    xs = torch.randn(1, 2, 8, 16, generator=g) + 5.0
    q, s, z = OQ.quantize_asymmetric_per_token(xs, 8)
    assert (xs - OQ.dequantize_kivi(q, s, z, False)).abs().mean().item() < 0.1


def test_decode_kivi_ref_matches_float64_brute_force():
    g = torch.Generator().manual_seed(21)
    B, Hq, Hkv, S, D = 2, 4, 2, 9, 128
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    kp = torch.randint(0, 256, (B, Hkv, S, D // 2), generator=g, dtype=torch.uint8)
    vp = torch.randint(0, 256, (B, Hkv, S, D // 2), generator=g, dtype=torch.uint8)
    ks, kz = torch.rand(B, Hkv, D, generator=g) * 0.3, torch.randn(B, Hkv, D, generator=g)
    vs, vz = torch.rand(B, Hkv, S, generator=g) * 0.3, torch.randn(B, Hkv, S, generator=g)
    ctx = torch.tensor([9, 4], dtype=torch.int32)
    sm = 1 / math.sqrt(D)
    out = OA.decode_attn_kivi_ref(q, kp, vp, ks, kz, vs, vz, ctx, sm)
    rep = Hq // Hkv
    for b in range(B):
        for h in range(Hq):
            kh = h // rep
            n = int(ctx[b])
            logits = []
            for t in range(n):
                acc = 0.0
                for d in range(D):
                    byte = int(kp[b, kh, t, d // 2])
                    nib = (byte >> 4) if d % 2 == 0 else (byte & 15)
                    kv = (nib - 8) * float(ks[b, kh, d]) + float(kz[b, kh, d])
                    acc += float(q[b, h, d]) * kv
                logits.append(acc * sm)
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            tot = sum(w)
            for d in range(0, D, 17):
                o = 0.0
                for t in range(n):
                    byte = int(vp[b, kh, t, d // 2])
                    nib = (byte >> 4) if d % 2 == 0 else (byte & 15)
                    o += w[t] * ((nib - 8) * float(vs[b, kh, t]) + float(vz[b, kh, t]))
                assert abs(o / tot - float(out[b, h, d])) <= 2e-3, (b, h, d)


def _f32_quantile_closed_form(vals, q):
    """torch.quantile of one 1-D float32 set, restated: fp32 rank = fp32(q) * (n - 1), the
    order statistics at floor / ceil, and ATen's lerp as one fused multiply-add computed in
    exact rational arithmetic (fma(w, b - a, a) for w < 0.5, else fma(w - 1, b - a, b))."""
    import numpy as np
    from fractions import Fraction

    v = np.sort(np.asarray(vals, dtype=np.float32))
    rank = np.float32(q) * np.float32(len(v) - 1)
    lo, hi = int(np.floor(rank)), int(np.ceil(rank))
    w = np.float32(rank - np.float32(lo))
    a, b = v[lo], v[hi]
    diff = np.float32(b - a)
    if w < 0.5:
        exact = Fraction(float(w)) * Fraction(float(diff)) + Fraction(float(a))
    else:
        exact = Fraction(float(np.float32(w - np.float32(1.0)))) * Fraction(float(diff)) + Fraction(float(b))
    return np.float32(float(exact))


def test_two_tailed_percentile_parameters_closed_form():
    """quantize_asymmetric with a percentile below 100 (src/quant/asymmetric_quant.py:97-103)
    takes torch.quantile at (100 - p) / 100 and p / 100 of each token (V) or channel (K):
    s and z equal the closed form from independently computed order statistics, bit for bit,
    for 4 and 8 bits; swapping the two levels, or using the upper level for both tails, gives
    other parameters."""
    import numpy as np

    g = torch.Generator().manual_seed(33)
    x = torch.randn(2, 2, 6, 128, generator=g) * 2
    x[0, 0, 1, 7] = 40.0  # one outlier the clipping removes
    for bits, qmin, span in ((4, -8, 15.0), (8, -128, 255.0)):
        for p in (99.9, 99.0, 97.5):
            qlo, qhi = (100.0 - p) / 100.0, p / 100.0
            _, s, z = OQ.quantize_asymmetric_per_token(x, bits, p)
            floor = np.float32(max(1e-5, float(torch.finfo(torch.float16).tiny) * span))
            for b in range(2):
                for h in range(2):
                    for t in range(6):
                        row = x[b, h, t].numpy()
                        mn, mx = _f32_quantile_closed_form(row, qlo), _f32_quantile_closed_form(row, qhi)
                        es = np.float32(max(np.float32(mx - mn), floor) / np.float32(span))
                        ez = np.float32(mn - np.float32(qmin) * es)
                        assert s[b, h, t].item() == es and z[b, h, t].item() == ez, (bits, p, b, h, t)
                        wrong = np.float32(max(np.float32(mx - _f32_quantile_closed_form(row, 1 - qhi)), floor)
                                           / np.float32(span))
                        if p == 97.5:
                            assert wrong != es or mn == _f32_quantile_closed_form(row, 1 - qhi)
            # K: the same levels over the tokens of each channel
            _, sk, zk = OQ.quantize_asymmetric_per_channel(x, bits, p)
            col = x[1, 0, :, 5].numpy()
            mn, mx = _f32_quantile_closed_form(col, qlo), _f32_quantile_closed_form(col, qhi)
            es = np.float32(max(np.float32(mx - mn), floor) / np.float32(span))
            assert sk[1, 0, 5].item() == es and zk[1, 0, 5].item() == np.float32(mn - np.float32(qmin) * es)


def test_kivi_family_ref_brute_force_mixed_bits():
    """decode_attn_kivi_family_ref for (8, 16) and (16, 4): float64 brute force with explicit
    per-element dequantisation (int8 codes x per-channel s + z; fp16 values as stored; packed
    nibbles unpacked with integer arithmetic)."""
    g = torch.Generator().manual_seed(44)
    B, Hq, Hkv, S, D = 1, 4, 2, 7, 128
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    k8 = torch.randint(-128, 128, (B, Hkv, S, D), generator=g, dtype=torch.int8)
    ks, kz = torch.rand(B, Hkv, D, generator=g) * 0.02, torch.randn(B, Hkv, D, generator=g) * 0.1
    k16 = torch.randn(B, Hkv, S, D, generator=g).to(torch.float16)
    v16 = torch.randn(B, Hkv, S, D, generator=g).to(torch.float16)
    vp = torch.randint(0, 256, (B, Hkv, S, D // 2), generator=g, dtype=torch.uint8).view(torch.int8)
    vs, vz = torch.rand(B, Hkv, S, generator=g) * 0.3, torch.randn(B, Hkv, S, generator=g)
    ctx = torch.tensor([6], dtype=torch.int32)
    sm = 1 / math.sqrt(D)
    cases = [(8, 16), (16, 4)]
    for kb, vb in cases:
        kstore = k8 if kb == 8 else k16
        vstore = v16 if vb == 16 else vp
        out = OA.decode_attn_kivi_family_ref(q, kstore, kb, ks if kb == 8 else None, kz if kb == 8 else None,
                                             vstore, vb, vs if vb == 4 else None, vz if vb == 4 else None,
                                             ctx, sm)
        for h in range(Hq):
            kh = h // 2
            n = int(ctx[0])
            logits = []
            for t in range(n):
                acc = 0.0
                for d in range(D):
                    kv = (int(k8[0, kh, t, d]) * float(ks[0, kh, d]) + float(kz[0, kh, d])) if kb == 8 \
                        else float(k16[0, kh, t, d])
                    acc += float(q[0, h, d]) * kv
                logits.append(acc * sm)
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            tot = sum(w)
            for d in range(0, D, 13):
                o = 0.0
                for t in range(n):
                    if vb == 16:
                        vv = float(v16[0, kh, t, d])
                    else:
                        byte = int(vp[0, kh, t, d // 2]) & 0xFF
                        nib = (byte >> 4) if d % 2 == 0 else (byte & 15)
                        vv = (nib - 8) * float(vs[0, kh, t]) + float(vz[0, kh, t])
                    o += w[t] * vv
                assert abs(o / tot - float(out[0, h, d])) <= 2e-3, (kb, vb, h, d)


def test_mixed_bits_ref_k4_brute_force():
    """decode_attn_mixed_bits_ref with a 4-bit K (MixedKVCache K at 4 bits: asymmetric per
    token, src/cache/mixed_kv_cache.py:159-162, 186-188) against a float64 brute force that
    unpacks the nibbles with integer arithmetic and rounds each dequantised K element to
    fp16, with V at 8 bits (per-group scales) and at 16 bits.  A K dequantised per channel,
    or without the zero-point, misses it."""
    g = torch.Generator().manual_seed(45)
    B, Hq, Hkv, S, D = 1, 4, 2, 9, 128
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    kp = torch.randint(0, 256, (B, Hkv, S, D // 2), generator=g, dtype=torch.uint8).view(torch.int8)
    ks, kz = torch.rand(B, Hkv, S, generator=g) * 0.4 + 0.05, torch.randn(B, Hkv, S, generator=g)
    v8 = torch.randint(-127, 128, (B, Hkv, S, D), generator=g, dtype=torch.int8)
    vs8 = (torch.rand(B, Hkv, S, 4, generator=g) * 0.02 + 0.001).to(torch.float16)
    v16 = torch.randn(B, Hkv, S, D, generator=g).to(torch.float16)
    ctx = torch.tensor([8], dtype=torch.int32)
    sm = 1 / math.sqrt(D)
    for vb in (8, 16):
        out = OA.decode_attn_mixed_bits_ref(q, kp, 4, ks, v8 if vb == 8 else v16, vb,
                                            vs8 if vb == 8 else None, None, ctx, sm, k_zp=kz)
        for h in range(Hq):
            kh = h // 2
            n = int(ctx[0])
            logits = []
            for t in range(n):
                acc = 0.0
                for d in range(D):
                    byte = int(kp[0, kh, t, d // 2]) & 0xFF
                    nib = (byte >> 4) if d % 2 == 0 else (byte & 15)
                    kv = float(np.float16(np.float32((nib - 8) * np.float32(ks[0, kh, t]) +
                                                     np.float32(kz[0, kh, t]))))
                    acc += float(q[0, h, d]) * kv
                logits.append(acc * sm)
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            tot = sum(w)
            for d in range(0, D, 11):
                o = 0.0
                for t in range(n):
                    vv = (int(v8[0, kh, t, d]) * float(vs8[0, kh, t, d // 32])) if vb == 8 \
                        else float(v16[0, kh, t, d])
                    o += w[t] * vv
                assert abs(o / tot - float(out[0, h, d])) <= 2e-3, (vb, h, d)
    # the plausible mistakes: no zero-point, or the parameters taken per channel
    bad = OA.decode_attn_mixed_bits_ref(q, kp, 4, ks, v16, 16, None, None, ctx, sm, k_zp=torch.zeros_like(kz))
    good = OA.decode_attn_mixed_bits_ref(q, kp, 4, ks, v16, 16, None, None, ctx, sm, k_zp=kz)
    assert (bad.float() - good.float()).abs().max() > 1e-2
