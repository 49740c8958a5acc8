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
