"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

How each oracle function is pinned, chosen so that a plausible mistake (a dropped
term, a wrong sign or index, a swapped nibble) fails at least one check:

* quantize_symmetric_int8_with_scale: exhaustive over every finite fp16 input and a
  sweep of scales, against a numpy closed form.  That closed form divides in float64,
  rounds to fp16, then to an integer with ties-to-even.  Double rounding is exact here
  because 53 >= 2*11 + 2.  Plus the clamp KATs.
* quantize_symmetric_int4_with_scale / dynamic INT4: numpy float64 -> float32 closed
  form, plus the KATs of reference tests/test_int4_cache.py:559-586.
* pack_int4 / unpack_int4: the KATs of tests/test_int4_cache.py:469-557 and the byte
  layout (high nibble = even element).
* quantize_asymmetric_static: numpy float32 closed form, plus the reference K
  quantize+pack formula of tests/test_fused_quantize_pack.py:8-17.
* outlier_rescue and the percentile-clipped dynamic quantizers: torch.quantile (the
  library routine the reference calls) against a float32 closed form -- the order
  statistics at floor / ceil of fp32(q) (n - 1) and ATen's CPU lerp, one fused
  multiply-add in exact rational arithmetic -- compared bitwise over 1500 random sets and
  every group of the quantizer tests.  The unfused a + w (b - a), a plausible
  restatement, misses torch in some of those cases (asserted).  The rescued set is
  checked against "values >= the interpolated threshold".
* decode_attn_int8_torch_ref: the KATs of tests/test_patch_model.py:280-368 (S=1 -> V,
  softmax [e/(e+1), 1/(e+1)], ctx=0 -> 0, GQA head h -> kv head h // n_rep), a float64
  brute force on tiny inputs, and permutation / scaling invariants.
* decode_attn_asym_ref: float64 brute force with explicit dequantisation.
* int8_cache_quantize(adaptive=True) (src/cache/int8_cache.py:389-453): known answers
  with scalar arithmetic per group -- a group whose absmax/127 lies between the static
  scale and static * margin takes static * margin, one above takes absmax/127, an all-zero
  group takes static * margin -- and the codes of the fp16 closed form.  The same data
  under the plausible mistakes (margin on the dynamic side, margin dropped, min for max)
  give other scales, so each mistake fails.
* int4_cache_quantize(adaptive / mixed_rescue / both / with outlier rescue)
  (src/cache/int4_cache.py:447-529): the same kind of known answers in fp32, and the
  reference's documented identity that outlier rescue after mixed rescue changes nothing
  (int4_cache.py:360-378).
* dequantize_symmetric / cache_get_kv: known answers (code x scale of its own group, the
  group index d // gs, per-token scalar scale) and the exactness of the fp32 product
  (an 8-bit code times an 11-bit fp16 scale is exact, so the cache's fp16 result is one
  rounding of the exact product, checked against float64).
* decode_attn_k8v4_ref: float64 brute force (INT8 K dequantised as the fp16 product the
  reference forms, asymmetric V in float64, q * inv_tau as an fp16 product).
* decode_attn_mixed_ref: float64 brute force with per-element dequantisation (K code x the
  scale of its token's group, V code x s_t + z_t of its token), a one-token known answer and
  a literal one (codes 3, -8, 7, 0 with s = 0.5, z = -1 give 0.5, -5, 2.5, -1).
* decode_attn_mixed_bits_ref: the (8, 4) pair equals decode_attn_mixed_ref bit for bit, and
  one-token contexts return the token's V for the 16- and 8-bit sides.
* The KIVI family (quantize_asymmetric with 8 bits and two-tailed percentiles,
  decode_attn_kivi_family_ref): tests/test_oracle_kivi.py.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import attn as OA
from oracle import quant as OQ


def all_finite_fp16():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    x = bits.view(np.float16)
    return x[np.isfinite(x)]


# ---------------------------------------------------------------- INT8


def int8_closed_form(x16: np.ndarray, s16: np.float16) -> np.ndarray:
    s = max(np.float64(s16), np.float64(np.float16(1e-5)))
    s = np.float16(s)
    qf = np.float16(x16.astype(np.float64) / np.float64(s))  # correctly rounded fp16 quotient
    q = np.rint(qf.astype(np.float64))
    return np.clip(q, -127, 127).astype(np.int8)


@pytest.mark.parametrize("s", [1e-6, 1.5e-5, 3.3e-4, 0.0078125, 0.0123, 0.37, 1.0, 3.7, 157.0])
def test_int8_exhaustive_fp16(s):
    x = all_finite_fp16()
    s16 = np.float16(s)
    expect = int8_closed_form(x, s16)
    xt = torch.from_numpy(x.copy()).view(1, 1, -1, 1).expand(1, 1, x.size, 32).contiguous()
    scale = torch.full((1, 1), float(s16), dtype=torch.float16)
    q, s_out = OQ.quantize_symmetric_int8_with_scale(xt, scale, 32)
    assert torch.equal(q[0, 0, :, 0], torch.from_numpy(expect))
    assert s_out.dtype == torch.float16


def test_int8_ties_round_to_even_and_clamp():
    # quotients exactly at .5 must round to even; |q| > 127 clamps
    x = torch.tensor([0.5, 1.5, 2.5, -0.5, -2.5, 200.0, -200.0, 126.5], dtype=torch.float16)
    xt = x.view(1, 1, 1, -1).repeat(1, 1, 1, 4)
    q, _ = OQ.quantize_symmetric_int8_with_scale(xt, torch.ones(1, 1, dtype=torch.float16), 32)
    assert q[0, 0, 0, :8].tolist() == [0, 2, 2, 0, -2, 127, -127, 126]


def test_int8_fp16_quotient_rounding_matters():
    # x/s lands just above k+0.5 in fp32 but rounds to exactly k+0.5 in fp16 -> rounds to even.
    # A plain fp32 quotient would give the next integer: this pins the fp16 step.
    x16 = np.float16(1.0009765625)  # 1 + 2^-10
    s16 = np.float16(0.4)
    q32 = np.rint(np.float32(x16) / np.float32(s16))
    qf16 = np.rint(np.float32(np.float16(np.float32(x16) / np.float32(s16))))
    cases = []
    for xv in all_finite_fp16()[::97]:
        a = np.rint(np.float64(np.float16(np.float64(xv) / np.float64(s16))))
        b = np.rint(np.float64(xv) / np.float64(s16))
        if a != b and abs(float(xv) / float(s16)) < 127:
            cases.append(xv)
    assert cases, "expected fp16-vs-fp32 quotient rounding differences"
    xt = torch.from_numpy(np.array(cases, dtype=np.float16)).view(1, 1, -1, 1).repeat(1, 1, 1, 32)
    q, _ = OQ.quantize_symmetric_int8_with_scale(xt, torch.full((1, 1), float(s16), dtype=torch.float16), 32)
    assert torch.equal(q[0, 0, :, 0], torch.from_numpy(int8_closed_form(np.array(cases, dtype=np.float16), s16)))
    del q32, qf16


def test_int8_dynamic_absmax():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 2, 3, 128, generator=g).to(torch.float16)
    q, s = OQ.quantize_symmetric_int8(x, 100.0, 32)
    xn = x.numpy().reshape(2, 2, 3, 4, 32)
    am = np.maximum(np.abs(xn).max(-1), np.float16(1e-5)).astype(np.float16)
    s_exp = np.float16(am.astype(np.float64) / 127.0)
    assert np.array_equal(s.numpy(), s_exp)
    qe = np.clip(np.rint(np.float16(xn.astype(np.float64) / s_exp[..., None].astype(np.float64)).astype(np.float64)), -127, 127)
    assert np.array_equal(q.numpy().reshape(2, 2, 3, 4, 32), qe.astype(np.int8))
    assert q.abs().max() == 127  # the absmax element maps to +-127


# ---------------------------------------------------------------- INT4 symmetric


def int4_closed_form(x16: np.ndarray, s32: np.ndarray) -> np.ndarray:
    s = np.maximum(s32.astype(np.float32), np.float32(1e-5))
    qf = (x16.astype(np.float64) / s.astype(np.float64)).astype(np.float32)
    return np.clip(np.rint(qf), -7, 7).astype(np.int8)


def test_int4_static_closed_form():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(3, 2, 17, 128, generator=g) * 3).to(torch.float16)
    scale = (torch.rand(2, 4, generator=g) * 0.5 + 1e-6).float()
    q, s = OQ.quantize_symmetric_int4_with_scale(x, scale, 32)
    xn = x.numpy().reshape(3, 2, 17, 4, 32)
    sn = scale.numpy()[None, :, None, :, None]
    assert np.array_equal(q.numpy().reshape(3, 2, 17, 4, 32), int4_closed_form(xn, sn))
    assert s.dtype == torch.float32
    assert torch.equal(s[0, :, 0], scale.clamp(min=1e-5))


def test_int4_kat_boundaries():
    # reference tests/test_int4_cache.py:559-586
    for val, code in ((7.0, 7), (-7.0, -7), (0.0, 0)):
        q, _ = OQ.quantize_symmetric_int4(torch.full((1, 1, 1, 128), val), 100.0, 128)
        assert (q == code).all()
    q, _ = OQ.quantize_symmetric_int4(torch.randn(1, 1, 1, 128) * 1000, 100.0, 128)
    assert q.min() >= -7 and q.max() <= 7


def test_pack_unpack_kats():
    # reference tests/test_int4_cache.py:469-557
    vals = torch.arange(-8, 8, dtype=torch.int8).view(1, 1, 1, 16)
    assert torch.equal(OQ.unpack_int4(OQ.pack_int4(vals)), vals)
    for a, b in [(-8, 7), (7, -8), (-8, -8), (7, 7), (0, 0), (-1, 1)]:
        x = torch.tensor([a, b], dtype=torch.int8).view(1, 1, 1, 2)
        p = OQ.pack_int4(x)
        assert int(p.view(torch.uint8)) == ((a + 8) << 4) | (b + 8)  # high nibble = even element
        assert torch.equal(OQ.unpack_int4(p), x)


def fused_lerp32(a, b, w):
    """torch.quantile's interpolation as ATen's CPU lerp computes it, one rounding per
    fused multiply-add (exact rational arithmetic, then the nearest float32)."""
    a, b, w = np.float32(a), np.float32(b), np.float32(w)
    d = Fraction(float(np.float32(b - a)))
    if w < 0.5:
        exact = Fraction(float(w)) * d + Fraction(float(a))
    else:
        exact = Fraction(float(np.float32(w - np.float32(1)))) * d + Fraction(float(b))
    return np.float32(float(exact))


def quantile32(v, q):
    """Closed form of torch.quantile(v, q) (linear) in float32: rank = fp32(q) * (n - 1),
    the order statistics at floor / ceil of it, fused_lerp32 between them."""
    s = np.sort(np.asarray(v, dtype=np.float32))
    n = s.shape[0]
    rank = np.float32(np.float32(q) * np.float32(n - 1))
    lo, hi = int(np.floor(rank)), int(np.ceil(rank))
    return fused_lerp32(s[lo], s[hi], np.float32(rank - np.float32(lo))), s[lo], s[hi]


def test_rescue_quantile_matches_torch_and_closed_form():
    rng = np.random.default_rng(0)
    unfused_misses = 0
    for trial in range(1500):
        n = int(rng.choice([1, 2, 3, 16, 127, 128, 129, 512, 4096, int(rng.integers(5, 6000))]))
        ratio = float(rng.choice([0.01, 0.05, 0.3, 0.5, 0.999, 0.0025]))
        v = (np.abs(rng.standard_normal(n)) * rng.uniform(0.1, 10)).astype(np.float32)
        if n > 8:
            v[rng.integers(0, n, 3)] = v[0]  # ties
        q = max(0.0, min(1.0, 1.0 - ratio))
        ref = np.float32(torch.quantile(torch.from_numpy(v), q).item())
        thr, a, b = quantile32(v, q)
        assert ref == thr, (n, ratio, ref, thr)
        # the unfused a + w (b - a) (a plausible restatement) misses in some of these cases
        rank = np.float32(np.float32(q) * np.float32(n - 1))
        w = np.float32(rank - np.float32(np.floor(rank)))
        d = np.float32(b - a)
        unf = np.float32(a + np.float32(w * d)) if w < 0.5 else np.float32(b - np.float32(d * np.float32(1 - w)))
        unfused_misses += int(unf != ref)
        # rescued set: everything >= sorted[hi], plus sorted[lo] only if thr == sorted[lo]
        mask = v >= thr
        hi = int(np.ceil(rank))
        assert mask.sum() >= n - hi
        assert set(np.flatnonzero(mask)) >= set(np.flatnonzero(v >= b))
    assert unfused_misses > 0


@pytest.mark.parametrize("percentile,gs", [(99.9, 128), (99.5, 16), (99.0, 16), (99.9, 32), (99.0, 128), (50.5, 8)])
def test_dynamic_percentile_quantizers_closed_form(percentile, gs):
    """quantize_symmetric_int8 / int4 below percentile 100 (src/quant/int8_basic.py:76-94,
    int4_basic.py:80-99): per group, abs_max = torch.quantile(|x| in fp32); the closed form
    takes the group's order statistics and fused_lerp32, then the INT8 fp16 / INT4 fp32
    scale chain."""
    g = torch.Generator().manual_seed(int(percentile * 10) + gs)
    x = (torch.randn(2, 2, 9, 128, generator=g) * torch.rand(2, 2, 9, 1, generator=g) * 4).to(torch.float16)
    x[0, 0, 0, :gs] = 0.0  # an all-zero group: the 1e-5 clamp
    q8, s8 = OQ.quantize_symmetric_int8(x, percentile, gs)
    q4, s4 = OQ.quantize_symmetric_int4(x, percentile, gs)
    xs = x.numpy().reshape(-1, gs)
    for i, row in enumerate(xs):
        am, _, _ = quantile32(np.abs(row.astype(np.float32)), percentile / 100.0)
        a16 = np.float16(max(am, np.float32(1e-5)))
        sc8 = np.float16(np.float32(a16) / np.float32(127))
        assert s8.reshape(-1)[i].item() == float(sc8)
        assert np.array_equal(q8.numpy().reshape(-1, gs)[i], int8_closed_form(row, sc8))
        sc4 = np.float32(max(am, np.float32(1e-5))) / np.float32(7)
        assert s4.reshape(-1)[i].item() == float(sc4)
        want4 = np.clip(np.rint(row.astype(np.float32) / sc4), -7, 7).astype(np.int8)
        assert np.array_equal(q4.numpy().reshape(-1, gs)[i], want4)
    # clipping: the largest |x| of a group can exceed 127 * scale
    assert (q8.abs() == 127).any()


def test_outlier_rescue_effect():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 2, 1, 128, generator=g).to(torch.float16)
    x[0, 1, 0, 5] = 60.0
    st = torch.full((2, 4), 0.3)
    q0, s0 = OQ.int4_cache_quantize(x, st, 32)
    # 16 groups, ratio 0.05: rank = 0.95 * 15 = 14.25 -> only the largest group is rescued
    q1, s1 = OQ.int4_cache_quantize(x, st, 32, outlier_rescue_ratio=0.05)
    assert s1[0, 1, 0, 0] == pytest.approx(60.0 / 7.0)  # the outlier group is rescued
    rest = torch.ones_like(s1, dtype=torch.bool)
    rest[0, 1, 0, 0] = False
    assert torch.equal(s0[rest], s1[rest])              # every other group keeps the static scale
    assert q0[0, 1, 0, 5] == 7 and q1[0, 1, 0, 5] == 7
    _, s_all = OQ.int4_cache_quantize(x, st, 32, outlier_rescue_ratio=1.0)
    dyn = OQ.int4_dynamic_group_scale(x, 32)
    assert torch.equal(s_all, torch.maximum(st[None, :, None, :].expand_as(dyn), dyn))


# ---------------------------------------------------------------- asymmetric static


def test_asym_static_closed_form_and_reference_formula():
    g = torch.Generator().manual_seed(9)
    x = (torch.randn(2, 3, 11, 128, generator=g) * 2).to(torch.float16)
    s16 = (torch.rand(3, 4, generator=g) * 0.4 + 0.05).to(torch.float16)
    z16 = (torch.randn(3, 4, generator=g) * 0.2).to(torch.float16)
    q = OQ.quantize_asymmetric_static(x, s16, z16)
    xn = x.numpy().astype(np.float32).reshape(2, 3, 11, 4, 32)
    sn = s16.numpy().astype(np.float32)[None, :, None, :, None]
    zn = z16.numpy().astype(np.float32)[None, :, None, :, None]
    expect = np.clip(np.rint((xn - zn) / sn), -8, 7).astype(np.int8)
    assert np.array_equal(q.numpy().reshape(2, 3, 11, 4, 32), expect)
    # reference K quantize+pack formula with per-channel params = group params broadcast
    ks = s16.float().repeat_interleave(32, dim=1)[None].expand(2, 3, 128)
    kz = z16.float().repeat_interleave(32, dim=1)[None].expand(2, 3, 128)
    ref_q = torch.round((x.float() - kz.unsqueeze(2)) / ks.unsqueeze(2)).clamp(-8, 7).to(torch.int8)
    assert torch.equal(ref_q, q)
    deq = OQ.dequantize_asymmetric_static(q, s16, z16)
    assert torch.allclose(deq.view(2, 3, 11, 4, 32), torch.from_numpy(expect * sn + zn), atol=0)


# ---------------------------------------------------------------- attention oracle


def test_attn_kat_single_token_is_v():
    q = torch.ones(1, 1, 4, dtype=torch.float16)
    k = torch.ones(1, 1, 1, 4, dtype=torch.int8)
    v = torch.tensor([[[[2, 3, 4, 5]]]], dtype=torch.int8)
    one = torch.ones(1, 1, 1, 1, dtype=torch.float16)
    out = OA.decode_attn_int8_torch_ref(q, k, v, one, one, torch.tensor([1]), 1.0)
    assert torch.equal(out, torch.tensor([[[2.0, 3.0, 4.0, 5.0]]], dtype=torch.float16))


def test_attn_kat_two_tokens_softmax():
    q = torch.tensor([[[1.0, 0.0]]], dtype=torch.float16)
    kv = torch.tensor([[[[1, 0], [0, 1]]]], dtype=torch.int8)
    one = torch.ones(1, 1, 2, 1, dtype=torch.float16)
    out = OA.decode_attn_int8_torch_ref(q, kv, kv, one, one, torch.tensor([2]), 1.0)
    e = math.e
    assert torch.allclose(out.float(), torch.tensor([[[e / (e + 1), 1 / (e + 1)]]]), atol=1e-3)


def test_attn_kat_zero_context_and_gqa_mapping():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 4, 8, generator=g).to(torch.float16)
    k = torch.randint(-3, 4, (2, 2, 5, 8), generator=g, dtype=torch.int8)
    v = torch.randint(-3, 4, (2, 2, 5, 8), generator=g, dtype=torch.int8)
    s = torch.ones(2, 2, 5, 1, dtype=torch.float16)
    out = OA.decode_attn_int8_torch_ref(q, k, v, s, s, torch.tensor([0, 5]), 0.5)
    assert torch.all(out[0] == 0)
    # head h uses kv head h // 2: recompute each head alone with Hq = Hkv = 1
    for h in range(4):
        single = OA.decode_attn_int8_torch_ref(q[1:2, h:h + 1], k[1:2, h // 2:h // 2 + 1],
                                               v[1:2, h // 2:h // 2 + 1], s[1:2, :1], s[1:2, :1],
                                               torch.tensor([5]), 0.5)
        assert torch.equal(single[0, 0], out[1, h])


def fp16_close(out16, ref64, rel=2e-4):
    """|out - ref| <= half an fp16 ulp of ref (the output rounding) + rel * |ref| + 1e-5."""
    ref = np.asarray(ref64, dtype=np.float64)
    half_ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) / 2
    err = np.abs(np.asarray(out16, dtype=np.float64) - ref)
    return bool(np.all(err <= half_ulp + rel * np.abs(ref) + 1e-5)), float(err.max())


def brute_attention(q, k, v, ctx, sm):
    """float64 triple loop; q [Hq, D], k/v [Hkv, S, D] as float64 numpy."""
    Hq, D = q.shape
    Hkv = k.shape[0]
    out = np.zeros((Hq, D))
    for h in range(Hq):
        kh = h // (Hq // Hkv)
        sc = np.array([sum(q[h, d] * k[kh, t, d] for d in range(D)) * sm for t in range(ctx)])
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[h] = (p[:, None] * v[kh, :ctx]).sum(0)
    return out


def test_attn_int8_brute_force():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 6, 16, generator=g).to(torch.float16)
    k = torch.randint(-127, 128, (1, 2, 7, 16), generator=g, dtype=torch.int8)
    v = torch.randint(-127, 128, (1, 2, 7, 16), generator=g, dtype=torch.int8)
    ks = (torch.rand(1, 2, 7, 2, generator=g) * 0.02).to(torch.float16)
    vs = (torch.rand(1, 2, 7, 2, generator=g) * 0.02).to(torch.float16)
    out = OA.decode_attn_int8_torch_ref(q, k, v, ks, vs, torch.tensor([6]), 0.25)
    kd = (k.view(1, 2, 7, 2, 8).to(torch.float16) * ks.unsqueeze(-1)).view(1, 2, 7, 16).double().numpy()
    vd = (v.view(1, 2, 7, 2, 8).to(torch.float16) * vs.unsqueeze(-1)).view(1, 2, 7, 16).double().numpy()
    ref = brute_attention(q[0].double().numpy(), kd[0], vd[0], 6, 0.25)
    ok, err = fp16_close(out[0].double().numpy(), ref)
    assert ok, err


def test_attn_invariants():
    g = torch.Generator().manual_seed(6)
    q = torch.randn(2, 6, 32, generator=g).to(torch.float16)
    k = torch.randint(-50, 50, (2, 1, 40, 32), generator=g, dtype=torch.int8)
    v = torch.randint(-50, 50, (2, 1, 40, 32), generator=g, dtype=torch.int8)
    ks = torch.full((2, 1, 40, 4), 0.01, dtype=torch.float16)
    ctx = torch.tensor([40, 33])
    out = OA.decode_attn_int8_torch_ref(q, k, v, ks, ks, ctx, 0.2)
    perm = torch.randperm(33, generator=g)
    k2, v2 = k.clone(), v.clone()
    k2[1, :, :33], v2[1, :, :33] = k[1, :, perm], v[1, :, perm]
    out2 = OA.decode_attn_int8_torch_ref(q, k2, v2, ks, ks, ctx, 0.2)
    assert torch.allclose(out[1].float(), out2[1].float(), atol=1e-3)
    # tokens past the context never matter
    k3 = k.clone()
    k3[1, :, 33:] = 127
    assert torch.equal(OA.decode_attn_int8_torch_ref(q, k3, v, ks, ks, ctx, 0.2)[1], out[1])


def test_asym_oracle_brute_force_with_outliers():
    g = torch.Generator().manual_seed(8)
    B, H, S, D = 1, 1, 5, 128
    kq = torch.randint(-8, 8, (B, H, S, D), generator=g, dtype=torch.int8)
    vq = torch.randint(-8, 8, (B, H, S, D), generator=g, dtype=torch.int8)
    ks = (torch.rand(H, 4, generator=g) + 0.1).to(torch.float16)
    kz = torch.randn(H, 4, generator=g).to(torch.float16)
    vs = (torch.rand(H, 4, generator=g) + 0.1).to(torch.float16)
    vz = torch.randn(H, 4, generator=g).to(torch.float16)
    oidx = torch.tensor([[3, 40, 77, 127]], dtype=torch.int32)
    oval = (torch.randn(B, H, S, 4, generator=g) * 20).to(torch.float16)
    q = torch.randn(B, 3, D, generator=g).to(torch.float16)
    tau = torch.tensor([0.9, 1.1, 1.0], dtype=torch.float16)
    out = OA.decode_attn_asym_ref(q, OQ.pack_int4(kq), OQ.pack_int4(vq), ks, kz, vs, vz,
                                  torch.tensor([S]), 0.1, inv_tau=tau, k_outlier_idx=oidx,
                                  k_outlier_val=oval)
    kd = np.zeros((H, S, D))
    vd = np.zeros((H, S, D))
    for t in range(S):
        for d in range(D):
            gi = d // 32
            kd[0, t, d] = float(kq[0, 0, t, d]) * float(ks[0, gi]) + float(kz[0, gi])
            vd[0, t, d] = float(vq[0, 0, t, d]) * float(vs[0, gi]) + float(vz[0, gi])
        for j, ch in enumerate(oidx[0].tolist()):
            kd[0, t, ch] = float(oval[0, 0, t, j])
    qs = (q[0] * tau.view(-1, 1)).double().numpy()  # fp16 product, as the reference
    ref = brute_attention(qs, kd, vd, S, 0.1)
    ok, err = fp16_close(out[0].double().numpy(), ref)
    assert ok, err


def test_planted_mistake_is_caught():
    """A pack with swapped nibbles (a plausible bug) must fail the layout KAT."""
    x = torch.tensor([[-8, 7]], dtype=torch.int8).view(1, 1, 1, 2)
    u = (x.to(torch.int16) + 8).to(torch.uint8).view(1, 1, 1, 1, 2)
    swapped = ((u[..., 1] << 4) | u[..., 0]).to(torch.int8)
    assert int(swapped.view(torch.uint8)) != ((-8 + 8) << 4) | (7 + 8)
    assert int(OQ.pack_int4(x).view(torch.uint8)) == ((-8 + 8) << 4) | (7 + 8)


# ---------------------------------------------------------------- scale policies (KATs)


def _groups_row(absmax, gs):
    """fp16 x [1, 1, 1, G * gs]: group g holds absmax[g] at its first channel, -absmax[g] / 2
    at its second and zeros elsewhere (so its absmax is absmax[g])."""
    G = len(absmax)
    x = torch.zeros(1, 1, 1, G * gs, dtype=torch.float16)
    for g, a in enumerate(absmax):
        x[0, 0, 0, g * gs] = a
        x[0, 0, 0, g * gs + 1] = -a / 2
    return x


def test_int8_adaptive_scale_kat():
    gs, m = 32, 2.0
    s16 = np.float16(0.01)
    absmax = [1.905, 3.81, 0.0, 1.0]
    x = _groups_row(absmax, gs)
    st = torch.full((1, 4), float(s16), dtype=torch.float16)
    q, sc = OQ.int8_cache_quantize(x, st, gs, adaptive=True, margin=m)
    st32 = np.float32(s16) * np.float32(m)                     # static side, times the margin
    dyn = [np.float32(max(np.float32(np.float16(a)), np.float32(1e-5))) / np.float32(127) for a in absmax]
    want = [np.float16(max(st32, d)) for d in dyn]
    # which side wins in each group: (s, s*m) -> s*m, above -> dyn, zero -> s*m, below s -> s*m
    assert [w == np.float16(st32) for w in want] == [True, False, True, True]
    assert sc.view(-1).tolist() == [float(w) for w in want]
    for g in range(4):
        xs = x[0, 0, 0, g * gs:(g + 1) * gs].numpy()
        assert np.array_equal(q[0, 0, 0, g * gs:(g + 1) * gs].numpy(), int8_closed_form(xs, want[g]))
    # plausible mistakes give other scales
    on_dyn = [np.float16(max(np.float32(s16), d * np.float32(m))) for d in dyn]
    no_margin = [np.float16(max(np.float32(s16), d)) for d in dyn]
    as_min = [np.float16(min(st32, d)) for d in dyn]
    for wrong in (on_dyn, no_margin, as_min):
        assert wrong != want


def test_int8_adaptive_off_keeps_static_and_dynamic_without_table():
    gs = 32
    x = _groups_row([1.905, 3.81, 0.0, 1.0], gs)
    st = torch.full((1, 4), 0.01, dtype=torch.float16)
    _, sc = OQ.int8_cache_quantize(x, st, gs, adaptive=False)
    assert sc.view(-1).tolist() == [float(np.float16(0.01))] * 4
    _, sd = OQ.int8_cache_quantize(x, None, gs)
    # dynamic: fp16 absmax clamped to 1e-5 in fp16, divided by 127 in fp16
    want = [np.float16(np.float16(max(np.float16(a), np.float16(1e-5))) / np.float16(127))
            for a in (1.905, 3.81, 0.0, 1.0)]
    assert sd.view(-1).tolist() == [float(w) for w in want]


def _int4_want(x, scale32, gs):
    xs = x.view(-1).numpy().astype(np.float32)
    out = np.empty_like(xs, dtype=np.int8)
    for i, v in enumerate(xs):
        s = np.float32(max(scale32[i // gs], np.float32(1e-5)))
        out[i] = np.int8(np.clip(np.rint(np.float32(v) / s), -7, 7))
    return out


def test_int4_adaptive_and_mixed_rescue_kat():
    gs = 32
    absmax = [0.7, 1.4, 0.91, 0.35]
    x = _groups_row(absmax, gs)
    s32, m = np.float32(0.1), np.float32(1.5)
    st = torch.full((1, 4), float(s32), dtype=torch.float32)
    dyn = [np.float32(max(np.float32(np.float16(a)), np.float32(1e-5))) / np.float32(7) for a in absmax]
    cases = {
        # adaptive: max(s * margin, absmax / 7)
        "adaptive": (dict(adaptive=True, margin=float(m)), [max(s32 * m, d) for d in dyn]),
        # mixed rescue: max(s, absmax / 7)
        "mixed": (dict(mixed_rescue=True), [max(s32, d) for d in dyn]),
        # both: adaptive first, then mixed (max is order-free, the margin is not)
        "both": (dict(adaptive=True, margin=float(m), mixed_rescue=True),
                 [max(max(s32 * m, d), d) for d in dyn]),
        # outlier rescue of every group after mixed rescue changes nothing (int4_cache.py:367-375)
        "mixed+rescue": (dict(mixed_rescue=True, outlier_rescue_ratio=0.5), [max(s32, d) for d in dyn]),
        "static": (dict(), [s32] * 4),
    }
    for name, (kw, want) in cases.items():
        q, sc = OQ.int4_cache_quantize(x, st, gs, **kw)
        got = sc.view(-1).tolist()
        assert got == [float(w) for w in want], (name, got, want)
        assert np.array_equal(q.view(-1).numpy(), _int4_want(x, want, gs)), name
    # the KAT separates the policies: adaptive differs from mixed in groups 0 and 2 (the
    # margin), both from static in groups 1 (dynamic wins)
    a = cases["adaptive"][1]
    mx = cases["mixed"][1]
    assert a[0] != mx[0] and a[2] != mx[2] and a[1] == mx[1] == dyn[1]
    # margin applied to the dynamic side instead would change group 2
    assert max(s32, dyn[2] * m) != a[2]


def test_k8v4_oracle_brute_force():
    g = torch.Generator().manual_seed(9)
    B, H, Hq, S, D = 1, 2, 6, 7, 128
    kq = torch.randint(-127, 128, (B, H, S, D), generator=g, dtype=torch.int8)
    ks16 = (torch.rand(B, H, S, 4, generator=g) * 0.02 + 0.001).to(torch.float16)
    vq = torch.randint(-8, 8, (B, H, S, D), generator=g, dtype=torch.int8)
    vs = (torch.rand(H, 4, generator=g) + 0.1).to(torch.float16)
    vz = torch.randn(H, 4, generator=g).to(torch.float16)
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    ctx = 5
    out = OA.decode_attn_k8v4_ref(q, kq, ks16, OQ.pack_int4(vq), vs, vz, torch.tensor([ctx]), 0.1,
                                  inv_tau=tau)
    kd = np.zeros((H, S, D))
    vd = np.zeros((H, S, D))
    for h in range(H):
        for t in range(S):
            for d in range(D):
                gi = d // 32
                # the reference's fp16 product code * scale (src/engine/patch_model.py:355-362)
                kd[h, t, d] = float(np.float16(np.float16(int(kq[0, h, t, d])) * np.float16(ks16[0, h, t, gi])))
                vd[h, t, d] = float(vq[0, h, t, d]) * float(vs[h, gi]) + float(vz[h, gi])
    qs = np.array([[float(np.float16(np.float16(q[0, i, d]) * np.float16(tau[i]))) for d in range(D)]
                   for i in range(Hq)])
    ref = brute_attention(qs, kd, vd, ctx, 0.1)
    ok, err = fp16_close(out[0].double().numpy(), ref)
    assert ok, err


def test_dequantize_symmetric_kats():
    q = torch.tensor([[-127, 0, 5, 7, -3, 2, 1, -1]], dtype=torch.int8).view(1, 1, 1, 8)
    sc = torch.tensor([0.5, 0.25, 2.0, 8.0], dtype=torch.float32).view(1, 1, 1, 4)  # groups of 2
    out = OQ.dequantize_symmetric(q, sc).view(-1).tolist()
    assert out == [-63.5, 0.0, 1.25, 1.75, -6.0, 4.0, 8.0, -8.0]
    one = torch.tensor([3.0]).view(1, 1, 1, 1)
    assert OQ.dequantize_symmetric(q, one).view(-1).tolist() == [3.0 * v for v in q.view(-1).tolist()]
    # the cache's fp16 result is the exact product rounded once
    g = torch.Generator().manual_seed(12)
    codes = torch.randint(-127, 128, (2, 2, 9, 128), generator=g, dtype=torch.int8)
    s16 = (torch.rand(2, 2, 9, 8, generator=g) * 0.05 + 1e-4).to(torch.float16)
    got = OQ.cache_get_kv(codes, s16).numpy()
    exact = codes.double().numpy().reshape(2, 2, 9, 8, 16) * s16.double().numpy()[..., None]
    assert np.array_equal(got, exact.reshape(2, 2, 9, 128).astype(np.float16))


def test_mixed_oracle_brute_force_and_kat():
    """decode_attn_mixed_ref against float64 with explicit per-element dequantisation: K =
    code x the scale of group d // gs of its own token (fp16 result of the exact product),
    V = code x s_t + z_t of its own token (fp16).  A transposed V broadcast (per channel
    instead of per token) or swapped s / z fails both checks."""
    g = torch.Generator().manual_seed(19)
    B, H, Hq, S, D, gs = 1, 2, 6, 7, 128, 64
    kq = torch.randint(-127, 128, (B, H, S, D), generator=g, dtype=torch.int8)
    ks = (torch.rand(B, H, S, D // gs, generator=g) * 0.02 + 0.001).to(torch.float16).float()
    vq = torch.randint(-8, 8, (B, H, S, D), generator=g, dtype=torch.int8)
    vs = torch.rand(B, H, S, generator=g) * 0.3 + 0.05
    vz = torch.randn(B, H, S, generator=g)
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    ctx = 6
    out = OA.decode_attn_mixed_ref(q, kq, ks, vq, vs, vz, torch.tensor([ctx]), 0.1, inv_tau=tau)
    kd = np.zeros((H, S, D))
    vd = np.zeros((H, S, D))
    for h in range(H):
        for t in range(S):
            for d in range(D):
                kd[h, t, d] = float(np.float16(int(kq[0, h, t, d]) * float(ks[0, h, t, d // gs])))
                vd[h, t, d] = float(np.float16(np.float32(int(vq[0, h, t, d])) * np.float32(vs[0, h, t])
                                               + np.float32(vz[0, h, t])))
    qs = np.array([[float(np.float16(np.float16(q[0, i, d]) * np.float16(tau[i]))) for d in range(D)]
                   for i in range(Hq)])
    ref = brute_attention(qs, kd, vd, ctx, 0.1)
    ok, err = fp16_close(out[0].double().numpy(), ref)
    assert ok, err
    # known answer: one-token context returns that token's V = code * s + z, per token
    one = OA.decode_attn_mixed_ref(q, kq, ks, vq, vs, vz, torch.tensor([1]), 0.1)
    v0 = (vq[0, :, 0].float() * vs[0, :, 0, None] + vz[0, :, 0, None]).to(torch.float16)
    assert torch.equal(one[0], v0.repeat_interleave(Hq // H, dim=0))
    vq2 = torch.tensor([3, -8, 7, 0], dtype=torch.int8).repeat(32).view(1, 1, 1, D).expand(1, H, S, D)
    sv = torch.full((1, H, S), 0.5)
    zv = torch.full((1, H, S), -1.0)
    lit = OA.decode_attn_mixed_ref(q, kq, ks, vq2.contiguous(), sv, zv, torch.tensor([1]), 0.1)
    assert lit[0, 0, :4].tolist() == [0.5, -5.0, 2.5, -1.0]


def test_mixed_bits_oracle_kats():
    """decode_attn_mixed_bits_ref: the (8, 4) pair is decode_attn_mixed_ref (same bits); a
    one-token context returns that token's V (fp16 values for a 16-bit side, code x scale of
    its group for an 8-bit side, code x s + z for 4 bits), for every head of its group."""
    g = torch.Generator().manual_seed(23)
    B, H, Hq, S, D = 1, 2, 6, 5, 128
    q = torch.randn(B, Hq, D, generator=g).to(torch.float16)
    k8 = torch.randint(-127, 128, (B, H, S, D), generator=g, dtype=torch.int8)
    ks = (torch.rand(B, H, S, 4, generator=g) * 0.02 + 0.001).to(torch.float16)
    v4 = torch.randint(-8, 8, (B, H, S, D), generator=g, dtype=torch.int8)
    vs, vz = torch.rand(B, H, S, generator=g) * 0.3 + 0.05, torch.randn(B, H, S, generator=g)
    ctx = torch.tensor([S])
    a = OA.decode_attn_mixed_bits_ref(q, k8, 8, ks, OQ.pack_int4(v4), 4, vs, vz, ctx, 0.1)
    b = OA.decode_attn_mixed_ref(q, k8, ks, v4, vs, vz, ctx, 0.1)
    assert torch.equal(a, b)
    k16 = torch.randn(B, H, S, D, generator=g).to(torch.float16)
    v16 = torch.randn(B, H, S, D, generator=g).to(torch.float16)
    one = torch.tensor([1])
    o = OA.decode_attn_mixed_bits_ref(q, k16, 16, None, v16, 16, None, None, one, 0.1)
    assert torch.equal(o[0], v16[0, :, 0].repeat_interleave(Hq // H, dim=0))
    v8 = torch.randint(-127, 128, (B, H, S, D), generator=g, dtype=torch.int8)
    o = OA.decode_attn_mixed_bits_ref(q, k8, 8, ks, v8, 8, ks, None, one, 0.1)
    exp = (v8[0, :, 0].view(H, 4, 32).float() * ks[0, :, 0].float().unsqueeze(-1)).view(H, D).to(torch.float16)
    assert torch.equal(o[0], exp.repeat_interleave(Hq // H, dim=0))
