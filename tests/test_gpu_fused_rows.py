"""GPU tests of the fused decode step of the row formats: kvq_append_decode_attn with the
append kernel's row quantizer run by the decode kernel's writer wave.  Formats: per-token
INT8 / INT4 scales (dynamic, adaptive, static tables, mixed rescue, rescue-all), the KIVI
family with quantized and 16-bit sides, and the mixed cache.

Twin caches take the same tokens: one through append_decode_attn (one launch), the other
through append and then the decode kernel (two launches).  At every step, codes, scales,
zero-points and outputs must be bit-identical.  The fused output must also be within
max-abs 2e-3 (one fp16 ulp where |out| >= 4) and cosine 0.9999 of the oracle's attention
over the stored cache.

When a wave runs long enough (the writer of a per-token INT4 / INT8 step holds at least
kShed + 3 tiles: KVQ_SHED_ROW = 1, KVQ_SHED_RESCUE = 3), the fused kernel's writer hands
its first tiles to waves of the other SIMDs; the two paths then sum the same tiles in different
waves, so their outputs agree within the oracle bound rather than bit for bit
(test_fused_rows_writer_sheds_tiles).  The cases above stay below that length.
"""
import math

import pytest
import torch

from oracle import attn as OA

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


def assert_close_ulp(out, ref, tag):
    o, r = out.detach().float().cpu(), ref.detach().float().cpu()
    assert o.shape == r.shape and torch.isfinite(o).all(), tag
    ulp = torch.exp2(torch.floor(torch.log2(r.abs().clamp(min=2.0 ** -14))) - 10)
    err = (o - r).abs()
    worst = (err - torch.maximum(torch.full_like(r, ATOL), ulp)).max().item()
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r.flatten(), dim=0).item()
    print(f"[{tag}] max_abs={err.max().item():.3e} excess={worst:.3e} cos={cos:.7f}", flush=True)
    assert worst <= 0 and cos >= COS_MIN, (tag, worst, cos)


def _kv(B, H, S, g):
    k = torch.randn(B, H, S, 128, generator=g) * 1.5
    k[..., 3] *= 15.0
    k[..., 90] = k[..., 90] * 8.0 + 4.0
    v = torch.randn(B, H, S, 128, generator=g) * (torch.rand(B, H, S, 1, generator=g) * 3 + 0.2)
    v = v + torch.randn(B, H, S, 1, generator=g)
    return k.to(torch.float16), v.to(torch.float16)


def _equal(a, b, tag):
    for i, (x, y) in enumerate(zip(a, b)):
        if x is None or y is None:
            assert x is None and y is None, (tag, i)
            continue
        assert torch.equal(x, y), f"{tag}: tensor {i} differs"


SYM = [
    # kind, engine arguments, B, H, Hq, S0, steps
    ("int8", dict(group_size=16), 2, 2, 12, 4095, 3),          # dynamic per-token, group 16
    ("int8", dict(group_size=128), 3, 2, 12, 0, 2),            # empty start: the token is the context
    ("int8", dict(group_size=32, clip_percentile=100.0), 2, 4, 28, 40, 2),
    ("int8", dict(group_size=32, static=True, adaptive_static_scales=True,
                  adaptive_static_margin=0.9), 2, 2, 12, 300, 2),
    ("int8", dict(group_size=16, static="k"), 2, 2, 12, 100, 2),  # static K table, per-token V
    ("int4", dict(group_size=32), 2, 4, 28, 700, 2),           # int4_baseline
    ("int4", dict(group_size=16, static=True), 2, 2, 12, 33, 2),
    ("int4", dict(group_size=32, static=True, outlier_rescue_ratio=1.0), 2, 2, 12, 64, 2),
    ("int4", dict(group_size=32, static=True, mixed_rescue=True), 2, 2, 12, 64, 2),
    # the group rescue (int4_fused / int4_ours): the writer finds the threshold over every row
    ("int4", dict(group_size=16, static=True, outlier_rescue_ratio=0.01), 8, 4, 28, 300, 2),  # 256 scales
    ("int4", dict(group_size=32, static=True, outlier_rescue_ratio=0.01), 4, 2, 12, 40, 2),   # 32 scales
    ("int4", dict(group_size=16, static=True, outlier_rescue_ratio=0.02), 8, 4, 28, 33, 2),  # 5 below the top
    ("int4", dict(group_size=64, static=True, outlier_rescue_ratio=0.05), 4, 8, 32, 50, 2),   # 64 scales
    ("int4", dict(group_size=128, static=True, outlier_rescue_ratio=0.1), 3, 5, 15, 20, 2),   # 15 rows
    ("int4", dict(group_size=16, static=True, outlier_rescue_ratio=0.1, ties=True), 4, 4, 16, 70, 2),
]


@pytest.mark.parametrize("kind,kw,B,H,Hq,S0,steps", SYM)
def test_fused_rows_symmetric(kind, kw, B, H, Hq, S0, steps):
    K = _k()
    print(f"[case] {kind} {kw} B{B} H{H} S0={S0}", flush=True)
    kw = dict(kw)
    g = gen(40 + S0 + B + len(kw))
    G = 128 // kw["group_size"]
    static = kw.pop("static", False)
    ties = kw.pop("ties", False)
    if static:
        st = torch.rand(1, H, G, generator=g) * 0.3 + 0.1
        kw["static_k_scale"] = st
        if static is True:
            kw["static_v_scale"] = st * 0.8
    cls = K.INT8KVCache if kind == "int8" else K.INT4KVCache
    mk = lambda: cls(1, device=DEV, check_numerics=False, **kw)
    one, two = mk(), mk()
    assert one._fused_step_ok(128, B, H), "the case must take the fused step"
    two._fused_step_ok = lambda *args: False  # append, then the decode kernel
    k, v = _kv(B, H, S0 + steps, g)
    if ties:  # few distinct group maxima: equal scales at the threshold
        k, v = (k * 2).round().div(2).half(), v.round().half()
    if S0:
        for c in (one, two):
            c.append(0, k[:, :, :S0].to(DEV), v[:, :, :S0].to(DEV))
    sm = 1 / math.sqrt(128)
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    get = (lambda c: c.get_int8_tensors(0)) if kind == "int8" else (lambda c: c.get_int4_tensors(0))
    for i in range(steps):
        kn, vn = k[:, :, S0 + i:S0 + i + 1].to(DEV), v[:, :, S0 + i:S0 + i + 1].to(DEV)
        q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
        out1 = one.append_decode_attn(0, q.to(DEV), kn, vn, sm_scale=sm, inv_tau=tau.to(DEV))
        out2 = two.append_decode_attn(0, q.to(DEV), kn, vn, sm_scale=sm, inv_tau=tau.to(DEV))
        torch.cuda.synchronize()
        t1, t2 = get(one), get(two)
        _equal(t1, t2, f"{kind} step {i}")
        assert torch.equal(out1, out2), f"{kind} step {i}: fused output differs from two launches"
        kc, vc, ks, vs = [t.cpu() for t in t1]
        n = S0 + i + 1
        cl = torch.full((B,), n, dtype=torch.int32)
        qq = OA.prescale_q(q, tau)
        # the reference's decode step casts the engines' scales to fp16 before either kernel
        # (src/engine/patch_model.py:910-917, 926-933, 944-948)
        if kind == "int8":
            ref = OA.decode_attn_int8_torch_ref(qq, kc, vc, ks.half(), vs.half(), cl, sm)
        else:
            ref = OA.decode_attn_int4_torch_ref(qq, kc, vc, ks.half(), vs.half(), cl, sm)
        assert_close_ulp(out1, ref, f"{kind} {n}")


KIVI = [
    # engine, arguments, B, H, Hq, S0, steps
    ("kivi", dict(quant_bits=4), 2, 2, 12, 300, 3),
    ("kivi", dict(quant_bits=8, k_percentile=99.0, v_percentile=99.0), 2, 4, 28, 4095, 2),
    ("kivi", dict(quant_bits=4, v_percentile=99.9), 3, 2, 10, 31, 2),
    ("alloc", dict(per_layer_bits=[(4, 16)]), 2, 2, 12, 100, 2),
    ("alloc", dict(per_layer_bits=[(16, 8)]), 2, 2, 12, 100, 2),
    ("alloc", dict(per_layer_bits=[(16, 16)]), 2, 2, 12, 64, 2),
    ("alloc", dict(per_layer_bits=[(8, 4)], v_percentile=99.5), 2, 2, 12, 64, 2),
]


@pytest.mark.parametrize("eng,kw,B,H,Hq,S0,steps", KIVI)
def test_fused_rows_kivi_family(eng, kw, B, H, Hq, S0, steps):
    K = _k()
    print(f"[case] {eng} {kw} B{B} H{H} S0={S0}", flush=True)
    g = gen(70 + S0 + B)
    if eng == "kivi":
        mk = lambda: K.KIVIStyleKVCache(1, device=DEV, **kw)
        kb = vb = kw["quant_bits"]
    else:
        mk = lambda: K.RoleAwareAllocatorKVCache(1, device=DEV, **kw)
        kb, vb = kw["per_layer_bits"][0]
    one, two = mk(), mk()
    k, v = _kv(B, H, S0 + steps, g)
    for c in (one, two):
        c.append(0, k[:, :, :S0].to(DEV), v[:, :, :S0].to(DEV))
    sm = 1 / math.sqrt(128)
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    for i in range(steps):
        kn, vn = k[:, :, S0 + i:S0 + i + 1].to(DEV), v[:, :, S0 + i:S0 + i + 1].to(DEV)
        q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
        out1 = one.append_decode_attn(0, q.to(DEV), kn, vn, sm_scale=sm, inv_tau=tau.to(DEV))
        two.append(0, kn, vn)
        out2 = two._attend(0, q.to(DEV), sm, tau.to(DEV))
        torch.cuda.synchronize()
        t1 = one.get_kivi_tensors(0)
        _equal(t1, two.get_kivi_tensors(0), f"{eng} step {i}")
        assert torch.equal(out1, out2), f"{eng} step {i}: fused output differs from two launches"
        kc, vc, ks, kz, vs, vz = [None if t is None else t.cpu() for t in t1]
        n = S0 + i + 1
        ref = OA.decode_attn_kivi_family_ref(q, kc, kb, ks, kz, vc, vb, vs, vz, torch.full((B,), n), sm,
                                             inv_tau=tau)
        assert_close_ulp(out1, ref, f"{eng} ({kb},{vb}) {n}")


@pytest.mark.parametrize("kb,vb,gs,vgs", [(8, 4, 128, 128), (8, 4, 16, 16), (8, 8, 32, 32), (8, 16, 64, 64),
                                          (16, 4, 128, 128), (16, 16, 128, 128), (4, 4, 128, 128),
                                          (4, 8, 128, 64), (4, 16, 128, 128), (16, 8, 128, 32),
                                          (8, 8, 128, 16)])
def test_fused_rows_mixed(kb, vb, gs, vgs):
    K = _k()
    print(f"[case] mixed ({kb},{vb}) gs={gs} vgs={vgs}", flush=True)
    g = gen(90 + kb + vb + gs + vgs)
    B, H, Hq, S0, steps = 2, 2, 10, 95, 3
    mk = lambda: K.MixedKVCache(1, device=DEV, k_group_size=gs, v_group_size=vgs, k_bits=kb, v_bits=vb,
                                v_percentile=99.9)
    one, two = mk(), mk()
    k, v = _kv(B, H, S0 + steps, g)
    for c in (one, two):
        c.append(0, k[:, :, :S0].to(DEV), v[:, :, :S0].to(DEV))
    sm = 1 / math.sqrt(128)
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    for i in range(steps):
        kn, vn = k[:, :, S0 + i:S0 + i + 1].to(DEV), v[:, :, S0 + i:S0 + i + 1].to(DEV)
        q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
        out1 = one.append_decode_attn(0, q.to(DEV), kn, vn, sm_scale=sm, inv_tau=tau.to(DEV))
        n = two._append(0, kn, vn)
        out2 = two._step_for(0, Hq).attend(q.to(DEV), n, sm, tau.to(DEV))
        torch.cuda.synchronize()
        t1 = one.get_mixed_tensors(0)
        _equal(t1, two.get_mixed_tensors(0), f"mixed step {i}")
        assert torch.equal(out1, out2), f"mixed step {i}: fused output differs from two launches"
        kc, ksc, vc, vsc, vz = [None if t is None else t.cpu() for t in t1]
        kz = one.get_k_zero_points(0)
        if kz is not None:
            assert torch.equal(kz, two.get_k_zero_points(0))
            kz = kz.cpu()
        ref = OA.decode_attn_mixed_bits_ref(q, kc, kb, ksc, vc, vb, vsc, vz, torch.full((B,), n), sm,
                                            inv_tau=tau, k_zp=kz)
        assert_close_ulp(out1, ref, f"mixed ({kb},{vb}) {n}")


def test_fused_rows_group_rescue_far_from_top_keeps_two_launches():
    """A group rescue threshold far from the top of the append's scales (here the median)
    is beyond the writer's walk: the engine keeps two launches, and the entry point refuses
    the fused call (enqueueing nothing), after which an engine that asked for it anyway makes
    the two launches itself with the same bits."""
    K = _k()
    st = torch.rand(1, 2, 4) * 0.3 + 0.1
    c = K.INT4KVCache(1, device=DEV, group_size=32, static_k_scale=st, static_v_scale=st,
                      outlier_rescue_ratio=0.5, check_numerics=False)
    assert not c._fused_step_ok(128, 16, 2)  # 128 scales, lower rank 63: 64 below the top
    c01 = K.INT4KVCache(1, device=DEV, group_size=32, static_k_scale=st, static_v_scale=st,
                        outlier_rescue_ratio=0.01, check_numerics=False)
    assert c01._fused_step_ok(128, 16, 2) and not c01._fused_step_ok(128, 16, 4)  # 32 rows at most
    g = gen(5)
    k, v = _kv(16, 2, 9, g)
    c.append(0, k[:, :, :8].to(DEV), v[:, :, :8].to(DEV))
    q = torch.randn(16, 12, 128, generator=g).to(torch.float16).to(DEV)
    out = c.append_decode_attn(0, q, k[:, :, 8:].to(DEV), v[:, :, 8:].to(DEV))  # two launches
    assert out.shape == q.shape and c.get_seq_len() == 9
    twin = K.INT4KVCache(1, device=DEV, group_size=32, static_k_scale=st, static_v_scale=st,
                         outlier_rescue_ratio=0.5, check_numerics=False)
    twin.append(0, k[:, :, :8].to(DEV), v[:, :, :8].to(DEV))
    twin.append_decode_attn(0, q, k[:, :, 8:].to(DEV), v[:, :, 8:].to(DEV))
    k2, v2 = _kv(16, 2, 1, g)
    k2, v2 = k2.to(DEV), v2.to(DEV)
    pk, pv = c._fused_apps(0, k2, v2, 9, None)
    with pytest.raises(NotImplementedError, match="group rescue"):
        c._step_for(0, 12).append_attend(q, 10, 1.0 / math.sqrt(128), None, pk, pv)
    assert c.get_seq_len() == 9
    c._fused_step_ok = lambda *args: True
    out = c.append_decode_attn(0, q, k2, v2)
    ref = twin.append_decode_attn(0, q, k2, v2)
    torch.cuda.synchronize()
    assert torch.equal(out, ref) and c.get_seq_len() == twin.get_seq_len() == 10
    for a, b in zip(c.get_int4_tensors(0), twin.get_int4_tensors(0)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("eng", ["int8", "mixed88", "int4"])
def test_fused_rows_one_row_first_token(eng):
    """Batch 1 and an empty cache: the first decode token is the whole context, so its
    per-token scale views have one row and one token (which look like a static table);
    the fused step still appends with the per-token arithmetic, bit-identical to two
    launches."""
    K = _k()
    g = gen(77)
    if eng == "int8":
        mk = lambda: K.INT8KVCache(1, device=DEV, group_size=128, check_numerics=False)
    elif eng == "int4":
        mk = lambda: K.INT4KVCache(1, device=DEV, group_size=32, check_numerics=False)
    else:
        mk = lambda: K.MixedKVCache(1, device=DEV, k_group_size=64, k_bits=8, v_bits=8, v_percentile=99.9)
    one, two = mk(), mk()
    k, v = _kv(1, 2, 3, g)
    sm = 1 / math.sqrt(128)
    for i in range(3):
        kn, vn = k[:, :, i:i + 1].to(DEV), v[:, :, i:i + 1].to(DEV)
        q = torch.randn(1, 10, 128, generator=g).to(torch.float16).to(DEV)
        out1 = one.append_decode_attn(0, q, kn, vn, sm_scale=sm)
        if eng == "mixed88":
            n = two._append(0, kn, vn)
            out2 = two._step_for(0, 10).attend(q, n, sm, None)
            t1, t2 = one.get_mixed_tensors(0), two.get_mixed_tensors(0)
        else:
            two._fused_step_ok = lambda *args: False
            out2 = two.append_decode_attn(0, q, kn, vn, sm_scale=sm)
            get = (lambda c: c.get_int8_tensors(0)) if eng == "int8" else (lambda c: c.get_int4_tensors(0))
            t1, t2 = get(one), get(two)
        torch.cuda.synchronize()
        _equal(t1, t2, f"{eng} step {i}")
        assert torch.equal(out1, out2), f"{eng} step {i}"


SHED = [
    # kind, engine arguments (per-token formats whose writer sheds tiles at long runs)
    ("int4", dict(group_size=16, static=True, outlier_rescue_ratio=0.01)),  # int4_fused: 3 tiles
    ("int4", dict(group_size=32)),                                          # int4_baseline: 1 tile
    ("int8", dict(group_size=16)),                                          # int8_baseline-like
]


@pytest.mark.parametrize("kind,kw", SHED)
def test_fused_rows_writer_sheds_tiles(kind, kw, monkeypatch):
    """Chunks of 4096 tokens over an 8.3k context: every wave holds about 11 tiles, so the
    fused writer sheds its first tiles to waves of other SIMDs.  Codes and scales stay
    bit-identical to the two-launch path; the outputs agree with each other within 2e-3 and
    with the oracle within the bound."""
    monkeypatch.setenv("KVQ_CHUNK_TOKENS", "4096")
    K = _k()
    B, H, Hq, S0, steps = 2, 2, 12, 8290, 2
    print(f"[case] shed {kind} {kw}", flush=True)
    kw = dict(kw)
    g = gen(99 + len(kw))
    G = 128 // kw["group_size"]
    if kw.pop("static", False):
        st = torch.rand(1, H, G, generator=g) * 0.3 + 0.1
        kw["static_k_scale"], kw["static_v_scale"] = st, st * 0.8
    cls = K.INT8KVCache if kind == "int8" else K.INT4KVCache
    one = cls(1, device=DEV, check_numerics=False, **kw)
    two = cls(1, device=DEV, check_numerics=False, **kw)
    assert one._fused_step_ok(128, B, H)
    two._fused_step_ok = lambda *args: False
    k, v = _kv(B, H, S0 + steps, g)
    for c in (one, two):
        c.append(0, k[:, :, :S0].to(DEV), v[:, :, :S0].to(DEV))
    assert one._step_for(0, Hq).params.chunk_tokens == 4096
    sm = 1 / math.sqrt(128)
    tau = (torch.rand(Hq, generator=g) * 0.4 + 0.8).to(torch.float16)
    get = (lambda c: c.get_int8_tensors(0)) if kind == "int8" else (lambda c: c.get_int4_tensors(0))
    for i in range(steps):
        kn, vn = k[:, :, S0 + i:S0 + i + 1].to(DEV), v[:, :, S0 + i:S0 + i + 1].to(DEV)
        q = torch.randn(B, Hq, 128, generator=g).to(torch.float16)
        out1 = one.append_decode_attn(0, q.to(DEV), kn, vn, sm_scale=sm, inv_tau=tau.to(DEV))
        out2 = two.append_decode_attn(0, q.to(DEV), kn, vn, sm_scale=sm, inv_tau=tau.to(DEV))
        torch.cuda.synchronize()
        t1 = get(one)
        _equal(t1, get(two), f"shed {kind} step {i}")
        d = (out1.float() - out2.float()).abs().max().item()
        assert d <= ATOL, (kind, i, d)
        kc, vc, ks, vs = [t.cpu() for t in t1]
        n = S0 + i + 1
        cl = torch.full((B,), n, dtype=torch.int32)
        qq = OA.prescale_q(q, tau)
        if kind == "int8":
            ref = OA.decode_attn_int8_torch_ref(qq, kc, vc, ks.half(), vs.half(), cl, sm)
        else:
            ref = OA.decode_attn_int4_torch_ref(qq, kc, vc, ks.half(), vs.half(), cl, sm)
        assert_close_ulp(out1, ref, f"shed {kind} {n}")
        assert_close_ulp(out2, ref, f"shed two {kind} {n}")
