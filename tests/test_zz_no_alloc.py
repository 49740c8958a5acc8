"""kvq_decode_attn_noalloc (the workspace-free variant of kvq_decode_attn) against
kvq_decode_attn: bit-identical outputs on two calls in a row, the second smaller, for a
format whose split partials are merged inside the launch (arrival counters in the fixed
scratch) and for one merged by a combine launch; oversized calls are rejected."""
import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _mods():
    from llm_kvcache_quantization_amd import _capi as C
    from llm_kvcache_quantization_amd import kernels as KK

    C.lib()
    return C, KK


def _asym_tiled_plan(C, KK, B, Hq, Hkv, S, ctx, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, Hq, 128, device=DEV, generator=g).half()
    k = torch.randint(0, 256, (B, Hkv, S, 64), device=DEV, dtype=torch.uint8, generator=g)
    nt = -(-S // 32)
    v = torch.randint(0, 256, (B, Hkv, nt, 2048), device=DEV, dtype=torch.uint8, generator=g)
    ks = (torch.rand(Hkv, 4, device=DEV, generator=g) * 0.2 + 0.05).half()
    kz = torch.randn(Hkv, 4, device=DEV, generator=g).half()
    vs = (torch.rand(Hkv, 4, device=DEV, generator=g) * 0.2 + 0.05).half()
    vz = torch.randn(Hkv, 4, device=DEV, generator=g).half()
    c = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    return KK.DecodePlan(q, C.KVQ_FMT_INT4_ASYM, KK.kv_view_static(k, ks, kz),
                         C.KVQ_FMT_INT4_ASYM, KK.kv_view_static(v, vs, vz), c, Hkv, S,
                         1 / math.sqrt(128), 32, keepalive=(k, v, ks, kz, vs, vz))


def _int8_rows_plan(C, KK, B, Hq, Hkv, S, ctx, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, Hq, 128, device=DEV, generator=g).half()
    k = torch.randint(-127, 128, (B, Hkv, S, 128), device=DEV, dtype=torch.int8, generator=g)
    v = torch.randint(-127, 128, (B, Hkv, S, 128), device=DEV, dtype=torch.int8, generator=g)
    ks = (torch.rand(B, Hkv, S, 8, device=DEV, generator=g) * 0.02 + 0.001).half()
    vs = (torch.rand(B, Hkv, S, 8, device=DEV, generator=g) * 0.02 + 0.001).half()
    c = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    return KK.DecodePlan(q, C.KVQ_FMT_INT8_SYM, KK.kv_view_tok(k, ks), C.KVQ_FMT_INT8_SYM,
                         KK.kv_view_tok(v, vs), c, Hkv, S, 1 / math.sqrt(128), 16,
                         keepalive=(k, v, ks, vs))


@pytest.mark.parametrize("kind", ["asym_tiled", "int8_rows"])
def test_noalloc_matches_workspace_entry_point(kind):
    C, KK = _mods()
    make = _asym_tiled_plan if kind == "asym_tiled" else _int8_rows_plan
    # the second call is smaller (fewer rows, shorter context, fewer chunks)
    for i, (B, Hq, Hkv, S, ctx) in enumerate([(4, 28, 4, 9000, [9000, 8999, 4100, 1]),
                                               (2, 12, 2, 700, [700, 33])]):
        print(f"[noalloc] {kind} call {i}: B{B} Hq{Hq} Hkv{Hkv} S{S}", flush=True)
        plan = make(C, KK, B, Hq, Hkv, S, ctx, 11 + i)
        ref = plan.launch().clone()
        plan.out.fill_(float("nan"))
        out = plan.launch_noalloc()
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (kind, i)
        # a repeated call (the merge counters it leaves are cleared again) gives the same bits
        plan.out.zero_()
        out2 = plan.launch_noalloc()
        torch.cuda.synchronize()
        assert torch.equal(out2.view(torch.int16), ref.view(torch.int16)), (kind, i)


def test_noalloc_rejects_workspace_above_the_scratch():
    C, KK = _mods()
    # 64 x 64 query heads x 8 chunks of partials = 17 MB > 16 MiB
    B, Hq, Hkv, S = 64, 64, 8, 2048
    q = torch.zeros(B, Hq, 128, device=DEV, dtype=torch.float16)
    k = torch.zeros(B, Hkv, S, 128, device=DEV, dtype=torch.int8)
    s = torch.ones(B, Hkv, S, 4, device=DEV, dtype=torch.float16)
    c = torch.full((B,), S, dtype=torch.int32, device=DEV)
    plan = KK.DecodePlan(q, C.KVQ_FMT_INT8_SYM, KK.kv_view_tok(k, s), C.KVQ_FMT_INT8_SYM,
                         KK.kv_view_tok(k, s), c, Hkv, S, 0.1, 32, chunk_tokens=256,
                         keepalive=(k, s))
    assert int(C.lib().kvq_decode_workspace_bytes(ctypes.byref(plan.params))) > C.KVQ_NOALLOC_SCRATCH_BYTES
    with pytest.raises(NotImplementedError, match="scratch"):
        plan.launch_noalloc()
