"""The HIP path against the committed golden fixtures (tests/golden/*.npz).

Each fixture is appended through the cache engine of its format in two calls (so the
second lands at a nonzero write position).  The codes, per-token scales and outlier
channels must equal the fixture bit for bit.  Decode attention through the
reference-named API must then match the fixture's output within max-abs 2e-3 and
cosine >= 0.9999.
"""
import glob
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
ATOL = 2e-3
COS_MIN = 0.9999
HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k].copy()) for k in z.files}


def check_out(out, ref, tag):
    o, r = out.float().cpu(), ref.float()
    err = (o - r).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(o.flatten(), r.flatten(), dim=0).item()
    print(f"[{tag}] max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= ATOL and cos >= COS_MIN, (tag, err, cos)


def append_twice(cache, k, v):
    S = k.shape[2]
    cut = max(1, S - 5)
    cache.append(0, k[:, :, :cut].to(DEV), v[:, :, :cut].to(DEV))
    cache.append(0, k[:, :, cut:].to(DEV), v[:, :, cut:].to(DEV))


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p)[:-4])
def test_gpu_matches_golden(path):
    import llm_kvcache_quantization_amd as K
    from llm_kvcache_quantization_amd import _capi

    _capi.lib()
    name = os.path.basename(path)[:-4]
    f = load(path)
    k, v, q, tau, cl = f["k"], f["v"], f["q"], f["inv_tau"], f["context_lens"]
    sm = float(f["sm_scale"])
    qd, taud, cld = q.to(DEV), tau.to(DEV), cl.to(DEV)
    print(f"[golden {name}] k {tuple(k.shape)} q {tuple(q.shape)} ctx {cl.tolist()}", flush=True)
    if name == "int4sym":
        cache = K.INT4KVCache(1, device=DEV, group_size=32, static_k_scale=f["k_static"][None],
                              static_v_scale=f["v_static"][None], check_numerics=True)
        append_twice(cache, k, v)
        kp, vp, ks, vs = cache.get_int4_tensors(0)
        assert torch.equal(kp.cpu().view(torch.uint8), f["k_codes"])
        assert torch.equal(vp.cpu().view(torch.uint8), f["v_codes"])
        assert torch.equal(ks.cpu(), f["k_scale_tok"]) and torch.equal(vs.cpu(), f["v_scale_tok"])
        out = K.decode_attn_int4(qd * taud.view(1, -1, 1), kp, vp, ks.to(torch.float16),
                                 vs.to(torch.float16), cld, sm)
    elif "k_zp" in f:  # configs 2 and 3: INT4 asym K and V
        oi = f.get("k_outlier_idx")
        cache = K.INT4AsymKVCache(1, f["k_static"][None], f["k_zp"][None], f["v_static"][None],
                                  f["v_zp"][None], device=DEV,
                                  k_outlier_idx=None if oi is None else oi[None], check_numerics=True)
        append_twice(cache, k, v)
        kc, vc, ks, kz, vs, vz, goi, gov = cache.get_int4_g32_tensors(0)
        S = k.shape[2]
        assert torch.equal(kc.cpu(), f["k_codes"])
        assert torch.equal(K.untile_v(vc, S).cpu(), f["v_codes"])  # V is kept in TILE32
        if oi is not None:
            assert torch.equal(gov.cpu(), f["k_outlier_val"])
        # V as packed rows takes the row-layout kernel
        out_rows = K.decode_attn_int4_asym(qd, kc, K.untile_v(vc, S).contiguous(), ks, kz, vs, vz,
                                           cld, sm, inv_tau=taud, k_outlier_idx=goi,
                                           k_outlier_val=gov)
        check_out(out_rows, f["out"], name + " rows")
        out = K.decode_attn_int4_asym(qd, kc, vc, ks, kz, vs, vz, cld, sm, inv_tau=taud,
                                      k_outlier_idx=goi, k_outlier_val=gov)
    elif "v_zp" in f:  # config 4: INT8 K, INT4 asym V
        cache = K.K8V4KVCache(1, f["k_static"][None], f["v_static"][None], f["v_zp"][None],
                              device=DEV, check_numerics=True)
        append_twice(cache, k, v)
        k8, ks, vc, vs, vz = cache.get_k8v4_tensors(0)
        S = k.shape[2]
        assert torch.equal(k8.cpu(), f["k_codes"])
        assert torch.equal(K.untile_v(vc, S).cpu(), f["v_codes"])  # V is kept in TILE32
        assert torch.equal(ks.cpu(), f["k_scale_tok"])
        # V as packed rows takes the row-layout kernel
        out_rows = K.decode_attn_k8v4(qd, k8, ks, K.untile_v(vc, S).contiguous(), vs, vz, cld, sm,
                                      inv_tau=taud)
        check_out(out_rows, f["out"], name + " rows")
        out = K.decode_attn_k8v4(qd, k8, ks, vc, vs, vz, cld, sm, inv_tau=taud)
    else:  # configs 0 and 1: INT8 K and V
        cache = K.INT8KVCache(1, device=DEV, group_size=32, static_k_scale=f["k_static"][None],
                              static_v_scale=f["v_static"][None], check_numerics=True)
        append_twice(cache, k, v)
        k8, v8, ks, vs = cache.get_int8_tensors(0)
        assert torch.equal(k8.cpu(), f["k_codes"]) and torch.equal(v8.cpu(), f["v_codes"])
        assert torch.equal(ks.cpu(), f["k_scale_tok"]) and torch.equal(vs.cpu(), f["v_scale_tok"])
        out = K.decode_attn_int8(qd * taud.view(1, -1, 1), k8, v8, ks, vs, cld, sm)
    check_out(out, f["out"], name)
