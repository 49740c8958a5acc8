"""Writes the golden fixtures of tests/golden/*.npz from the CPU oracle.

One small case per benchmark configuration (the configurations' head counts and formats
at a reduced batch and context) plus one INT4-symmetric case for ``decode_attn_int4``.
Each fixture holds its inputs (fp16 K/V rows, q, inv_tau, context lengths, static tables)
and the expected outputs:

* the quantised cache exactly as the reference's torch quantizers produce it (codes,
  per-token scales where the format stores them, fp16 outlier channels);
* the decode attention output of the reference's dequantise-then-attention path (fp16).

The fixtures pin the oracle against later edits (tests/test_golden.py) and give the GPU
tests a fixed target (tests/test_gpu_golden.py).  Regenerate with

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from llm_kvcache_quantization_amd import calib  # noqa: E402
from llm_kvcache_quantization_amd import synthetic as SY  # noqa: E402
from oracle import attn as OA  # noqa: E402
from oracle import quant as OQ  # noqa: E402

SM_SCALE = 1.0 / math.sqrt(128)

# name -> (config index, batch, cache tokens, context lengths)
CASES = {
    "cfg0": (0, 1, 40, [40]),
    "cfg1": (1, 2, 33, [33, 20]),
    "cfg2": (2, 2, 40, [40, 17]),
    "cfg3": (3, 1, 45, [45]),
    "cfg4": (4, 2, 16, [16, 5]),
    "int4sym": (0, 1, 40, [40]),
}


def make(name: str) -> dict:
    ci, B, S, ctx = CASES[name]
    cfg = SY.CONFIGS[ci]
    t = SY.calibrate(cfg, 0)
    g = torch.Generator().manual_seed(SY.seed_for(ci, 0) + 777 + (5 if name == "int4sym" else 0))
    k, v = SY.draw_kv(cfg, 0, B, S, g)
    q = SY.draw_q(cfg, B, g)
    tau = SY.inv_tau(cfg)[0]
    cl = torch.tensor(ctx, dtype=torch.int32)
    f = dict(k=k, v=v, q=q, inv_tau=tau, context_lens=cl, sm_scale=torch.tensor(SM_SCALE))
    q16 = OA.prescale_q(q, tau)
    if name == "int4sym":
        # INT4KVCache with static absmax/7 tables; scales go to the kernel as fp16, the
        # way the reference's decode glue casts them (src/engine/patch_model.py:915-916)
        gcal = torch.Generator().manual_seed(SY.seed_for(ci, 0) + 500_000)
        kc, vc = SY.draw_kv(cfg, 0, 1, SY.CALIB_TOKENS, gcal)
        sk, sv = calib.int4_static_scale(kc, 32), calib.int4_static_scale(vc, 32)
        kq, ks = OQ.int4_cache_quantize(k, sk, 32)
        vq, vs = OQ.int4_cache_quantize(v, sv, 32)
        kp, vp = OQ.pack_int4(kq), OQ.pack_int4(vq)
        out = OA.decode_attn_int4_torch_ref(q16, kp, vp, ks.to(torch.float16), vs.to(torch.float16),
                                            cl, SM_SCALE)
        f.update(k_static=sk, v_static=sv, k_codes=kp.view(torch.uint8), v_codes=vp.view(torch.uint8),
                 k_scale_tok=ks, v_scale_tok=vs, out=out)
        return f
    if cfg.k_format == "int8":
        k8, ks = OQ.int8_cache_quantize(k, t.k_scale, 32)
        f.update(k_static=t.k_scale, k_codes=k8, k_scale_tok=ks)
    else:
        kq = OQ.quantize_asymmetric_static(k, t.k_scale, t.k_zp)
        f.update(k_static=t.k_scale, k_zp=t.k_zp, k_codes=OQ.pack_int4(kq).view(torch.uint8))
        if cfg.outlier_channels:
            oi = t.k_outlier_idx
            ov = torch.stack([k[:, h][..., oi[h].long()] for h in range(cfg.kv_heads)], dim=1)
            f.update(k_outlier_idx=oi, k_outlier_val=ov)
    if cfg.v_format == "int8":
        v8, vs = OQ.int8_cache_quantize(v, t.v_scale, 32)
        f.update(v_static=t.v_scale, v_codes=v8, v_scale_tok=vs)
        out = OA.decode_attn_int8_torch_ref(q16, k8, v8, ks, vs, cl, SM_SCALE)
    else:
        vq = OQ.quantize_asymmetric_static(v, t.v_scale, t.v_zp)
        vp = OQ.pack_int4(vq)
        f.update(v_static=t.v_scale, v_zp=t.v_zp, v_codes=vp.view(torch.uint8))
        if cfg.k_format == "int8":
            out = OA.decode_attn_k8v4_ref(q, k8, ks, vp, t.v_scale, t.v_zp, cl, SM_SCALE, inv_tau=tau)
        else:
            out = OA.decode_attn_asym_ref(q, f["k_codes"], vp, t.k_scale, t.k_zp, t.v_scale, t.v_zp, cl,
                                          SM_SCALE, inv_tau=tau, k_outlier_idx=f.get("k_outlier_idx"),
                                          k_outlier_val=f.get("k_outlier_val"))
    f["out"] = out
    return f


def to_numpy(f: dict) -> dict:
    return {k: v.numpy() for k, v in f.items()}


def main():
    torch.set_num_threads(1)
    for name in CASES:
        arrs = to_numpy(make(name))
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrs)
        print(f"{path}: {os.path.getsize(path)} bytes, {sorted(arrs)}")


if __name__ == "__main__":
    main()
