"""CPU restatement of the reference decode-attention oracles (test infrastructure).

``decode_attn_int8_torch_ref`` follows ``_decode_attn_int8_torch_ref``
(/root/reference/src/engine/patch_model.py:281-377) op for op.  K and V are
dequantised in fp16 (code.to(fp16) * fp16 scale), then GQA heads are expanded
with repeat_interleave, and scores, softmax and the weighted sum run in fp32 with
the output cast to q's dtype.  It is also the timed CPU baseline of bench.py
(``cpu_baseline.kind = "port"``).

``decode_attn_asym_ref`` is the dequantise-then-attention oracle of the
asymmetric group-32 format.  The reference has no kernel for this format.  It
dequantises with q * s + zp in fp32 (src/quant/asymmetric_quant.py:196), writes
the fp16 outlier channels back in verbatim, and applies the same fp32 attention.
"""
from __future__ import annotations

from typing import Optional

import torch

from .quant import dequantize_asymmetric_static, dequantize_kivi, dequantize_symmetric, unpack_int4


def prescale_q(q: torch.Tensor, inv_tau: Optional[torch.Tensor]) -> torch.Tensor:
    """q * inv_tau in q's dtype (src/engine/patch_model.py:723,746)."""
    if inv_tau is None:
        return q
    return q * inv_tau.to(dtype=q.dtype).view(1, -1, 1)


def decode_attn_int8_torch_ref(q, k_int8, v_int8, k_scale, v_scale, context_lens, sm_scale):
    """src/engine/patch_model.py:281-377."""
    if q.ndim != 3:
        raise ValueError(f"Expected q [B, H, D], got {q.shape}")
    bsz, q_heads, head_dim = q.shape
    _, kv_heads, _, _ = k_int8.shape
    if q_heads % kv_heads:
        raise ValueError("GQA unsupported: q_heads not divisible by kv_heads")
    G = int(k_scale.shape[-1])
    gs = head_dim // G
    n_rep = q_heads // kv_heads
    outs = []
    for b in range(bsz):
        ctx = int(context_lens[b].item())
        if ctx <= 0:
            outs.append(torch.zeros((q_heads, head_dim), dtype=q.dtype))
            continue
        kq = k_int8[b, :, :ctx, :]
        vq = v_int8[b, :, :ctx, :]
        ks = k_scale[b, :, :ctx, :]
        vs = v_scale[b, :, :ctx, :]
        k = (kq.reshape(kv_heads, ctx, G, gs).to(torch.float16) * ks.unsqueeze(-1)).view(kv_heads, ctx, head_dim)
        v = (vq.reshape(kv_heads, ctx, G, gs).to(torch.float16) * vs.unsqueeze(-1)).view(kv_heads, ctx, head_dim)
        if n_rep != 1:
            k = k.repeat_interleave(n_rep, dim=0)
            v = v.repeat_interleave(n_rep, dim=0)
        scores = torch.einsum("hd,hsd->hs", q[b].float(), k.float()) * sm_scale
        probs = torch.softmax(scores, dim=-1)
        outs.append(torch.einsum("hs,hsd->hd", probs, v.float()).to(dtype=q.dtype))
    return torch.stack(outs, dim=0)


def decode_attn_int4_torch_ref(q, k_packed, v_packed, k_scale, v_scale, context_lens, sm_scale):
    """Packed INT4 through the INT8 oracle after unpack_int4
    (src/engine/patch_model.py:823-831,940-953; src/kernels/triton_decode_attn_int4.py:99-121)."""
    return decode_attn_int8_torch_ref(q, unpack_int4(k_packed), unpack_int4(v_packed),
                                      k_scale, v_scale, context_lens, sm_scale)


def attention_fp32(q16: torch.Tensor, k: torch.Tensor, v: torch.Tensor, context_lens, sm_scale):
    """fp32 GQA decode attention over dequantised k/v [B, Hkv, S, D] (float)."""
    bsz, q_heads, head_dim = q16.shape
    kv_heads = k.shape[1]
    n_rep = q_heads // kv_heads
    outs = []
    for b in range(bsz):
        ctx = int(context_lens[b].item())
        if ctx <= 0:
            outs.append(torch.zeros((q_heads, head_dim), dtype=q16.dtype))
            continue
        kb = k[b, :, :ctx].float().repeat_interleave(n_rep, dim=0)
        vb = v[b, :, :ctx].float().repeat_interleave(n_rep, dim=0)
        scores = torch.einsum("hd,hsd->hs", q16[b].float(), kb) * sm_scale
        probs = torch.softmax(scores, dim=-1)
        outs.append(torch.einsum("hs,hsd->hd", probs, vb).to(q16.dtype))
    return torch.stack(outs, dim=0)


def dequant_asym_k(k_packed, k_scale, k_zp, k_outlier_idx=None, k_outlier_val=None):
    k = dequantize_asymmetric_static(unpack_int4(k_packed), k_scale, k_zp)
    if k_outlier_idx is not None:
        for h in range(k.shape[1]):
            k[:, h, :, k_outlier_idx[h].long()] = k_outlier_val[:, h, :, :].float()
    return k


def decode_attn_asym_ref(q, k_packed, v_packed, k_scale, k_zp, v_scale, v_zp, context_lens,
                         sm_scale, inv_tau=None, k_outlier_idx=None, k_outlier_val=None):
    """Dequantise-then-attention oracle of the asymmetric INT4 group-32 format."""
    k = dequant_asym_k(k_packed, k_scale, k_zp, k_outlier_idx, k_outlier_val)
    v = dequantize_asymmetric_static(unpack_int4(v_packed), v_scale, v_zp)
    return attention_fp32(prescale_q(q, inv_tau), k, v, context_lens, sm_scale)


def decode_attn_k8v4_ref(q, k_int8, k_scale16, v_packed, v_scale, v_zp, context_lens, sm_scale,
                         inv_tau=None):
    """INT8 K dequantised as the reference does (fp16 product) + asymmetric INT4 V (fp32)."""
    B, H, S, D = k_int8.shape
    G = k_scale16.shape[-1]
    k = (k_int8.view(B, H, S, G, D // G).to(torch.float16) * k_scale16.unsqueeze(-1)).view(B, H, S, D)
    v = dequantize_asymmetric_static(unpack_int4(v_packed), v_scale, v_zp)
    return attention_fp32(prescale_q(q, inv_tau), k, v, context_lens, sm_scale)


def decode_attn_mixed_ref(q, k_int8, k_scale, v_codes, v_scale, v_zp, context_lens, sm_scale,
                          inv_tau=None):
    """MixedKVCache (src/cache/mixed_kv_cache.py:170-190, 242-254) decoded as the reference
    decodes kv_mode="int4_mixed_kv" (src/engine/generate_loop.py:1357-1364): get_kv's K =
    code x its group's scale in fp32 (dequantize_symmetric_int8, src/quant/int8_basic.py:
    167-246) and V = code x s + z of its token in fp32 (dequantize_asymmetric_per_token,
    src/quant/asymmetric_quant.py:273-290), each cast to fp16, then fp32 attention.
    v_codes are the unpacked int8 codes [B, H, S, D]."""
    k = dequantize_symmetric(k_int8, k_scale.float()).to(torch.float16)
    v = dequantize_kivi(v_codes, v_scale, v_zp, per_channel=False).to(torch.float16)
    return attention_fp32(prescale_q(q, inv_tau), k, v, context_lens, sm_scale)


def decode_attn_mixed_bits_ref(q, k_store, k_bits, k_scale, v_store, v_bits, v_scale, v_zp,
                               context_lens, sm_scale, inv_tau=None, k_zp=None):
    """MixedKVCache of any (k_bits, v_bits) pair of {4, 8, 16} (src/cache/mixed_kv_cache.py:
    150-254), decoded as get_kv then attention: an 8-bit side is code x its group's scale in
    fp32, a 4-bit side (packed) code x s + z of its token in fp32 (K: k_scale / k_zp
    [B, H, S]), a 16-bit side the stored fp16 values; each side cast to fp16, then fp32
    attention."""
    if k_bits == 16:
        k = k_store
    elif k_bits == 8:
        k = dequantize_symmetric(k_store, k_scale.float()).to(torch.float16)
    else:
        k = dequantize_kivi(unpack_int4(k_store), k_scale, k_zp, per_channel=False).to(torch.float16)
    if v_bits == 16:
        v = v_store
    elif v_bits == 8:
        v = dequantize_symmetric(v_store, v_scale.float()).to(torch.float16)
    else:
        v = dequantize_kivi(unpack_int4(v_store), v_scale, v_zp, per_channel=False).to(torch.float16)
    return attention_fp32(prescale_q(q, inv_tau), k, v, context_lens, sm_scale)


def dequant_kivi_side(store, bits: int, s, z, per_channel: bool) -> torch.Tensor:
    """One side of a KIVI-family layer as float (src/cache/role_aware_allocator_cache.py:
    402-440): 4 bits packed, 8 bits int8 codes, both code x s + z in fp32 (per channel for K,
    per token for V); 16 bits the stored fp16 values."""
    if bits == 16:
        return store.float()
    codes = unpack_int4(store) if bits == 4 else store
    return dequantize_kivi(codes, s, z, per_channel=per_channel)


def decode_attn_kivi_family_ref(q, k_store, k_bits, k_scale, k_zp, v_store, v_bits, v_scale, v_zp,
                                context_lens, sm_scale, inv_tau=None):
    """A KIVI-family layer of any (k_bits, v_bits) pair from {4, 8, 16}: K and V dequantised
    in fp32 (dequant_kivi_side), fp32 logits of q' = fp16(q * inv_tau), fp32 softmax and PV."""
    k = dequant_kivi_side(k_store, k_bits, k_scale, k_zp, True)
    v = dequant_kivi_side(v_store, v_bits, v_scale, v_zp, False)
    return attention_fp32(prescale_q(q, inv_tau), k, v, context_lens, sm_scale)


def decode_attn_kivi_ref(q, k_packed, v_packed, k_scale, k_zp, v_scale, v_zp, context_lens,
                         sm_scale, inv_tau=None):
    """KIVI layout (src/kernels/triton_decode_attn_int4_asym.py:28-160): K and V dequantised
    in fp32 ((n - 8) s + z, K per channel, V per token), fp32 logits of fp16 q, fp32
    softmax and PV."""
    k = dequantize_kivi(unpack_int4(k_packed), k_scale, k_zp, per_channel=True)
    v = dequantize_kivi(unpack_int4(v_packed), v_scale, v_zp, per_channel=False)
    return attention_fp32(prescale_q(q, inv_tau), k, v, context_lens, sm_scale)
