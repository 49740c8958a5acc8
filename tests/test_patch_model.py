"""CPU tests of the attention hook (llm_kvcache_quantization_amd/patch.py).

They restate the behaviour the reference's own tests pin for src/engine/patch_model.py
(tests/test_patch_model.py: RoPE helpers :53-215, the torch decode path :218-436, the HF
cache duck types :438-637, INT4 materialisation :640-748, the patch and its dispatch
:841-1300), with fake engines where the reference uses fakes, and add an end-to-end check
on a randomly initialised transformers Qwen2 model: decode steps through the patched
attention and a torch fake engine match the unpatched model.
"""
import inspect
import math
import warnings
from unittest.mock import MagicMock, patch as mock_patch

import pytest
import torch

from llm_kvcache_quantization_amd import patch as P


# ---------------------------------------------------------------- fakes


class FakeEngine:
    """Stand-in for a quantized engine: records appends, serves get_kv from a dict."""

    def __init__(self, num_layers=4, seq_len=10):
        self.num_layers = num_layers
        self._seq_len = seq_len
        self.appended = []
        self.kv = {}

    def get_seq_len(self):
        return self._seq_len

    def get_int8_tensors(self, layer_idx):
        return (None, None, None, None)

    def get_kv(self, layer_idx):
        return self.kv.get(layer_idx, (None, None))

    def append(self, layer_idx, k, v):
        self.appended.append((layer_idx, k, v))


class NonFusedEngine:
    num_layers = 2

    def get_seq_len(self):
        return 5


class TorchAttnEngine:
    """A float cache (no quantization) whose append_decode_attn is plain softmax attention
    in fp32: the hook's integration is checked against the unpatched model with it."""

    decode_attn_impl = "triton_fused"

    def __init__(self, num_layers, inv_tau=None):
        self.num_layers = num_layers
        self.inv_tau = inv_tau
        self.use_attn_temperature = inv_tau is not None
        self.k = [None] * num_layers
        self.v = [None] * num_layers
        self.calls = []

    def get_int8_tensors(self, layer_idx):
        raise AssertionError("the HIP branch must not read the cache tensors")

    def get_seq_len(self):
        return 0 if self.k[0] is None else int(self.k[0].shape[2])

    def append(self, i, k, v):
        self.k[i] = k if self.k[i] is None else torch.cat([self.k[i], k], 2)
        self.v[i] = v if self.v[i] is None else torch.cat([self.v[i], v], 2)

    def get_kv(self, i):
        return self.k[i], self.v[i]

    def append_decode_attn(self, i, q, k, v, sm_scale=None, inv_tau=None):
        self.calls.append((i, q.clone(), None if inv_tau is None else inv_tau.clone()))
        self.append(i, k, v)
        if inv_tau is not None:
            q = (q.float() * inv_tau.float().view(1, -1, 1)).to(q.dtype)
        K, V = self.k[i].float(), self.v[i].float()
        rep = q.shape[1] // K.shape[1]
        K, V = K.repeat_interleave(rep, 1), V.repeat_interleave(rep, 1)
        s = torch.einsum("bhd,bhsd->bhs", q.float(), K) * sm_scale
        return torch.einsum("bhs,bhsd->bhd", s.softmax(-1), V).to(q.dtype)


def pack_nibbles(codes: torch.Tensor) -> torch.Tensor:
    """Codes in [-8, 7] -> bytes (c[2i] + 8) << 4 | (c[2i+1] + 8) (src/quant/int4_basic.py:230-271)."""
    u = (codes.to(torch.int16) + 8)
    return ((u[..., 0::2] << 4) | u[..., 1::2]).to(torch.uint8).view(torch.int8)


# ---------------------------------------------------------------- RoPE helpers


def test_rotate_half_values_and_order_four():
    x = torch.tensor([1.0, 2.0, 3.0, 4.0])
    assert torch.equal(P._rotate_half(x), torch.tensor([-3.0, -4.0, 1.0, 2.0]))
    y = torch.randn(2, 3, 5, 8)
    assert torch.equal(P._rotate_half(P._rotate_half(y)), -y)
    assert torch.equal(P._rotate_half(P._rotate_half(P._rotate_half(P._rotate_half(y)))), y)


def test_apply_rope_identity_and_quarter_turn():
    q, k = torch.randn(2, 3, 4, 8), torch.randn(2, 3, 4, 8)
    one, zero = torch.ones(4, 8), torch.zeros(4, 8)
    q1, k1 = P._apply_rope(q, k, one, zero)
    assert torch.equal(q1, q) and torch.equal(k1, k)
    q2, k2 = P._apply_rope(q, k, zero, one)
    assert torch.equal(q2, P._rotate_half(q)) and torch.equal(k2, P._rotate_half(k))


def _cos_sin(pos, dim, base=10000.0, dtype=torch.float32):
    inv = 1.0 / base ** (torch.arange(0, dim, 2, dtype=dtype) / dim)
    ang = torch.outer(pos.to(dtype), inv)
    emb = torch.cat([ang, ang], -1)
    return emb.cos(), emb.sin()


def test_apply_rope_broadcast_shapes_agree():
    q, k = torch.randn(3, 2, 5, 8), torch.randn(3, 2, 5, 8)
    c, s = _cos_sin(torch.arange(5), 8)
    ref = P._apply_rope(q, k, c, s)
    for cc, ss in ((c[None], s[None]), (c[None].expand(3, -1, -1), s[None].expand(3, -1, -1)),
                   (c[None, None], s[None, None])):
        got = P._apply_rope(q, k, cc, ss)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])


def test_apply_rope_partial_rotary_passes_tail_through():
    q, k = torch.randn(1, 2, 3, 8), torch.randn(1, 2, 3, 8)
    c, s = _cos_sin(torch.arange(3), 4)
    qo, ko = P._apply_rope(q, k, c, s)
    assert torch.equal(qo[..., 4:], q[..., 4:]) and torch.equal(ko[..., 4:], k[..., 4:])
    qf, _ = P._apply_rope(q[..., :4].contiguous(), k[..., :4].contiguous(), c, s)
    assert torch.equal(qo[..., :4], qf)


def test_apply_rope_rejects_rotary_dim_above_head_dim():
    q = torch.randn(1, 1, 2, 4)
    c, s = _cos_sin(torch.arange(2), 8)
    with pytest.raises(ValueError):
        P._apply_rope(q, q, c, s)


def test_apply_rope_scores_depend_on_relative_position_only():
    """<R(m) q, R(n) k> is a function of m - n (the defining property of RoPE)."""
    torch.manual_seed(1)
    q, k = torch.randn(1, 1, 1, 16, dtype=torch.float64), torch.randn(1, 1, 1, 16, dtype=torch.float64)

    def score(m, n):
        cm, sm = _cos_sin(torch.tensor([m]), 16, dtype=torch.float64)
        cn, sn = _cos_sin(torch.tensor([n]), 16, dtype=torch.float64)
        qm, _ = P._apply_rope(q, q, cm, sm)
        _, kn = P._apply_rope(k, k, cn, sn)
        return float((qm * kn).sum())

    assert score(7, 3) == pytest.approx(score(14, 10), rel=1e-9)
    assert score(5, 5) == pytest.approx(score(0, 0), rel=1e-9)
    assert score(9, 2) != pytest.approx(score(9, 3), rel=1e-6)


# ---------------------------------------------------------------- the torch decode path


def _ref_inputs(B=1, Hq=1, Hkv=1, S=4, D=4, G=1, dtype=torch.float16, ctx=None, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).to(dtype)
    k = torch.randint(-3, 4, (B, Hkv, S, D), generator=g, dtype=torch.int8)
    v = torch.randint(-3, 4, (B, Hkv, S, D), generator=g, dtype=torch.int8)
    ks = torch.ones(B, Hkv, S, G, dtype=dtype)
    vs = torch.ones(B, Hkv, S, G, dtype=dtype)
    cl = torch.full((B,), S if ctx is None else ctx, dtype=torch.int32)
    return q, k, v, ks, vs, cl, 1.0 / math.sqrt(D)


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(1, 1, 1, 4, 4), (2, 4, 4, 8, 8), (1, 4, 2, 6, 8)])
def test_torch_ref_output_shape(B, Hq, Hkv, S, D):
    out = P._decode_attn_int8_torch_ref(*_ref_inputs(B, Hq, Hkv, S, D))
    assert out.shape == (B, Hq, D)


def test_torch_ref_single_token_returns_value_row():
    q = torch.ones(1, 1, 4, dtype=torch.float16)
    k = torch.ones(1, 1, 1, 4, dtype=torch.int8)
    v = torch.tensor([[[[2, 3, 4, 5]]]], dtype=torch.int8)
    s = torch.ones(1, 1, 1, 1, dtype=torch.float16)
    out = P._decode_attn_int8_torch_ref(q, k, v, s, s, torch.tensor([1], dtype=torch.int32), 1.0)
    assert torch.equal(out, torch.tensor([[[2.0, 3.0, 4.0, 5.0]]], dtype=torch.float16))


def test_torch_ref_empty_context_rows_are_zero():
    q, k, v, ks, vs, _, sm = _ref_inputs(B=2, Hq=2, Hkv=2)
    out = P._decode_attn_int8_torch_ref(q, k, v, ks, vs, torch.tensor([0, 4], dtype=torch.int32), sm)
    assert torch.all(out[0] == 0) and torch.any(out[1] != 0)


def test_torch_ref_two_token_closed_form():
    """q = e0, K = V = I: scores [1, 0] -> out = [e/(e+1), 1/(e+1)]."""
    q = torch.tensor([[[1.0, 0.0]]], dtype=torch.float16)
    kv = torch.tensor([[[[1, 0], [0, 1]]]], dtype=torch.int8)
    s = torch.ones(1, 1, 2, 1, dtype=torch.float16)
    out = P._decode_attn_int8_torch_ref(q, kv, kv, s, s, torch.tensor([2], dtype=torch.int32), 1.0)
    e = math.e
    want = torch.tensor([[[e / (e + 1), 1 / (e + 1)]]])
    assert torch.allclose(out.float(), want, atol=1e-3)


def test_torch_ref_group_scales_and_gqa_against_float64_brute_force():
    torch.manual_seed(3)
    B, Hq, Hkv, S, D, G = 2, 4, 2, 5, 8, 2
    q = torch.randn(B, Hq, D, dtype=torch.float16)
    k = torch.randint(-127, 128, (B, Hkv, S, D), dtype=torch.int8)
    v = torch.randint(-127, 128, (B, Hkv, S, D), dtype=torch.int8)
    ks = (torch.rand(B, Hkv, S, G) * 0.02 + 0.001).half()
    vs = (torch.rand(B, Hkv, S, G) * 0.02 + 0.001).half()
    cl = torch.tensor([3, 5], dtype=torch.int32)
    out = P._decode_attn_int8_torch_ref(q, k, v, ks, vs, cl, 0.25)
    for b in range(B):
        n = int(cl[b])
        for h in range(Hq):
            kh = h // (Hq // Hkv)
            kd = (k[b, kh, :n].double().view(n, G, D // G) * ks[b, kh, :n].double()[..., None]).view(n, D)
            vd = (v[b, kh, :n].double().view(n, G, D // G) * vs[b, kh, :n].double()[..., None]).view(n, D)
            p = torch.softmax(kd @ q[b, h].double() * 0.25, 0)
            want = p @ vd
            assert torch.allclose(out[b, h].double(), want, atol=2e-3, rtol=2e-3), (b, h)


def test_torch_ref_batch_rows_are_independent():
    q, k, v, ks, vs, _, sm = _ref_inputs(B=2, S=6, seed=5)
    both = P._decode_attn_int8_torch_ref(q, k, v, ks, vs, torch.tensor([3, 6], dtype=torch.int32), sm)
    first = P._decode_attn_int8_torch_ref(q[:1], k[:1, :, :3], v[:1, :, :3], ks[:1, :, :3], vs[:1, :, :3],
                                          torch.tensor([3], dtype=torch.int32), sm)
    assert torch.equal(both[:1], first)


def test_torch_ref_validation_errors():
    q, k, v, ks, vs, cl, sm = _ref_inputs(Hq=3, Hkv=2)
    with pytest.raises(ValueError):
        P._decode_attn_int8_torch_ref(q, k, v, ks, vs, cl, sm)          # 3 % 2
    q, k, v, ks, vs, cl, sm = _ref_inputs()
    with pytest.raises(ValueError):
        P._decode_attn_int8_torch_ref(q[:, :, None], k, v, ks, vs, cl, sm)
    with pytest.raises(ValueError):
        P._decode_attn_int8_torch_ref(q, torch.zeros(1, 1, 4, 6, dtype=torch.int8), v, ks, vs, cl, sm)
    with pytest.raises(ValueError):
        P._decode_attn_int8_torch_ref(q, k, v, ks[..., 0], vs, cl, sm)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_torch_ref_output_dtype_follows_query(dtype):
    out = P._decode_attn_int8_torch_ref(*_ref_inputs(S=2, dtype=dtype))
    assert out.dtype == dtype


# ---------------------------------------------------------------- HF cache duck types


def test_wrapper_delegates_to_engine():
    eng = FakeEngine(num_layers=6, seq_len=42)
    eng.kv.update({i: (f"k{i}", f"v{i}") for i in range(6)})
    w = P.INT8CacheWrapper(eng, layer_idx=2)
    assert w.layer_idx == 2 and w.get_seq_length() == 42 and w.get_seq_length(layer_idx=99) == 42
    assert len(w) == 6 and w[3] == ("k3", "v3") and list(w)[5] == ("k5", "v5")
    w.update(torch.zeros(1), torch.ones(1), layer_idx=1)
    assert len(eng.appended) == 1 and eng.appended[0][0] == 1


def test_container_interface():
    eng = FakeEngine(num_layers=3, seq_len=50)
    eng.kv.update({i: (f"k{i}", f"v{i}") for i in range(3)})
    c = P.INT8CacheWrapperContainer(eng, num_layers=3)
    assert len(c) == 3 and c.get_seq_length() == 50 and c.get_query_offset(1) == 50
    assert all(isinstance(w, P.INT8CacheWrapper) and w.layer_idx == i for i, w in enumerate(c))
    assert c[1].layer_idx == 1 and c.get_max_cache_shape() is None
    assert c.to_legacy_cache() == (("k0", "v0"), ("k1", "v1"), ("k2", "v2"))
    assert c.is_sliding == [False] * 3
    c.update(torch.zeros(1), torch.ones(1), layer_idx=0)
    assert eng.appended[0][0] == 0


def test_container_mask_sizes():
    c = P.INT8CacheWrapperContainer(FakeEngine(num_layers=2, seq_len=50), num_layers=2)
    assert c.get_mask_sizes(None, 0) == (50, 0)
    assert c.get_mask_sizes(torch.arange(5), 0) == (55, 0)      # a position tensor (4.x)
    assert c.get_mask_sizes(1, 0) == (51, 0)                      # a query length (5.x)


def test_container_rejects_engines_without_quantized_getters():
    with pytest.raises(TypeError):
        P.INT8CacheWrapperContainer(NonFusedEngine(), num_layers=2)


# ---------------------------------------------------------------- INT4 materialisation


def test_materialize_unpacked_passthrough_and_shape_errors():
    k = torch.randint(-7, 8, (1, 2, 4, 8), dtype=torch.int8)
    v = torch.randint(-7, 8, (1, 2, 4, 8), dtype=torch.int8)
    ko, vo = P._materialize_int4_cache_as_int8(k, v, head_dim=8, bit_packed=False)
    assert ko is k and vo is v
    with pytest.raises(ValueError):
        P._materialize_int4_cache_as_int8(torch.zeros(1, 2, 4, 10, dtype=torch.int8), v, head_dim=8,
                                          bit_packed=False)
    with pytest.raises(ValueError):
        P._materialize_int4_cache_as_int8(k, torch.zeros(1, 2, 4, 6, dtype=torch.int8), head_dim=8,
                                          bit_packed=False)
    with pytest.raises(ValueError):
        P._materialize_int4_cache_as_int8(torch.zeros(1, 2, 4, 5, dtype=torch.int8),
                                          torch.zeros(1, 2, 4, 5, dtype=torch.int8), head_dim=8,
                                          bit_packed=True)


def test_materialize_packed_round_trip_full_range():
    k = torch.randint(-8, 8, (2, 4, 8, 16), dtype=torch.int8)
    v = torch.randint(-8, 8, (2, 4, 8, 16), dtype=torch.int8)
    ko, vo = P._materialize_int4_cache_as_int8(pack_nibbles(k), pack_nibbles(v), head_dim=16, bit_packed=True)
    assert ko.dtype == torch.int8 and torch.equal(ko, k) and torch.equal(vo, v)
    edge = torch.tensor([[[[-8, -7, 0, 7]]]], dtype=torch.int8)
    ko, _ = P._materialize_int4_cache_as_int8(pack_nibbles(edge), pack_nibbles(edge), head_dim=4, bit_packed=True)
    assert torch.equal(ko, edge)


# ---------------------------------------------------------------- apply / remove the patch


def _mock_model(num_layers=2, head_dim=8, q_heads=4, kv_heads=2, plural=False):
    log = []
    if plural:
        def original(self, hidden_states, attention_mask=None, position_ids=None, past_key_values=None,
                     output_attentions=False, use_cache=False):
            log.append(dict(past_key_values=past_key_values, attention_mask=attention_mask))
            return ("original_output", None)
    else:
        def original(self, hidden_states, attention_mask=None, position_ids=None, past_key_value=None,
                     output_attentions=False, use_cache=False):
            log.append(dict(past_key_value=past_key_value, attention_mask=attention_mask))
            return ("original_output", None)
    Attn = type("MockAttnPlural" if plural else "MockAttn", (), {"forward": original})
    layers = []
    for i in range(num_layers):
        a = Attn()
        a.head_dim = head_dim
        a.layer_idx = i
        layer = MagicMock()
        layer.self_attn = a
        layers.append(layer)
    model = MagicMock()
    model.model.layers = layers
    model.config.num_attention_heads = q_heads
    model.config.num_key_value_heads = kv_heads
    return model, log, Attn, original


@pytest.fixture(autouse=True)
def _fresh_patch_state():
    P._reset_fused_state()
    yield
    P._reset_fused_state()


def test_patch_replaces_forward_once_and_remove_restores():
    model, _, Attn, original = _mock_model()
    P.apply_int8_fused_patch(model)
    assert Attn.forward is not original and Attn._original_forward is original
    P.apply_int8_fused_patch(model)                    # a second patch keeps the true original
    assert Attn._original_forward is original
    assert P.remove_int8_fused_patch(model) is True
    assert Attn.forward is original and not hasattr(Attn, "_original_forward")
    assert P.remove_int8_fused_patch(model) is False


def test_remove_without_model_restores_every_patched_class():
    m1, _, A1, o1 = _mock_model()
    m2, _, A2, o2 = _mock_model(plural=True)
    P.apply_int8_fused_patch(m1)
    P.apply_int8_fused_patch(m2)
    assert P.remove_int8_fused_patch() is True
    assert A1.forward is o1 and A2.forward is o2


def test_patch_sets_layer_metadata():
    model, _, _, _ = _mock_model(num_layers=3, q_heads=8, kv_heads=2)
    for layer in model.model.layers:
        del layer.self_attn.layer_idx
    P.apply_int8_fused_patch(model)
    for i, layer in enumerate(model.model.layers):
        a = layer.self_attn
        assert a.layer_idx == i and a._kv_num_attention_heads == 8 and a._kv_num_key_value_heads == 2


def test_patch_needs_decoder_layers():
    class Broken:
        @property
        def layers(self):
            raise AttributeError("no layers")

    model = MagicMock()
    model.model = Broken()
    with pytest.raises(ValueError):
        P.apply_int8_fused_patch(model)


def _route(model, Attn, hidden, **kw):
    with mock_patch.object(P, "_fused_forward_impl") as fused:
        fused.return_value = ("fused_output", None)
        Attn.forward(model.model.layers[0].self_attn, hidden, **kw)
        return fused


def test_proxy_dispatch():
    model, log, Attn, _ = _mock_model()
    P.apply_int8_fused_patch(model)
    eng = FakeEngine(num_layers=2, seq_len=10)
    w = P.INT8CacheWrapper(eng, 0)
    one, five = torch.randn(1, 1, 32), torch.randn(1, 5, 32)
    # a one-token step over a wrapper / container / duck-typed cache takes the fused path
    f = _route(model, Attn, one, past_key_value=w)
    assert f.call_args[0][2] is w
    f = _route(model, Attn, one, past_key_value=P.INT8CacheWrapperContainer(eng, 2))
    assert isinstance(f.call_args[0][2], P.INT8CacheWrapper) and f.call_args[0][2].layer_idx == 0

    class Duck:
        engine = eng

        def __getitem__(self, i):
            return w

    assert _route(model, Attn, one, past_key_value=Duck()).call_args[0][2] is w
    assert _route(model, Attn, one, past_key_values=w).call_count == 1          # plural alias
    assert _route(model, Attn, one, past_key_value=MagicMock(spec=P.INT8CacheWrapper)).call_count == 1
    # prefill, no cache, or something that is not a cache: the original forward
    for kw in (dict(past_key_value=w), ):
        assert _route(model, Attn, five, **kw).call_count == 0
    assert _route(model, Attn, one, past_key_value=None).call_count == 0
    assert _route(model, Attn, one, past_key_value="not_a_cache").call_count == 0
    assert len(log) == 3


def test_proxy_filters_kwargs_for_the_original_forward():
    model, log, Attn, _ = _mock_model()
    P.apply_int8_fused_patch(model)
    mask = torch.ones(1, 1, 5, 5)
    Attn.forward(model.model.layers[0].self_attn, torch.randn(1, 5, 32), attention_mask=mask,
                 past_key_value=None, cache_position=torch.tensor([0]),
                 position_embeddings=(torch.randn(1), torch.randn(1)))
    assert len(log) == 1 and log[0]["attention_mask"] is mask
    assert set(log[0]) == {"past_key_value", "attention_mask"}


def test_proxy_routes_cache_to_plural_signature():
    model, log, Attn, _ = _mock_model(plural=True)
    P.apply_int8_fused_patch(model)
    Attn.forward(model.model.layers[0].self_attn, torch.randn(1, 5, 32), past_key_value="some_cache")
    assert log[0]["past_key_values"] == "some_cache"


def test_proxy_warns_on_output_attentions():
    model, _, Attn, _ = _mock_model()
    P.apply_int8_fused_patch(model)
    w = P.INT8CacheWrapper(FakeEngine(num_layers=2), 0)
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        _route(model, Attn, torch.randn(1, 1, 32), past_key_value=w, output_attentions=True)
    assert any("output_attentions" in str(r.message) for r in rec if issubclass(r.category, UserWarning))


# ---------------------------------------------------------------- the fused forward on a real HF model


def _tiny_qwen2(num_layers=2, hidden=256, heads=4, kv_heads=2, seed=0):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(seed)
    cfg = Qwen2Config(vocab_size=97, hidden_size=hidden, intermediate_size=2 * hidden,
                      num_hidden_layers=num_layers, num_attention_heads=heads,
                      num_key_value_heads=kv_heads, max_position_embeddings=256)
    return Qwen2ForCausalLM(cfg).eval()


def test_fused_decode_through_hf_model_matches_unpatched():
    """Prefill with the model's own attention, then 3 decode steps: the patched model over a
    container of a torch fake engine gives the unpatched model's logits and tokens."""
    from transformers.cache_utils import DynamicCache

    m = _tiny_qwen2()
    ids = torch.randint(0, 97, (2, 9), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        out = m(input_ids=ids, use_cache=True)
        eng = TorchAttnEngine(2)
        for i, (k, v, *_) in enumerate(out.past_key_values):
            eng.append(i, k, v)
        ref_cache = out.past_key_values
        tok_ref = tok = out.logits[:, -1].argmax(-1, keepdim=True)
        P.apply_int8_fused_patch(m)
        try:
            for step in range(3):
                with warnings.catch_warnings():
                    warnings.simplefilter("error")
                    got = m(input_ids=tok, past_key_values=P.INT8CacheWrapperContainer(eng, 2),
                            use_cache=True).logits
                P.remove_int8_fused_patch(m)
                ref = m(input_ids=tok_ref, past_key_values=ref_cache, use_cache=True)
                P.apply_int8_fused_patch(m)
                ref_cache = ref.past_key_values
                assert isinstance(ref_cache, DynamicCache)
                assert torch.allclose(got, ref.logits, atol=1e-3, rtol=0), step
                assert len(eng.calls) == 2 * (step + 1)
                tok = got[:, -1].argmax(-1, keepdim=True)
                tok_ref = ref.logits[:, -1].argmax(-1, keepdim=True)
                assert torch.equal(tok, tok_ref)
            assert eng.get_seq_len() == 9 + 3
        finally:
            P.remove_int8_fused_patch(m)


def test_fused_forward_applies_inv_tau_and_validates_it():
    """fp16 queries hand inv_tau[layer] to the engine (the kernel applies fp16(q * tau));
    other dtypes are scaled in their own dtype first (src/engine/patch_model.py:711-746),
    then cast to fp16 for the kernel."""
    m = _tiny_qwen2()
    attn = m.model.layers[1].self_attn
    hidden = torch.randn(1, 1, 256)
    pos = torch.tensor([[4]])
    cos, sin = m.model.rotary_emb(hidden, pos)
    tau = torch.rand(2, 4) + 0.5
    P.apply_int8_fused_patch(m)
    try:
        eng = TorchAttnEngine(2, inv_tau=tau)
        for i in range(2):
            eng.append(i, torch.randn(1, 2, 4, 64), torch.randn(1, 2, 4, 64))
        with torch.no_grad():
            attn(hidden, position_embeddings=(cos, sin), attention_mask=None,
                 past_key_values=P.INT8CacheWrapperContainer(eng, 2))
            q = attn.q_proj(hidden).view(1, 1, 4, 64).transpose(1, 2)
            q, _ = P._apply_rope(q, q, cos, sin)
        layer, q_seen, tau_seen = eng.calls[-1]
        assert layer == 1 and tau_seen is None and q_seen.dtype == torch.float16
        assert torch.equal(q_seen, (q[:, :, 0] * tau[1].view(1, -1, 1)).half())
        bad = TorchAttnEngine(2, inv_tau=torch.rand(2, 2))          # per-kv-head table
        for i in range(2):
            bad.append(i, torch.randn(1, 2, 4, 64), torch.randn(1, 2, 4, 64))
        with pytest.raises(ValueError, match="q_heads"):
            with torch.no_grad():
                attn(hidden, position_embeddings=(cos, sin), attention_mask=None,
                     past_key_values=P.INT8CacheWrapperContainer(bad, 2))
        short = TorchAttnEngine(2, inv_tau=torch.rand(1, 4))        # fewer layers than the model
        for i in range(2):
            short.append(i, torch.randn(1, 2, 4, 64), torch.randn(1, 2, 4, 64))
        with pytest.raises(ValueError, match="layers"):
            with torch.no_grad():
                attn(hidden, position_embeddings=(cos, sin), attention_mask=None,
                     past_key_values=P.INT8CacheWrapperContainer(short, 2))
    finally:
        P.remove_int8_fused_patch(m)


def test_fused_forward_hands_fp16_tau_to_the_engine():
    m = _tiny_qwen2(num_layers=1).half()
    attn = m.model.layers[0].self_attn
    hidden = torch.randn(1, 1, 256).half()
    cos, sin = m.model.rotary_emb(hidden, torch.tensor([[3]]))
    tau = torch.rand(1, 4) + 0.5
    eng = TorchAttnEngine(1, inv_tau=tau)
    eng.append(0, torch.randn(1, 2, 3, 64).half(), torch.randn(1, 2, 3, 64).half())
    with torch.no_grad():
        P._fused_forward_impl(attn, hidden, P.INT8CacheWrapper(eng, 0), position_embeddings=(cos, sin))
    _, q_seen, tau_seen = eng.calls[-1]
    assert q_seen.dtype == torch.float16 and torch.equal(tau_seen, tau[0].half())


def test_fused_forward_rejects_unknown_impl_with_eng042_warning():
    m = _tiny_qwen2(num_layers=1)
    attn = m.model.layers[0].self_attn
    hidden = torch.randn(1, 1, 256)
    cos, sin = m.model.rotary_emb(hidden, torch.tensor([[0]]))
    eng = TorchAttnEngine(1)
    eng.append(0, torch.randn(1, 2, 1, 64), torch.randn(1, 2, 1, 64))
    eng.decode_attn_impl = "no_such_kernel"
    wrapper = P.INT8CacheWrapper(eng, 0)
    with warnings.catch_warnings(record=True) as rec, pytest.raises(ValueError, match="decode_attn_impl"):
        warnings.simplefilter("always")
        with torch.no_grad():
            P._fused_forward_impl(attn, hidden, wrapper, position_embeddings=(cos, sin))
    assert any("ENG-042" in str(r.message) for r in rec)
    with pytest.raises(ValueError, match="q_len"):
        P._fused_forward_impl(attn, torch.randn(1, 2, 256), wrapper, position_embeddings=(cos, sin))


class Int8TorchEngine:
    """Per-token group-32 INT8 codes with fp16 scales, quantized by the oracle's restatement
    of src/quant/int8_basic.py; only ``append`` and ``get_int8_tensors`` are used."""

    decode_attn_impl = "torch_ref"
    inv_tau = None

    def __init__(self, num_layers):
        self.num_layers = num_layers
        self.codes = [None] * num_layers
        self.scales = [None] * num_layers

    def get_seq_len(self):
        return 0 if self.codes[0] is None else int(self.codes[0][0].shape[2])

    def append(self, i, k, v):
        from oracle.quant import quantize_symmetric_int8

        new = [quantize_symmetric_int8(x.half(), 100.0, 32) for x in (k, v)]
        if self.codes[i] is None:
            self.codes[i] = [n[0] for n in new]
            self.scales[i] = [n[1] for n in new]
        else:
            self.codes[i] = [torch.cat([a, n[0]], 2) for a, n in zip(self.codes[i], new)]
            self.scales[i] = [torch.cat([a, n[1]], 2) for a, n in zip(self.scales[i], new)]

    def get_int8_tensors(self, i):
        return self.codes[i][0], self.codes[i][1], self.scales[i][0], self.scales[i][1]


def test_torch_ref_impl_through_the_hook_matches_dequantized_attention():
    m = _tiny_qwen2(num_layers=1)
    attn = m.model.layers[0].self_attn
    eng = Int8TorchEngine(1)
    eng.append(0, torch.randn(1, 2, 6, 64), torch.randn(1, 2, 6, 64))
    hidden = torch.randn(1, 1, 256)
    cos, sin = m.model.rotary_emb(hidden, torch.tensor([[6]]))
    with torch.no_grad():
        out, _ = P._fused_forward_impl(attn, hidden, P.INT8CacheWrapper(eng, 0), position_embeddings=(cos, sin))
        q = attn.q_proj(hidden).view(1, 1, 4, 64).transpose(1, 2)
        k = attn.k_proj(hidden).view(1, 1, 2, 64).transpose(1, 2)
        q, _ = P._apply_rope(q, k, cos, sin)
        kc, vc, ks, vs = eng.get_int8_tensors(0)
        assert kc.shape[2] == 7
        kd = (kc.float().view(1, 2, 7, 2, 32) * ks.float()[..., None]).view(1, 2, 7, 64).repeat_interleave(2, 1)
        vd = (vc.float().view(1, 2, 7, 2, 32) * vs.float()[..., None]).view(1, 2, 7, 64).repeat_interleave(2, 1)
        p = torch.softmax(torch.einsum("bhd,bhsd->bhs", q[:, :, 0].float(), kd) / 8.0, -1)
        want = attn.o_proj(torch.einsum("bhs,bhsd->bhd", p, vd).reshape(1, 1, 256))
    assert torch.allclose(out, want, atol=1e-3)


def test_proxy_signature_accepts_transformers_keywords():
    """The proxy takes what transformers 5.x passes its attention layers by keyword."""
    m = _tiny_qwen2(num_layers=1)
    P.apply_int8_fused_patch(m)
    try:
        params = inspect.signature(type(m.model.layers[0].self_attn).forward).parameters
        for name in ("hidden_states", "attention_mask", "past_key_values", "past_key_value"):
            assert name in params
    finally:
        P.remove_int8_fused_patch(m)
