"""Static-table production (calib.compute_absmax_per_group, collect_absmax_samples,
scales_from_absmax_samples, calibration_json) against the reference's own known answers
(tests/test_calibrate_behavior.py:125-146, 387-425) and a closed form of the percentile:
per (kv head, group), the order statistics of the sample maxima at floor / ceil of
fp32(p / 100) * (n - 1), torch.quantile's fused lerp between them in exact rational
arithmetic, then the 1e-5 clamp and the division by qmax
(scripts/calibrate_behavior.py:228-259, 764-811).  CPU only."""
import json

import numpy as np
import pytest
import torch

from llm_kvcache_quantization_amd import calib
from test_oracle_pinning import quantile32


def test_absmax_per_group_reference_known_answers():
    t = torch.tensor([[[1.0, -2.0, 3.0, -4.0]]])
    r = calib.compute_absmax_per_group(t, 2)
    assert r.tolist() == [[2.0, 4.0]]
    assert calib.compute_absmax_per_group(torch.randn(4, 8, 128), 64).shape == (4, 2)
    for bad in (0, -1, 48):
        with pytest.raises(ValueError, match="divisible"):
            calib.compute_absmax_per_group(torch.randn(2, 3, 128), bad)


def test_absmax_is_over_the_sequence_and_the_group():
    # one large value per (head, group) at a different token each: the maximum is taken
    # over tokens and channels of the group, never across heads or groups
    t = torch.zeros(3, 5, 128)
    for h in range(3):
        for g in range(4):
            t[h, (h + g) % 5, 32 * g + (7 * g + h) % 32] = -(10.0 * h + g + 1)
    r = calib.compute_absmax_per_group(t, 32)
    assert r.tolist() == [[10.0 * h + g + 1 for g in range(4)] for h in range(3)]


def test_collect_absmax_samples_structure():
    g = torch.Generator().manual_seed(0)
    kv = [[torch.randn(2, 8, 64, generator=g) for _ in range(2)] for _ in range(3)]
    out = calib.collect_absmax_samples(kv, 32)
    assert len(out) == 2 and len(out[0]) == 3 and out[0][0].shape == (2, 2)
    assert torch.equal(out[1][2], calib.compute_absmax_per_group(kv[2][1], 32))
    assert calib.collect_absmax_samples([], 64) == []


@pytest.mark.parametrize("p,n,qmax", [(99.9, 7, 127), (99.5, 64, 127), (99.0, 33, 7),
                                      (100.0, 5, 127), (50.0, 10, 7), (99.9, 1, 127)])
def test_scales_from_absmax_samples_closed_form(p, n, qmax):
    g = torch.Generator().manual_seed(int(p * 10) + n)
    layers = 2
    samples = [[(torch.randn(3, 4, generator=g).abs() * torch.rand(1, generator=g) * 9)
                for _ in range(n)] for _ in range(layers)]
    samples[1][0][0, 0] = 0.0
    for s in samples[1]:
        s[2, 3] = 0.0  # an all-zero (head, group): the 1e-5 clamp comes before / qmax
    scales = calib.scales_from_absmax_samples(samples, p, qmax)
    assert len(scales) == layers
    for layer in range(layers):
        st = np.stack([s.numpy() for s in samples[layer]]).astype(np.float32)
        for h in range(3):
            for gi in range(4):
                q, _, _ = quantile32(st[:, h, gi], np.float32(p / 100.0))
                want = np.float32(max(q, np.float32(1e-5))) / np.float32(qmax)
                assert scales[layer][h, gi].item() == float(want), (layer, h, gi)
    assert scales[1][2, 3].item() == float(np.float32(1e-5) / np.float32(qmax))
    if p == 100.0:
        st = torch.stack(samples[0])
        assert torch.equal(scales[0], st.amax(dim=0).clamp(min=1e-5) / qmax)


def test_scales_take_the_quantile_over_samples_not_heads():
    # samples differ per head: a quantile over the wrong axis gives other scales
    samples = [[torch.tensor([[1.0, 2.0], [100.0, 200.0]]) * (k + 1) for k in range(9)]]
    s = calib.scales_from_absmax_samples(samples, 50.0, 1)[0]
    assert s.tolist() == [[5.0, 10.0], [500.0, 1000.0]]


def test_scales_from_empty_layer_raises():
    with pytest.raises(ValueError, match="empty"):
        calib.scales_from_absmax_samples([[torch.ones(1, 1)], []], 99.9, 127)


def test_calibration_json_round_trip(tmp_path):
    g = torch.Generator().manual_seed(3)
    kv = [[torch.randn(2, 16, 128, generator=g) * (1 + layer) for layer in range(3)]
          for _ in range(4)]
    ab = calib.collect_absmax_samples(kv, 16)
    ks = calib.scales_from_absmax_samples(ab, 99.5, 127)
    vs = calib.scales_from_absmax_samples(ab, 99.9, 127)
    tau = torch.linspace(0.8, 1.2, 3 * 12).reshape(3, 12)
    d = calib.calibration_json(ks, vs, group_size=16, clip_percentile_k=99.5,
                               clip_percentile_v=99.9, inv_tau=tau)
    path = tmp_path / "calib.json"
    path.write_text(json.dumps(d))
    t = calib.load_calibration_json(str(path), quant_bits=8)
    assert t.group_size == 16 and t.k_scale.dtype == torch.float16
    assert torch.equal(t.k_scale, torch.stack(ks).to(torch.float16))
    assert torch.equal(t.v_scale, torch.stack(vs).to(torch.float16))
    assert torch.allclose(t.inv_tau, tau)
    d4 = calib.calibration_json(ks, vs, group_size=16, clip_percentile_k=99.5, quant_bits=4,
                                outlier_ratio=0.01)
    path.write_text(json.dumps(d4))
    t4 = calib.load_calibration_json(str(path), quant_bits=4)
    assert t4.k_scale.dtype == torch.float32 and torch.equal(t4.k_scale, torch.stack(ks))
    assert t4.outlier_ratio == 0.01 and t4.inv_tau is None
