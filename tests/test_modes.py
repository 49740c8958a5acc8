"""CPU tests of the kv_mode switch (llm_kvcache_quantization_amd/modes.py): the
calibration-JSON rules of src/engine/generate_loop.py:751-889, the engine of each mode
(generate_loop.py:891-938), the argument checks of generate_from_ids and the
prefill-to-decode K / V hand-off rules (generate_loop.py:1368-1440)."""
import json
import warnings

import pytest
import torch

from llm_kvcache_quantization_amd import modes as M
from llm_kvcache_quantization_amd.cache import FP16KVCache, INT4KVCache, INT8KVCache, KIVIStyleKVCache


def _write(tmp_path, name, data):
    p = tmp_path / name
    p.write_text(json.dumps(data))
    return str(p)


def _table(L=2, H=2, G=4, val=0.05):
    return [[[val] * G for _ in range(H)] for _ in range(L)]


def test_load_calibration_v2_tables_and_dtypes(tmp_path):
    data = dict(version=2, group_size_k=16, group_size_v=16, clip_percentile_k=99.5,
                clip_percentile_v=99.5, k_scale=_table(), v_scale=_table(val=0.07),
                inv_tau=[[1.0, 1.1, 0.9, 1.2]] * 2, int4_outlier_ratio=0.01)
    path = _write(tmp_path, "c.json", data)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        c8 = M.load_calibration("int8_ours", path)
        c4 = M.load_calibration("int4_ours", path)
    assert c8.static_k_scale.dtype == torch.float16 and c4.static_k_scale.dtype == torch.float32
    assert c8.static_v_scale.shape == (2, 2, 4) and c8.inv_tau.dtype == torch.float32
    assert c8.group_size == 16 and c8.clip_percentile == 99.5
    assert c4.outlier_rescue_ratio == 0.01 and c4.mixed_rescue is False
    assert M.load_calibration("int4_ours_mixed", path).mixed_rescue is True
    # tables are read only by the calibrated modes
    base = M.load_calibration("int8_baseline", path, group_size=64)
    assert base.static_k_scale is None and base.group_size == 64


def test_load_calibration_switches(tmp_path):
    path = _write(tmp_path, "c.json", dict(version=2, k_scale=_table(), v_scale=_table(), inv_tau=[[1.0] * 4] * 2))
    c = M.load_calibration("int8_ours", path, use_static_scales=False, use_attn_temperature=False)
    assert c.static_k_scale is None and c.static_v_scale is None and c.inv_tau is None
    legacy = _write(tmp_path, "g.json", dict(version=2, group_size=32, clip_percentile=99.0))
    c = M.load_calibration("int8_ours", legacy, group_size=128, clip_percentile=99.9)
    assert c.group_size == 32 and c.clip_percentile == 99.0


def test_load_calibration_warnings(tmp_path):
    cases = [
        (dict(version=1, k_scale=_table(), v_scale=_table()), "version=1"),
        (dict(version=2, group_size_k=16, group_size_v=32), "CAL-022"),
        (dict(version=2, clip_percentile_k=99.0, clip_percentile_v=99.9), "CAL-022"),
        (dict(version=2, k_scale=_table()), "'k_scale' but no 'v_scale'"),
        (dict(version=2, v_scale=_table()), "'v_scale' but no 'k_scale'"),
    ]
    for i, (data, needle) in enumerate(cases):
        path = _write(tmp_path, f"w{i}.json", data)
        with pytest.warns(UserWarning, match=needle):
            c = M.load_calibration("int8_ours", path)
        if "group_size_k" in data:
            assert c.group_size == 16


def test_load_calibration_missing_and_broken_files(tmp_path):
    missing = str(tmp_path / "nope.json")
    with pytest.raises(FileNotFoundError):
        M.load_calibration("int8_ours", missing)
    with pytest.raises(FileNotFoundError):
        M.load_calibration("int4_fused", "")
    with pytest.warns(UserWarning, match="not found"):
        c = M.load_calibration("int8_ours", missing, allow_missing_calib=True)
    assert c.static_k_scale is None and c.inv_tau is None
    broken = tmp_path / "broken.json"
    broken.write_text("{not json")
    with pytest.raises(RuntimeError, match="Failed to load"):
        M.load_calibration("int8_ours", str(broken))
    with pytest.warns(UserWarning, match="equivalent to baseline"):
        c = M.load_calibration("int8_ours", str(broken), allow_missing_calib=True, group_size=64)
    assert c.static_k_scale is None and c.group_size == 64


def test_shipped_calibration_fixture_loads():
    """The trimmed Qwen2.5-1.5B tables under tests/golden load as the reference loads them."""
    import os

    here = os.path.join(os.path.dirname(__file__), "golden")
    with pytest.warns(UserWarning, match="version=1"):
        c8 = M.load_calibration("int8_ours", os.path.join(here, "calib_qwen25_1p5b_int8.json"))
    with pytest.warns(UserWarning, match="version=1"):
        c4 = M.load_calibration("int4_fused", os.path.join(here, "calib_qwen25_1p5b_int4.json"))
    assert c8.static_k_scale.dtype == torch.float16 and c8.static_k_scale.shape[0] == 28
    assert c4.static_k_scale.dtype == torch.float32 and c4.group_size == 16
    assert c4.outlier_rescue_ratio == pytest.approx(0.01)


def test_create_kv_cache_engine_per_mode():
    expect = {"fp16": FP16KVCache, "int8_baseline": INT8KVCache, "int8_fused": INT8KVCache,
              "int8_ours": INT8KVCache, "int4_baseline": INT4KVCache, "int4_fused": INT4KVCache,
              "int4_ours": INT4KVCache, "int4_ours_mixed": INT4KVCache}
    for mode, cls in expect.items():
        assert type(M.create_kv_cache(mode, 2, device="cpu")) is cls, mode
    cal = M.Calibration(group_size=16, clip_percentile=99.0, outlier_rescue_ratio=0.02, mixed_rescue=True)
    e = M.create_kv_cache("int4_ours_mixed", 2, device="cpu", calib=cal)
    assert e.group_size == 16 and e.outlier_rescue_ratio == 0.02 and e.mixed_rescue is True
    assert type(M.create_kv_cache("kivi_style", 2, device="cpu", quant_bits=4)) is KIVIStyleKVCache


def test_unknown_mode_raises():
    with pytest.raises(ValueError):
        M.check_kv_mode("int3_magic")


def test_append_delta_rules():
    """The three hand-off cases and the two warnings of generate_loop.py:1368-1440."""
    eng = FP16KVCache(num_layers=4, device="cpu")
    for i in range(4):
        eng.append(i, torch.zeros(1, 1, 5, 4), torch.zeros(1, 1, 5, 4))
    prev = [5, 5, 5, 5]
    only_new = torch.ones(1, 1, 1, 4)
    whole = torch.cat([torch.zeros(1, 1, 5, 4), 2 * torch.ones(1, 1, 1, 4)], 2)
    odd = torch.cat([torch.zeros(1, 1, 5, 4), 3 * torch.ones(1, 1, 2, 4)], 2)
    stale = torch.zeros(1, 1, 5, 4)
    with pytest.warns(RuntimeWarning) as rec:
        M._append_delta(eng, [(only_new, only_new), (whole, whole), (odd, odd), (stale, stale)], prev, 1)
    msgs = [str(r.message) for r in rec]
    assert any("ENG-045A" in m for m in msgs) and any("ENG-045B" in m for m in msgs)
    k = [eng.get_kv(i)[0] for i in range(4)]
    assert k[0].shape[2] == 6 and float(k[0][0, 0, -1, 0]) == 1.0
    assert k[1].shape[2] == 6 and float(k[1][0, 0, -1, 0]) == 2.0
    assert k[2].shape[2] == 7 and float(k[2][0, 0, -1, 0]) == 3.0
    assert k[3].shape[2] == 5


def test_generate_argument_checks():
    class Stub:
        device = torch.device("cpu")

    with pytest.raises(ValueError, match="decode_attn_impl"):
        M.generate_from_ids(Stub(), None, torch.zeros(1, 3, dtype=torch.long), decode_attn_impl="nope")
    with pytest.raises(ValueError, match="kv_mode"):
        M.generate_from_ids(Stub(), None, torch.zeros(1, 3, dtype=torch.long), kv_mode="int4_kivi")
    with pytest.raises(ValueError, match="policy_json"):
        M.generate_from_ids(Stub(), None, torch.zeros(1, 3, dtype=torch.long), kv_mode="int4_ours_asym_alloc")


def test_every_reference_kv_mode_is_accepted():
    """src/engine/generate_loop.py:438-460: the fourteen kv_modes."""
    ref = ["fp16", "int8_baseline", "int8_fused", "int8_ours", "int4_baseline", "int4_fused", "int4_ours",
           "int4_ours_mixed", "kivi_style", "int4_kivi_aligned", "int4_mixed_kv", "int4_ours_asym",
           "int4_ours_asym_ba", "int4_ours_asym_alloc"]
    assert sorted(M.KV_MODES) == sorted(ref)
    for m in ref:
        M.check_kv_mode(m)


def test_role_calibration_rules(tmp_path):
    """generate_loop.py:955-1131: the role_aware section, the k_calibration fallback (with its
    warning), v3 inv_tau for int4_kivi_aligned, inv_tau only for int4_ours_asym_ba, relative
    paths against the project root, a missing file."""
    import json

    ra = {"role_aware": {"k_percentile": 99.5, "v_percentile": 99.0, "inv_tau": [[1.0, 0.5]]},
          "k_calibration": {"inv_tau": [[2.0, 2.0]], "k_percentile": 98.0},
          "v_calibration": {"v_percentile": 97.0}}
    fb = {"k_calibration": {"k_percentile": 98.0, "inv_tau": [[2.0, 3.0]]}, "v_calibration": {"v_percentile": 97.0},
          "inv_tau": [[4.0, 4.0]]}
    (tmp_path / "ra.json").write_text(json.dumps(ra))
    (tmp_path / "fb.json").write_text(json.dumps(fb))
    r = M.load_role_calibration("int4_ours_asym", "ra.json", project_root=str(tmp_path))
    assert (r.k_percentile, r.v_percentile, r.inv_tau) == (99.5, 99.0, None)
    r = M.load_role_calibration("int4_ours_asym_ba", str(tmp_path / "ra.json"))
    assert r.inv_tau.tolist() == [[1.0, 0.5]]
    with pytest.warns(UserWarning, match="k_calibration fallback"):
        r = M.load_role_calibration("int4_ours_asym_ba", str(tmp_path / "fb.json"))
    assert (r.k_percentile, r.v_percentile) == (98.0, 97.0) and r.inv_tau.tolist() == [[2.0, 3.0]]
    with pytest.warns(UserWarning, match="Allocator RoleAlign"):
        r = M.load_role_calibration("int4_ours_asym_alloc", str(tmp_path / "fb.json"))
    assert r.inv_tau is None
    r = M.load_role_calibration("int4_kivi_aligned", str(tmp_path / "ra.json"))
    assert r.inv_tau.tolist() == [[2.0, 2.0]] and r.v_percentile == 97.0 and r.k_percentile == 100.0
    r = M.load_role_calibration("int4_kivi_aligned", str(tmp_path / "fb.json"))
    assert r.inv_tau.tolist() == [[2.0, 3.0]]
    assert M.load_role_calibration("kivi_style", str(tmp_path / "nope.json")).inv_tau is None
    with pytest.raises(FileNotFoundError):
        M.load_role_calibration("int4_ours_asym", "nope.json", project_root=str(tmp_path))


def test_policy_json_loader(tmp_path):
    """src/cache/role_aware_allocator_cache.py:36-70."""
    import json

    from llm_kvcache_quantization_amd import load_per_layer_bits_from_policy as load

    (tmp_path / "p.json").write_text(json.dumps({"per_layer_bits": [[4, 8], [16, 4]]}))
    assert load("p.json", project_root=str(tmp_path)) == [(4, 8), (16, 4)]
    (tmp_path / "bad.json").write_text(json.dumps({"per_layer_bits": [[4, 3]]}))
    with pytest.raises(ValueError, match="unsupported bits"):
        load(str(tmp_path / "bad.json"), project_root="/")
    (tmp_path / "nokey.json").write_text(json.dumps({}))
    with pytest.raises(ValueError, match="per_layer_bits"):
        load(str(tmp_path / "nokey.json"), project_root="/")
    with pytest.raises(FileNotFoundError):
        load("missing.json", project_root=str(tmp_path))


def test_past_layers_reads_dynamic_cache_and_tuples():
    from transformers.cache_utils import DynamicCache

    pairs = [(torch.randn(1, 2, 3, 4), torch.randn(1, 2, 3, 4)) for _ in range(2)]
    for src in (tuple(pairs), M._to_model_cache(pairs)):
        got = M._past_layers(src)
        assert len(got) == 2 and all(torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
                                     for a, b in zip(got, pairs))
    assert isinstance(M._to_model_cache(pairs), DynamicCache)
