"""The committed golden fixtures (tests/golden/*.npz) against the CPU oracle.

The fixtures were written by tests/golden/make_golden.py.  These tests check that the
oracle still reproduces them exactly (codes bit for bit, attention within one fp16
rounding), and check properties of the stored data that do not depend on the oracle's
formulas: every code dequantises to within half a quantisation step of its input
(unless clipped), outlier channels are stored verbatim, and context lengths bound
the attention.
"""
import glob
import math
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden as MG  # noqa: E402

FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: torch.from_numpy(z[k].copy()) for k in z.files}


def test_every_case_has_a_fixture():
    names = {os.path.basename(p)[:-4] for p in FIXTURES}
    assert names == set(MG.CASES)


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_fixture(path):
    torch.set_num_threads(1)
    name = os.path.basename(path)[:-4]
    want = load(path)
    got = MG.make(name)
    assert set(got) == set(want)
    for key, w in want.items():
        g = got[key]
        if key == "out":
            assert g.dtype == torch.float16
            torch.testing.assert_close(g.float(), w.float(), rtol=1e-3, atol=1e-3)
        else:
            assert torch.equal(g.reshape(w.shape).view(w.dtype) if g.dtype != w.dtype else g, w), key


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_fixture_codes_round_trip_within_half_step(path):
    f = load(path)
    for side in ("k", "v"):
        x = f[side].float()
        codes = f[f"{side}_codes"]
        B, H, S, D = x.shape
        if codes.shape[-1] == D // 2:  # packed nibbles, high nibble = even channel
            u = codes.to(torch.int16)
            c = torch.stack([(u >> 4) & 15, u & 15], dim=-1).view(B, H, S, D) - 8
        else:
            c = codes.view(torch.int8).to(torch.int16)
        if f"{side}_zp" in f:  # asymmetric static g32: x ~ s*c + z
            s = f[f"{side}_static"].float()[None, :, None, :, None]
            z = f[f"{side}_zp"].float()[None, :, None, :, None]
            lo, hi = -8, 7
        else:  # symmetric: per-token scale
            s = f[f"{side}_scale_tok"].float()[..., None]
            z = torch.zeros(())
            lo, hi = (-127, 127) if codes.shape[-1] == D else (-7, 7)
        xg = x.view(B, H, S, -1, 32 if s.shape[-2] == 4 else D // s.shape[-2])
        cg = c.view(xg.shape).float()
        err = (cg * s + z - xg).abs()
        inside = (cg > lo) & (cg < hi)
        assert inside.float().mean() > 0.95
        # INT8 rounds the quotient to fp16 first: up to half an fp16 ulp (2^-5 below 128)
        half = 0.5 + (2.0 ** -5 if codes.shape[-1] == D and "%s_zp" % side not in f else 0.0)
        assert torch.all(err[inside] <= half * s.expand_as(err)[inside] * (1 + 2e-3) + 1e-6), side
    if "k_outlier_idx" in f:
        oi, ov, k = f["k_outlier_idx"].long(), f["k_outlier_val"], f["k"]
        for h in range(oi.shape[0]):
            assert torch.equal(ov[:, h], k[:, h][..., oi[h]])


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_fixture_context_lengths_bound_the_attention(path):
    """Changing K/V beyond a row's context must not change that row's expected output."""
    name = os.path.basename(path)[:-4]
    f = load(path)
    cl = f["context_lens"]
    if int(cl.min()) == f["k"].shape[2]:
        pytest.skip("no row with a short context")
    ci, B, S, ctx = MG.CASES[name]
    assert list(cl.tolist()) == ctx and f["out"].shape[0] == B
    assert torch.isfinite(f["out"].float()).all()
    assert f["out"].abs().max() < 10 and f["out"].abs().max() > 0
    assert math.isclose(float(f["sm_scale"]), 1 / math.sqrt(128), rel_tol=1e-6)
