"""Writes tests/golden/calib_qwen25_1p5b_int8.json and _int4.json: the calibration tables
the reference ships for Qwen2.5-1.5B (artifacts/kv_calib_mse_1p5b_int8.json and
artifacts/kv_calib_mse_1p5b_int4.json under the reference checkout), reduced to the keys
its calibration loader reads (src/engine/generate_loop.py:769-849).  The search log under
"selection" is dropped; every table value is kept exactly as stored.

    python tests/golden/make_calib_fixture.py [/root/reference]

The reference checkout is read only by this script; the tests read the fixtures.
"""
from __future__ import annotations

import json
import os
import sys

KEEP = ("version", "model_id", "quant_bits", "qmax", "num_layers", "num_heads", "num_kv_heads",
        "head_dim", "clip_percentile_k", "clip_percentile_v", "group_size_k", "group_size_v",
        "k_scale", "v_scale", "inv_tau", "int4_outlier_ratio", "int4_mixed_rescue")


def main(ref_root: str) -> None:
    here = os.path.dirname(os.path.abspath(__file__))
    for bits in (8, 4):
        src = os.path.join(ref_root, "artifacts", f"kv_calib_mse_1p5b_int{bits}.json")
        with open(src, encoding="utf-8") as f:
            data = json.load(f)
        out = {k: data[k] for k in KEEP if k in data}
        dst = os.path.join(here, f"calib_qwen25_1p5b_int{bits}.json")
        with open(dst, "w", encoding="utf-8") as f:
            json.dump(out, f, separators=(",", ":"))
            f.write("\n")
        print(f"wrote {dst} ({os.path.getsize(dst)} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
