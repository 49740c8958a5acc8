"""CPU checks of the C-ABI boundary: libkvq.so loads, exports every function
include/kvq.h declares, and the ctypes mirrors of the structs have the C layout
(checked against offsetof/sizeof from a gcc-compiled probe).  No kernel runs here."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvq.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int32_t|int64_t|const char\*)\s+(kvq_\w+)\(", text, re.M)))


def test_header_declares_entry_points():
    assert declared_functions() == sorted([
        "kvq_abi_version", "kvq_append_decode_attn", "kvq_decode_attn", "kvq_decode_attn_noalloc",
        "kvq_decode_chunk_tokens",
        "kvq_append_scratch_bytes", "kvq_decode_workspace_bytes", "kvq_last_error",
        "kvq_quant_append", "kvq_stream_read"])


def test_library_loads_and_exports_all_symbols():
    from llm_kvcache_quantization_amd import _capi as C

    if not C.LIB_PATH.exists():
        pytest.skip("libkvq.so not built (run __graft_entry__.build())")
    L = C.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    assert set(C.EXPORTED_SYMBOLS) == set(declared_functions())
    assert L.kvq_abi_version() == C.ABI_VERSION
    assert L.kvq_last_error() == b""


def _probe(tmp_path, structs):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "kvq.h"', "int main(void){"]
    for sname, fields in structs.items():
        lines.append(f'printf("{sname} size %zu\\n", sizeof({sname}));')
        for f in fields:
            lines.append(f'printf("{sname} {f} %zu\\n", offsetof({sname}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    res = {}
    for line in out.splitlines():
        s, f, v = line.split()
        res[(s, f)] = int(v)
    return res


def test_ctypes_struct_layout_matches_c(tmp_path):
    import ctypes

    from llm_kvcache_quantization_amd import _capi as C

    pairs = {"kvq_kv_view": C.KvView, "kvq_decode_params": C.DecodeParams,
             "kvq_append_params": C.AppendParams}
    structs = {s: [f for f, _ in cls._fields_] for s, cls in pairs.items()}
    res = _probe(tmp_path, structs)
    for s, cls in pairs.items():
        assert res[(s, "size")] == ctypes.sizeof(cls), s
        for f, _ in cls._fields_:
            assert res[(s, f)] == getattr(cls, f).offset, (s, f)
