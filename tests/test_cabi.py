"""The C ABI (CPU only): libssa_hip.so loads, exports every function include/ssa_hip.h declares,
and the ctypes mirrors of the header's structs have the C layout (checked against gcc's).
No entry point is called: there is no GPU here."""

from __future__ import annotations

import ctypes as ct
import re
import subprocess
from pathlib import Path

import pytest

from ssa_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ssa_hip.h"


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ssa_\w+)\s*\(", text, flags=re.M)))


def _lib_handle():
    if not _lib.LIB_PATH.exists():
        from ssa_amd.build import build
        build()
    return _lib.lib()


def test_header_declares_the_bound_entry_points():
    assert _declared_functions() == sorted(_lib.ENTRY_POINTS)


def test_library_loads_and_exports_every_declared_symbol():
    h = _lib_handle()
    for name in _declared_functions():
        assert getattr(h, name) is not None, name


STRUCTS = {"ssa_attn_args_t": _lib.AttnArgs, "ssa_index_state_t": _lib.IndexState,
           "ssa_insert_args_t": _lib.InsertArgs, "ssa_select_args_t": _lib.SelectArgs,
           "ssa_build_args_t": _lib.BuildArgs, "ssa_split_args_t": _lib.SplitArgs}


def test_struct_layouts_match_the_c_compiler(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "ssa_hip.h"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(line.split()[:2]): int(line.split()[2]) for line in out if line}
    for cname, py in STRUCTS.items():
        assert got[(cname, "size")] == ct.sizeof(py), cname
        for f, _ in py._fields_:
            assert got[(cname, f)] == getattr(py, f).offset, (cname, f)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()
