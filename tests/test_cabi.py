"""The C ABI (CPU only): libssa_hip.so loads, exports every function include/ssa_hip.h declares,
and the ctypes mirrors of the header's structs have the C layout (checked against gcc's).
No entry point launches anything: there is no GPU here (argument checks return first)."""

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
           "ssa_build_args_t": _lib.BuildArgs, "ssa_split_args_t": _lib.SplitArgs,
           "ssa_maint_args_t": _lib.MaintArgs}


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


def test_glue_entry_points_refuse_bad_arguments_before_any_launch():
    """Null pointers, empty or oversized batches and a missing work buffer are refused on the host
    (a nonzero return before any HIP call), so nothing here needs a GPU."""
    h = _lib_handle()
    fake = 1 << 20                                       # never dereferenced: every call returns early
    assert h.ssa_linear_swiglu(None, fake, fake, 2, 64, 64, 1, None) != 0
    assert h.ssa_linear_swiglu(fake, fake, fake, 9, 64, 64, 1, None) != 0      # batch above 8
    assert h.ssa_linear_swiglu(fake, fake, fake, 2, 64, 60, 1, None) != 0      # K not a multiple of 8
    assert h.ssa_linear_swiglu(fake, fake, fake, 2, 64, 64, 0, None) != 0      # fp32 weights
    assert h.ssa_linear_skinny(fake, fake, fake, 0, 64, 64, 1, None) != 0
    assert h.ssa_linear_skinny_res(fake, fake, fake, 9, 64, 64, 1, None) != 0          # batch above 8
    assert h.ssa_rmsnorm_linear_skinny(fake, None, 1e-6, fake, fake, 2, 64, 64, 1, None) != 0   # no norm weight
    assert h.ssa_rmsnorm_linear_skinny(fake, fake + 8, 1e-6, fake, fake, 2, 64, 64, 1, None) != 0  # misaligned
    assert h.ssa_rmsnorm_linear_swiglu(fake, fake, 1e-6, fake, fake, 2, 64, 60, 1, None) != 0   # K not a multiple of 8
    assert h.ssa_argmax_rows(fake, fake, 2, 100, 1, None, None) != 0           # no work buffer
    assert h.ssa_argmax_rows(fake, fake, 0, 100, 1, fake, None) != 0
    assert h.ssa_embed_rmsnorm(None, fake, fake, fake, fake, 2, 64, 10, 1e-6, fake, fake, 1, None) != 0
    assert h.ssa_embed_rmsnorm(fake, fake, fake, fake, fake, 2, 64, 10, 1e-6, None, fake, 1, None) != 0


def test_attention_refuses_misaligned_rows_before_any_launch():
    """q, K, V and the split accumulators are read as 16-byte vectors: a 4-byte-aligned part_a
    (or row stride) is refused with hipErrorInvalidValue (1) before anything is launched."""
    h = _lib_handle()
    base = 1 << 20                                       # 16-byte aligned; never dereferenced

    def args(**kw):
        a = _lib.AttnArgs()
        a.q, a.s_qh, a.q_dtype = base, 128, 1
        a.k, a.s_kh, a.s_kn = base, 128 * 64, 128
        a.v, a.s_vh, a.s_vn = base, 128 * 64, 128
        a.kv_dtype = 1
        a.part_m, a.part_l, a.part_a, a.part_cnt, a.counter = base, base, base, base, base
        a.out, a.s_oh, a.out_dtype = base, 128, 1
        a.n_heads, a.G, a.d, a.S, a.n_host = 2, 2, 128, 4, 64
        a.labels, a.s_lh, a.w, a.s_wr, a.w_len = base, 64, base, 17, 17
        for k, v in kw.items():
            setattr(a, k, v)
        return a

    for bad in (dict(part_a=base + 4), dict(q=base + 2), dict(k=base + 8), dict(s_kn=124), dict(s_qh=36),
                dict(part_a=None), dict(counter=None)):
        a = args(**bad)
        assert h.ssa_label_attention(ct.byref(a), None) == 1, bad
        assert h.ssa_dense_attention(ct.byref(a), None) == 1, bad


def test_noalloc_step_refuses_a_workspace_beyond_its_array_before_any_call():
    """ssa_sparse_step_noalloc checks the split workspace against SSA_NOALLOC_SCRATCH_BYTES (4 MiB)
    first: an oversized one returns hipErrorInvalidValue (1) before any HIP call."""
    h = _lib_handle()
    text = HEADER.read_text()
    assert re.search(r"#define SSA_NOALLOC_SCRATCH_BYTES \(4u << 20\)", text)
    a = _lib.AttnArgs()
    a.n_heads, a.G, a.d, a.S = 64, 8, 256, 32            # 64 * 32 * 8 * 256 * 4 B = 16 MiB of partials
    assert h.ssa_sparse_step_noalloc(None, None, ct.byref(a), None, None) == 1
    a.n_heads, a.G, a.d, a.S = 8, 2, 128, 300            # more splits than a head takes
    assert h.ssa_sparse_step_noalloc(None, None, ct.byref(a), None, None) == 1
