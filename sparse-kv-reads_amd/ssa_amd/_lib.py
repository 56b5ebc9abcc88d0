"""ctypes binding of ``libssa_hip.so`` (declared in ``include/ssa_hip.h``).

The library is the only compute path: if it is missing or cannot be loaded, every entry point
raises. Tensors cross the boundary as raw device pointers (``tensor.data_ptr()``) and element
strides; kernels are enqueued on torch's current stream, so they are captured by
``torch.cuda.graph`` like any other work on that stream.
"""

from __future__ import annotations

import ctypes as ct
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libssa_hip.so"

F32, BF16, F16 = 0, 1, 2
_DT = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

i32, i64, f32, f64, vp = ct.c_int32, ct.c_int64, ct.c_float, ct.c_double, ct.c_void_p


class AttnArgs(ct.Structure):
    _fields_ = [("q", vp), ("s_qh", i64), ("q_dtype", i32),
                ("k", vp), ("s_kh", i64), ("s_kn", i64),
                ("v", vp), ("s_vh", i64), ("s_vn", i64),
                ("kv_dtype", i32),
                ("labels", vp), ("s_lh", i64),
                ("w", vp), ("s_wr", i64), ("w_len", i32), ("per_head", i32),
                ("n_dev", vp), ("n_host", i32),
                ("part_m", vp), ("part_l", vp), ("part_a", vp), ("part_cnt", vp),
                ("counter", vp),
                ("out", vp), ("s_oh", i64), ("out_dtype", i32),
                ("cnt_out", vp),
                ("n_heads", i32), ("G", i32), ("d", i32), ("S", i32), ("chunk_align", i32)]


class IndexState(ct.Structure):
    _fields_ = [("n_heads", i32), ("heads_per_layer", i32), ("C", i32), ("d", i32), ("capacity", i32),
                ("ms", i32), ("summary_bits", i32), ("shared_dirs", i32),
                ("n_c", vp), ("sum_dir", vp), ("dir8", vp), ("cent", vp), ("cent8", vp),
                ("mmax", vp), ("mmin", vp), ("count", vp),
                ("ksum", vp), ("mu_ref", vp),
                ("rbar", vp), ("cap", vp), ("vthr", vp),
                ("flags", vp), ("end", vp), ("nsplit", vp),
                ("labels", vp),
                ("mem", vp), ("proj", vp), ("side", vp), ("smag", vp),
                ("stage", vp),
                ("knbuf", vp), ("kn_rows", i32)]

STAGE_WORDS = 80          # SSA_STAGE_WORDS


class InsertArgs(ct.Structure):
    _fields_ = [("k", vp), ("k_dtype", i32), ("s_kh", i64), ("s_kn", i64),
                ("koff", vp),
                ("n_dev", vp), ("n_host", i32),
                ("window", i32), ("delta", f32), ("capk", f32), ("reset_at", i32), ("var_min", i32)]


class SelectArgs(ct.Structure):
    _fields_ = [("q", vp), ("q_dtype", i32), ("s_qh", i64), ("G", i32),
                ("w", vp), ("s_wr", i64),
                ("budget", f64),
                ("group", i32),
                ("scale", f32),
                ("need_out", vp)]


class BuildArgs(ct.Structure):
    _fields_ = [("k", vp), ("k_dtype", i32), ("s_kh", i64), ("s_kn", i64),
                ("heads", vp), ("n_sel", i32),
                ("start", i32), ("end", i32),
                ("mu", vp),
                ("xn", vp), ("mag", vp),
                ("sq", vp),
                ("assign", vp),
                ("part", vp),
                ("part_cnt", vp),
                ("init_idx", vp),
                ("fit", i32),
                ("C_fit", i32), ("iters", i32)]


class SplitArgs(ct.Structure):
    _fields_ = [("k", vp), ("k_dtype", i32), ("s_kh", i64), ("s_kn", i64),
                ("heads", vp), ("n_sel", i32),
                ("start", i32), ("end", i32),
                ("split_factor", f32), ("cap_min", f32),
                ("nmeans", i32), ("iters", i32),
                ("mem", vp), ("side", vp), ("proj", vp), ("smag", vp),
                ("ms", i32),
                ("over", vp), ("done", vp),
                ("refresh_only", i32),
                ("parts", vp), ("max_parts", i32)]


class MaintArgs(ct.Structure):
    _fields_ = [("k", vp), ("k_dtype", i32), ("s_kh", i64), ("s_kn", i64),
                ("refit_all", i32), ("refit", i32),
                ("C_init", i32), ("iters", i32), ("seed", i32),
                ("split_factor", f32), ("cap_keys", f32),
                ("capk", f64),
                ("max_heads", i32),
                ("plan", vp), ("mu", vp),
                ("xn", vp), ("mag", vp), ("sq", vp), ("assign", vp),
                ("part", vp), ("part_cnt", vp),
                ("init_idx", vp),
                ("mem", vp), ("side", vp), ("proj", vp), ("smag", vp),
                ("parts", vp),
                ("over", vp)]


MAINT_PLAN_WORDS = 8      # SSA_MAINT_PLAN_WORDS


# (name, restype, argtypes) of every exported entry point; the C-ABI test checks this list
# against the header.
ENTRY_POINTS = {
    "ssa_error_string": (ct.c_char_p, [ct.c_int]),
    "ssa_label_attention": (ct.c_int, [ct.POINTER(AttnArgs), vp]),
    "ssa_dense_attention": (ct.c_int, [ct.POINTER(AttnArgs), vp]),
    "ssa_merge_splits": (ct.c_int, [vp, vp, vp, i64, i64, i64, i64, i64, ct.c_int, ct.c_int, ct.c_int, ct.c_int,
                                    vp, i64, ct.c_int, vp]),
    "ssa_compact_positions": (ct.c_int, [vp, i64, vp, i64, ct.c_int, ct.c_int, ct.c_int, vp, ct.c_int, ct.c_int,
                                         vp, vp, i64, vp, vp]),
    "ssa_insert": (ct.c_int, [ct.POINTER(IndexState), ct.POINTER(InsertArgs), vp]),
    "ssa_select": (ct.c_int, [ct.POINTER(IndexState), ct.POINTER(InsertArgs), ct.POINTER(SelectArgs), vp]),
    "ssa_build": (ct.c_int, [ct.POINTER(IndexState), ct.POINTER(BuildArgs), vp]),
    "ssa_split_fit": (ct.c_int, [ct.POINTER(IndexState), ct.POINTER(SplitArgs), vp]),
    "ssa_maintain": (ct.c_int, [ct.POINTER(IndexState), ct.POINTER(MaintArgs), vp]),
    "ssa_sparse_step": (ct.c_int, [ct.POINTER(IndexState), ct.POINTER(SelectArgs), ct.POINTER(AttnArgs),
                                   ct.POINTER(InsertArgs), vp]),
    "ssa_sparse_step_noalloc": (ct.c_int, [ct.POINTER(IndexState), ct.POINTER(SelectArgs), ct.POINTER(AttnArgs),
                                           ct.POINTER(InsertArgs), vp]),
    "ssa_rmsnorm_add": (ct.c_int, [vp, vp, vp, vp, ct.c_int32, ct.c_int32, ct.c_float, ct.c_int32, vp]),
    "ssa_qk_norm_rope_cache": (ct.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, ct.c_int32, ct.c_int32,
                                          ct.c_int32, ct.c_int32, ct.c_float, ct.c_int32, vp]),
    "ssa_silu_mul": (ct.c_int, [vp, vp, ct.c_int32, ct.c_int32, ct.c_int32, vp]),
    "ssa_linear_skinny": (ct.c_int, [vp, vp, vp, ct.c_int32, ct.c_int32, ct.c_int32, ct.c_int32, vp]),
    "ssa_argmax_rows": (ct.c_int, [vp, vp, ct.c_int32, ct.c_int32, ct.c_int32, vp, vp]),
    "ssa_linear_swiglu": (ct.c_int, [vp, vp, vp, ct.c_int32, ct.c_int32, ct.c_int32, ct.c_int32, vp]),
    "ssa_linear_skinny_res": (ct.c_int, [vp, vp, vp, ct.c_int32, ct.c_int32, ct.c_int32, ct.c_int32, vp]),
    "ssa_rmsnorm_linear_skinny": (ct.c_int, [vp, vp, ct.c_float, vp, vp, ct.c_int32, ct.c_int32, ct.c_int32,
                                             ct.c_int32, vp]),
    "ssa_rmsnorm_linear_swiglu": (ct.c_int, [vp, vp, ct.c_float, vp, vp, ct.c_int32, ct.c_int32, ct.c_int32,
                                             ct.c_int32, vp]),
    "ssa_embed_rmsnorm": (ct.c_int, [vp, vp, vp, vp, vp, ct.c_int32, ct.c_int32, i64, ct.c_float, vp, vp, ct.c_int32,
                                     vp]),
}

_lib = None


def lib() -> ct.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                               f"g.build()'` (hipcc, gfx950); there is no fallback path")
        handle = ct.CDLL(str(LIB_PATH))
        for name, (res, args) in ENTRY_POINTS.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().ssa_error_string(rc)
        raise RuntimeError(f"{what} failed: hip error {rc} ({msg.decode() if msg else '?'})")


def dtype_tag(t: torch.dtype) -> int:
    try:
        return _DT[t]
    except KeyError:
        raise TypeError(f"unsupported dtype {t}; expected float32, bfloat16 or float16") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"expected a GPU tensor, got one on {t.device}")
