"""ctypes wrapper of the canonical-arithmetic oracle (oracle/canon.c): TEST INFRASTRUCTURE ONLY.

``CanonIndex`` holds one layer's cluster state for ``H_kv`` heads as numpy arrays, in the same
layout as the GPU index, and advances it with the C restatement:
  build(K, ...)    prefill of SphereIndexGPU._build (src/ssa/attn/sphere_gpu.py:187-219)
  insert(K, n)     _bin_kernel + _split_cluster (src/ssa/kernels/sphere_fused.py:49-227)
  select(q, ...)   labels_and_weights (src/ssa/attn/sphere_gpu.py:412-442)
  compact(w, n)    the exact selected set {j < n : w[label_j] > 0} (src/ssa/kernels/labeled_attn.py:186-199)
``CanonIndex.from_gpu(index)`` copies a GPU index's state, so a test can run both sides from
identical summaries.
"""

from __future__ import annotations

import ctypes as ct
import math
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libcanon.so"


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = ct.CDLL(str(LIB))
        _lib.canon_dot.restype = ct.c_float
        _lib.canon_dot.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_int]
        _lib.canon_dot_chunked.restype = ct.c_float
        _lib.canon_dot_chunked.argtypes = [ct.c_void_p, ct.c_void_p, ct.c_int]
        _lib.canon_exp.restype = ct.c_float
        _lib.canon_exp.argtypes = [ct.c_float]
        _lib.canon_q8.restype = ct.c_int8
        _lib.canon_q8.argtypes = [ct.c_float]
        _lib.canon_insert.restype = None
        _lib.canon_insert.argtypes = [ct.POINTER(HeadC), ct.c_void_p, ct.c_int, ct.c_int, ct.c_float, ct.c_float,
                                      ct.c_int, ct.c_int]
        _lib.canon_select.restype = None
        _lib.canon_select.argtypes = [ct.POINTER(HeadC), ct.c_void_p, ct.c_int, ct.c_double, ct.c_int, ct.c_float,
                                      ct.c_void_p]
        _lib.canon_split_fit_head.restype = ct.c_int
        _lib.canon_split_fit_head.argtypes = [ct.POINTER(HeadC), ct.c_void_p, ct.c_int, ct.c_int, ct.c_float,
                                              ct.c_float, ct.c_int, ct.c_int, ct.c_int, ct.POINTER(ct.c_int)]
        _lib.canon_refresh8.restype = None
        _lib.canon_refresh8.argtypes = [ct.POINTER(HeadC)]
        _lib.canon_bisect.restype = None
        _lib.canon_bisect.argtypes = [ct.c_void_p, ct.c_int, ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_int,
                                      ct.c_void_p]
        _lib.canon_kmeans_parts.restype = None
        _lib.canon_kmeans_parts.argtypes = [ct.c_void_p, ct.c_int, ct.c_void_p, ct.c_void_p, ct.c_void_p, ct.c_int,
                                            ct.c_int, ct.c_int, ct.c_void_p]
        _lib.canon_build.restype = None
        _lib.canon_build.argtypes = [ct.POINTER(HeadC), ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p, ct.c_int,
                                     ct.c_int, ct.c_int, ct.c_void_p]
    return _lib


class HeadC(ct.Structure):
    _fields_ = [("C", ct.c_int), ("d", ct.c_int), ("ms", ct.c_int), ("summary_bits", ct.c_int),
                ("shared_dirs", ct.c_int),
                ("n_c", ct.c_void_p), ("sum_dir", ct.c_void_p), ("dir8", ct.c_void_p), ("cent", ct.c_void_p),
                ("cent8", ct.c_void_p), ("mmax", ct.c_void_p), ("mmin", ct.c_void_p), ("count", ct.c_void_p),
                ("ksum", ct.c_void_p), ("mu_ref", ct.c_void_p), ("rbar", ct.c_void_p), ("cap", ct.c_void_p),
                ("vthr", ct.c_void_p), ("flags", ct.c_void_p), ("end", ct.c_void_p), ("nsplit", ct.c_void_p),
                ("labels", ct.c_void_p)]


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def canon_dot(a, b) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return float(lib().canon_dot(_p(a), _p(b), a.shape[0]))


def canon_dot_chunked(a, b) -> float:
    """The selection's scoring dot: chain j over elements [j*d/8, (j+1)*d/8)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return float(lib().canon_dot_chunked(_p(a), _p(b), a.shape[0]))


def canon_exp(x: float) -> float:
    return float(lib().canon_exp(float(x)))


def canon_q8(u: float) -> int:
    return int(lib().canon_q8(float(u)))


def _members(K, mu):
    K = np.ascontiguousarray(K, dtype=np.float32)
    m, d = K.shape
    mu = np.zeros(d, np.float32) if mu is None else np.ascontiguousarray(mu, dtype=np.float32)
    mem = np.arange(m, dtype=np.int32)
    mag = np.array([np.float32(np.sqrt(np.float32(canon_dot(K[j] - mu, K[j] - mu)))) for j in range(m)], np.float32)
    return K, mu, mem, mag


def canon_bisect(K, mu=None) -> np.ndarray:
    """Sides of the bisection of the rows of ``K [m, d]`` (centred by ``mu``; _bisect_padded)."""
    K, mu, mem, mag = _members(K, mu)
    side = np.zeros(K.shape[0], np.int32)
    lib().canon_bisect(_p(K), K.shape[1], _p(mu), _p(mem), _p(mag), K.shape[0], _p(side))
    return side


def canon_kmeans_parts(K, k: int, iters: int, mu=None) -> np.ndarray:
    """Parts of the cosine k-means division of the rows of ``K [m, d]`` into ``k`` (_kmeans_padded)."""
    K, mu, mem, mag = _members(K, mu)
    part = np.zeros(K.shape[0], np.int32)
    lib().canon_kmeans_parts(_p(K), K.shape[1], _p(mu), _p(mem), _p(mag), K.shape[0], int(k), int(iters), _p(part))
    return part


GROUP_ID = {"sum_share": 0, "per_head": 1, "max": 2, "max_rel": 3}
STATE = ("n_c", "sum_dir", "dir8", "cent", "cent8", "mmax", "mmin", "count", "ksum", "mu_ref", "rbar", "cap", "vthr",
         "flags", "end", "nsplit", "labels")


class CanonIndex:
    """One layer's cluster state for ``H_kv`` heads (numpy), advanced by the C oracle."""

    def __init__(self, H_kv: int, d: int, *, C: int, capacity: int, C_init: int | None = None,
                 partition: str = "kmeans", summary_bits: int = 8, ms: int = 8192, cap: float = math.inf,
                 vthr: float = math.inf, dirs: np.ndarray | None = None):
        self.H_kv, self.d, self.C, self.capacity = H_kv, d, C, capacity
        self.C_init = C if C_init is None else C_init
        self.partition, self.summary_bits, self.ms = partition, summary_bits, min(ms, capacity)
        kmeans = partition == "kmeans"
        self.n_c = np.full(H_kv, self.C_init if kmeans else C, np.int32)
        self.sum_dir = np.zeros((H_kv, C, d), np.float32)
        self.dir8 = np.zeros((H_kv, C, d), np.int8) if summary_bits == 8 else None
        if kmeans:
            self.cent = np.zeros((H_kv, C, d), np.float32)
            self.cent8 = np.zeros((H_kv, C, d), np.int8) if summary_bits == 8 else None
        else:
            self.cent = np.ascontiguousarray(dirs, dtype=np.float32)
            self.cent8 = None
        self.mmax = np.zeros((H_kv, C), np.float32)
        self.mmin = np.full((H_kv, C), np.inf, np.float32)
        self.count = np.zeros((H_kv, C), np.int32)
        self.ksum = np.zeros((H_kv, d), np.float32)
        self.mu_ref = np.zeros((H_kv, d), np.float32)
        self.rbar = np.zeros(H_kv, np.float32)
        self.cap = np.full(H_kv, cap, np.float32)
        self.vthr = np.full(H_kv, vthr, np.float32)
        self.flags = np.zeros(H_kv, np.int32)
        self.end = np.zeros(H_kv, np.int32)
        self.nsplit = np.zeros(H_kv, np.int32)
        self.labels = np.full((H_kv, capacity), C, np.int16)

    @classmethod
    def from_gpu(cls, idx) -> "CanonIndex":
        """A copy of a GPU ``SphereIndexFused``'s state."""
        o = cls.__new__(cls)
        o.H_kv, o.d, o.C, o.capacity = idx.H_kv, idx.d, idx.C, idx.capacity
        o.C_init, o.partition, o.summary_bits, o.ms = idx.C_init, idx.partition, idx.summary_bits, idx.MS
        for name in STATE:
            src = "end_dev" if name == "end" else name
            t = getattr(idx, src)
            setattr(o, name, None if t is None else np.ascontiguousarray(t.detach().cpu().numpy()))
        return o

    def _head(self, h: int) -> HeadC:
        s = HeadC()
        s.C, s.d, s.ms, s.summary_bits = self.C, self.d, self.ms, self.summary_bits
        s.shared_dirs = int(self.partition != "kmeans")
        for name in STATE:
            a = getattr(self, name)
            if a is None:
                setattr(s, name, None)
            elif name == "cent" and self.partition != "kmeans":
                s.cent = _p(a)
            else:
                setattr(s, name, a[h:h + 1].ctypes.data if a.ndim == 1 else a[h].ctypes.data)
        return s

    @staticmethod
    def _keys(K) -> np.ndarray:
        """[H_kv, >=n, d] keys (torch or numpy, any float dtype) widened exactly to fp32."""
        if hasattr(K, "detach"):
            K = K.detach().float().cpu().numpy()
        return np.ascontiguousarray(K, dtype=np.float32)

    def build(self, K, *, start: int, end: int, heads=None, mu=None, fit: bool = True, iters: int = 10,
              init_idx=None) -> None:
        Kf = self._keys(K)
        heads = range(self.H_kv) if heads is None else heads
        nb = end - start
        fit = fit and nb > 0 and self.partition == "kmeans"
        init = None if init_idx is None else np.ascontiguousarray(init_idx, dtype=np.int32)
        for i, h in enumerate(heads):
            m = None if mu is None else np.ascontiguousarray(mu[i], dtype=np.float32)
            kh = np.ascontiguousarray(Kf[h])
            lib().canon_build(self._head(h), _p(kh), start, end, _p(m), int(fit), self.C_init, iters, _p(init))

    def split_after_fit(self, K, *, start: int, end: int, split_factor: float, capk: float = 0.0,
                        iters: int = 10, heads=None) -> int:
        """Divide the clusters over their cap after a fit, in rounds (src/ssa/attn/sphere_gpu.py:
        307-338): a k-means round, then bisection rounds until no cluster is over the cap or a round
        divides nothing; then the int8 copies. Returns the number of rounds."""
        Kf = self._keys(K)
        heads = list(range(self.H_kv)) if heads is None else list(heads)
        nmeans, rounds = True, 0
        while True:
            rank = over = done = 0
            for h in heads:
                cap_now = max(float(self.cap[h]), float(np.float32(capk * (end - start))))   # float32 clamp
                n_over = ct.c_int(0)
                kh = np.ascontiguousarray(Kf[h])
                done += lib().canon_split_fit_head(self._head(h), _p(kh), start, end, float(split_factor),
                                                   float(cap_now), int(nmeans), iters, rank, ct.byref(n_over))
                rank += n_over.value
                over += n_over.value
            rounds += 1
            if over == 0 or (done == 0 and not nmeans):
                break
            nmeans = False
        for h in heads:
            lib().canon_refresh8(self._head(h))
        return rounds

    def insert(self, K, n: int, *, window: int = 64, delta: float = 0.03, capk: float = 0.0, reset_at: int = 0,
               var_min: int = 8) -> None:
        Kf = self._keys(K)
        for h in range(self.H_kv):
            kh = np.ascontiguousarray(Kf[h])
            lib().canon_insert(self._head(h), _p(kh), int(n), int(window), float(delta), float(capk),
                               int(reset_at or 2 ** 30), int(var_min))

    def select(self, q, *, budget: float, group: str = "sum_share") -> np.ndarray:
        """``w`` [H_kv or H, C+1] for ``q`` [H, d]."""
        if hasattr(q, "detach"):
            q = q.detach().float().cpu().numpy()
        q = np.ascontiguousarray(q, dtype=np.float32)
        H, d = q.shape
        G = H // self.H_kv
        gid = GROUP_ID[group]
        rows = G if gid == 1 else 1
        w = np.zeros((self.H_kv * rows, self.C + 1), np.float32)
        scale = np.float32(1.0 / math.sqrt(d))
        for h in range(self.H_kv):
            qh = np.ascontiguousarray(q[h * G:(h + 1) * G])
            wh = np.zeros((rows, self.C + 1), np.float32)
            lib().canon_select(self._head(h), _p(qh), G, float(budget), gid, float(scale), _p(wh))
            w[h * rows:(h + 1) * rows] = wh
        return w

    def compact(self, w: np.ndarray, n: int) -> list[np.ndarray]:
        """Ascending selected positions per KV head."""
        G = w.shape[0] // self.H_kv
        out = []
        for h in range(self.H_kv):
            wk = w[h * G:(h + 1) * G].max(0)
            lab = self.labels[h, :n].astype(np.int64)
            out.append(np.nonzero(wk[lab] > 0)[0].astype(np.int32))
        return out
