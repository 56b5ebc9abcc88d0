"""Writes the golden fixtures under tests/golden/ from the reference's own pure-PyTorch functions.

Run in the build container only (the reference checkout is not present on the GPU machine, and
nothing else in this repository imports it):

    python tests/golden/make_fixtures.py [/root/reference]

Functions pinned (float64 CPU; the inputs are float32 values, so the same numbers feed both sides):
  * spherical_kmeans              src/ssa/attn/clusterkv.py:27-46 (10-iteration trajectory)
  * _kmeans_padded                src/ssa/attn/sphere_gpu.py:56-73 (post-fit k-means division)
  * _bisect_padded                src/ssa/attn/sphere_gpu.py:76-102
  * SphereIndexGPU observe with split_factor > 0 (post-fit division and slot handout
    _split_overflow / _split_batch :307-391, then one key per step with in-step splits) and
    labels_and_weights in all four group modes (:412-442).
Each fixture is a small .npz holding its inputs and the reference's outputs; MANIFEST.json
records the SHA-256 of every file, the torch version and the reference revision they came from.
"""

from __future__ import annotations

import hashlib
import json
import math
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _mixture(rng: np.random.Generator, H: int, n: int, d: int, centers: int, kappa: float, *,
             alpha: float = 1.0, mean_scale: float = 0.5) -> np.ndarray:
    """Keys around ``centers`` directions per head (ragged popularity), float32 values."""
    out = np.empty((H, n, d), np.float32)
    for h in range(H):
        c = rng.standard_normal((centers, d))
        c /= np.linalg.norm(c, axis=1, keepdims=True)
        pi = rng.dirichlet(alpha * np.ones(centers))
        lab = rng.choice(centers, size=n, p=pi)
        u = kappa * c[lab] + rng.standard_normal((n, d))
        u /= np.linalg.norm(u, axis=1, keepdims=True)
        r = np.exp(0.3 * rng.standard_normal(n))
        mu = mean_scale * rng.standard_normal(d)
        out[h] = (mu + r[:, None] * u).astype(np.float32)
    return out


def main(ref_root: str) -> None:
    sys.path.insert(0, str(Path(ref_root) / "src"))
    import torch
    from ssa.attn.clusterkv import spherical_kmeans
    from ssa.attn.sphere_gpu import SphereIndexGPU, _bisect_padded, _kmeans_padded
    torch.set_num_threads(4)
    rng = np.random.default_rng(20260101)
    files = {}

    # -- A: the k-means trajectory on overlapping clusters (moves for several iterations) --------
    X = _mixture(rng, 2, 320, 16, centers=8, kappa=2.5)
    C, iters = 8, 10
    assign, cent = spherical_kmeans(torch.from_numpy(X).double(), C=C, iters=iters, seed=0)
    init = torch.randperm(X.shape[1], generator=torch.Generator().manual_seed(0))[torch.arange(C) % X.shape[1]]
    moves = []
    for it in range(1, iters + 1):                  # how the assignment changes with the iteration count
        a_it, _ = spherical_kmeans(torch.from_numpy(X).double(), C=C, iters=it, seed=0)
        moves.append(int((a_it != assign).sum()))
    files["kmeans_trajectory.npz"] = dict(X=X, C=C, iters=iters, seed=0, init=init.numpy().astype(np.int32),
                                          assign=assign.numpy().astype(np.int32), cent=cent.numpy(),
                                          moves_vs_final=np.array(moves, np.int32))

    # -- B: _kmeans_padded and _bisect_padded on padded rows ---------------------------------
    Kn = _mixture(rng, 3, 150, 16, centers=6, kappa=3.0, mean_scale=0.0)
    Kn = (Kn / np.linalg.norm(Kn, axis=-1, keepdims=True)).astype(np.float32)
    cnt = np.array([150, 97, 41], np.int64)
    valid = np.arange(150)[None, :] < cnt[:, None]
    k = np.array([5, 3, 2], np.int64)
    part = _kmeans_padded(torch.from_numpy(Kn).double(), torch.from_numpy(valid), torch.from_numpy(k), 10)
    side = _bisect_padded(torch.from_numpy(Kn).double(), torch.from_numpy(valid))
    files["padded_division.npz"] = dict(Kn=Kn, valid=valid, k=k.astype(np.int32), iters=10,
                                        part=part.numpy().astype(np.int32), side=side.numpy().astype(np.int32))

    # -- C: SphereIndexGPU with splitting: post-fit division, then one key per step -----------
    H_kv, G, d, n0, steps, window = 2, 2, 16, 400, 110, 16
    Cs, C_init, budget = 64, 8, 0.3
    K = _mixture(rng, H_kv, n0 + steps, d, centers=8, kappa=4.0, alpha=0.6)
    # a tight blob of 35% of the prompt keys (a sink-like direction): one fitted cluster holds it
    # whole and is over its cap at the fit, so the post-fit k-means division runs (k >= 3 parts)
    for h in range(H_kv):
        blob = rng.choice(np.arange(1, n0 - window), size=int(0.35 * n0), replace=False)
        v = rng.standard_normal(d)
        v = 1.5 * v / np.linalg.norm(v)
        K[h, blob] = (K[h, 1:n0 - window].mean(0) + v + 0.08 * rng.standard_normal((blob.size, d))).astype(np.float32)
    # the keys of the decode steps crowd into one direction per head, so clusters pass their cap
    for h in range(H_kv):
        u = K[h, n0 - window - 1]                   # a binned key's direction (relative to the mean)
        extra = u[None, :] + 0.05 * rng.standard_normal((steps + window, d)).astype(np.float32)
        K[h, n0 - window:] = extra[: steps + window].astype(np.float32)
    Q = rng.standard_normal((steps, H_kv * G, d)).astype(np.float32) * 2.0
    idx = SphereIndexGPU(C=Cs, window=window, delta=1e9, capacity=n0 + steps, partition="kmeans", C_init=C_init,
                         split_factor=2.0, kmeans_iters=10, check_every=10 ** 9, seed=0)
    Kt = torch.from_numpy(K).double()
    idx.observe(Kt, n0)
    # copies: the index updates its tensors in place during the steps below
    fit = dict(n_c=idx.n_c.numpy().astype(np.int32), labels=idx.labels[:, :n0].numpy().astype(np.int16),
               count=idx.count.numpy().astype(np.int32), sum_dir=idx.sum_dir.numpy().copy(),
               mmax=idx.mmax.numpy().copy(), mmin=idx.mmin.numpy().copy(), cap=idx.cap.numpy().copy(),
               mu_ref=idx.mu_ref.numpy().copy(), splits=idx.splits)
    W = {g: [] for g in ("sum_share", "per_head", "max", "max_rel")}
    n_c, splits = [], []
    for s in range(steps):
        idx.observe(Kt, n0 + 1 + s)
        for g in W:
            _, w = idx.labels_and_weights(torch.from_numpy(Q[s]).double(), n=n0 + 1 + s, budget=budget, group=g)
            W[g].append(w.numpy().astype(np.float32))
        n_c.append(idx.n_c.numpy().astype(np.int32))
        splits.append(idx.splits)
    end = dict(labels=idx.labels[:, :n0 + steps].numpy().astype(np.int16), count=idx.count.numpy().astype(np.int32),
               sum_dir=idx.sum_dir.numpy().copy(), mmax=idx.mmax.numpy().copy(), mmin=idx.mmin.numpy().copy(),
               n_c=idx.n_c.numpy().astype(np.int32))
    files["index_steps.npz"] = dict(
        K=K, Q=Q, H_kv=H_kv, G=G, C=Cs, C_init=C_init, window=window, n0=n0, steps=steps, budget=budget,
        split_factor=2.0, kmeans_iters=10, seed=0,
        **{f"fit_{k2}": v for k2, v in fit.items()}, **{f"end_{k2}": v for k2, v in end.items()},
        n_c_steps=np.stack(n_c), splits_steps=np.array(splits, np.int32),
        **{f"w_{g}": np.stack(v) for g, v in W.items()})

    manifest = {"torch": torch.__version__, "numpy": np.__version__, "files": {}}
    try:
        manifest["reference_rev"] = subprocess.check_output(["git", "-C", ref_root, "rev-parse", "HEAD"], text=True,
                                                            stderr=subprocess.DEVNULL).strip()
    except Exception:
        manifest["reference_rev"] = "unknown"
    for name, arrs in files.items():
        p = HERE / name
        np.savez_compressed(p, **{k2: np.asarray(v) for k2, v in arrs.items()})
        manifest["files"][name] = hashlib.sha256(p.read_bytes()).hexdigest()
        print(name, p.stat().st_size, "bytes")
    (HERE / "MANIFEST.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print("k-means: assignments that differ from the final one after 1..10 iterations:", files[
        "kmeans_trajectory.npz"]["moves_vs_final"].tolist())
    print("index: post-fit n_c", fit["n_c"].tolist(), "splits", fit["splits"], "-> after steps n_c", end["n_c"].tolist(),
          "splits", splits[-1])


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
