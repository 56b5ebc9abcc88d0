"""Host-side logic of the package (CPU only): argument checks and error behaviour of the API
that mirrors the reference (ValueError / AssertionError as in src/ssa/attn/sphere_gpu.py:119-128,
src/ssa/kernels/sphere_fused.py:339-360, src/ssa/kernels/labeled_attn.py:96-101), the seeded
k-means seed members, the synthetic cache generator, the byte accounting of bench.py and the
one-GPU guard of bench.py. Nothing here launches a kernel."""

from __future__ import annotations

import json
import math
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import reference as ref
from ssa_amd.sphere_fused import SphereIndexFused, fixed_directions, kmeans_init_indices

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.parametrize("kw,exc", [
    (dict(partition="voronoi"), ValueError),
    (dict(summary_bits=16), ValueError),
    (dict(C=64, C_init=128, partition="kmeans"), ValueError),
    (dict(split_factor=2.0, partition="random"), ValueError),
    (dict(C=100), AssertionError),
    (dict(C=2048), AssertionError),
])
def test_bad_configuration_is_rejected(kw, exc):
    with pytest.raises(exc):
        SphereIndexFused(**kw)


def test_capacity_is_checked_before_any_device_work():
    idx = SphereIndexFused(C=64, capacity=100, partition="kmeans")
    with pytest.raises(ValueError, match="exceeds capacity"):
        idx.observe(torch.zeros(2, 200, 16), 150)


def test_unknown_group_is_rejected():
    idx = SphereIndexFused(C=64, partition="kmeans")
    with pytest.raises(ValueError, match="unknown group"):
        idx.labels_and_weights(torch.zeros(4, 16), n=10, budget=0.2, group="top")


def test_attention_shape_checks_come_before_the_device():
    from ssa_amd.labeled_attn import label_weighted_attention_compact
    q = torch.zeros(8, 16)
    with pytest.raises(AssertionError):
        label_weighted_attention_compact(q, torch.zeros(2, 10, 32), torch.zeros(2, 10, 32),
                                         torch.zeros(2, 10, dtype=torch.int16), torch.ones(2, 5))
    with pytest.raises(AssertionError):
        label_weighted_attention_compact(torch.zeros(8, 24), torch.zeros(2, 10, 24), torch.zeros(2, 10, 24),
                                         torch.zeros(2, 10, dtype=torch.int16), torch.ones(2, 5))
    with pytest.raises(ValueError, match="GPU"):
        label_weighted_attention_compact(q, torch.zeros(2, 10, 16), torch.zeros(2, 10, 16),
                                         torch.zeros(2, 10, dtype=torch.int16), torch.ones(2, 5))


def test_kmeans_seed_members_follow_the_reference_rule():
    # src/ssa/attn/clusterkv.py:34-35: randperm(m, CPU generator seeded)[arange(C) % m]
    g = torch.Generator().manual_seed(3)
    assert torch.equal(kmeans_init_indices(500, 64, 3), torch.randperm(500, generator=g)[:64])
    small = kmeans_init_indices(5, 12, 0)
    assert sorted(small[:5].tolist()) == list(range(5)) and torch.equal(small[5:10], small[:5])


def test_fixed_directions_are_unit_and_seeded():
    a = fixed_directions(256, 128, seed=1)
    assert torch.allclose(a.norm(dim=1), torch.ones(256), atol=1e-6)
    assert torch.equal(a, fixed_directions(256, 128, seed=1))
    assert not torch.equal(a, fixed_directions(256, 128, seed=2))


def test_synthetic_keys_cluster_by_direction():
    from ssa_amd.synth import KAPPA, make_cache
    K, V, q, which = make_cache(2, 2, 3000, 128, H=4, centers=16, seed=1, dtype=torch.float64)
    K2, _, _, which2 = make_cache(2, 2, 3000, 128, H=4, centers=16, seed=1, dtype=torch.float64)
    assert torch.equal(K, K2) and torch.equal(which, which2)                 # seeded, reproducible
    for b in range(2):
        for h in range(2):
            Kr = K[b, h] - K[b, h].mean(0)
            u = Kr / Kr.norm(dim=1, keepdim=True)
            cos = []
            for c in range(16):
                m = which[b, h] == c
                if m.sum() > 20:
                    cen = u[m].mean(0)
                    cos.append(float((u[m] @ (cen / cen.norm())).mean()))
            assert np.mean(cos) > 0.6                                          # tight around a centre
            sizes = torch.bincount(which[b, h], minlength=16).float()
            assert sizes.max() > 2 * sizes.mean()                              # ragged cluster sizes
    assert KAPPA / math.sqrt(KAPPA ** 2 + 127) > 0.85
    assert not torch.equal(K[0], K[1])                                         # sequences differ


def test_bench_bytes_follow_the_reference_accounting():
    sys.path.insert(0, str(ROOT))
    import bench
    rows = [6000, 7000]
    got = bench.step_bytes(rows, 32768)
    want = sum(2 * r * 256 + ref.overhead_rows(n=32768, rows=r, clusters=256, d=128) * 256 for r in rows)
    assert abs(got - want) < 1e-6 * want


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


def test_provenance_stamp_has_the_reference_fields():
    """src/ssa/harness/stamp.py:35-45: revision, torch version, python, platform, GPU."""
    from ssa_amd.stamp import stamp
    s = stamp({"x": 1})
    for k in ("git_sha", "torch_version", "hip_version", "python_version", "platform", "gpu", "x"):
        assert k in s
    assert s["git_sha"] and s["git_sha"] != "nogit"


def test_cpu_baseline_path_matches_the_numpy_oracle():
    """oracle/torch_ref.py (the timed CPU baseline) selects the same clusters as the numpy
    restatement and attends over every key to the same output."""
    import numpy as np
    import torch
    from oracle.reference import SphereIndexRef
    from oracle.torch_ref import SphereIndexTorch
    from ssa_amd.sphere_fused import kmeans_init_indices
    from ssa_amd.synth import make_cache
    K, V, q, _ = make_cache(1, 2, 700, 32, H=4, centers=16, seed=3, dtype=torch.float32)
    K, V, q = K[0].contiguous(), V[0].contiguous(), q[0].contiguous()
    t = SphereIndexTorch(C=16, window=16, init_indices=lambda m, c: kmeans_init_indices(m, c, 0))
    r = SphereIndexRef(C=16, window=16, init_indices=lambda m, c, s: kmeans_init_indices(m, c, s).numpy())
    for n in (640, 641, 642):
        out_t, lab_t, w_t = t.attend(q, K, V, n=n, budget=0.3)
        out_r, lab_r, w_r = r.attend(q.numpy(), K.numpy(), V.numpy(), n=n, budget=0.3)
        assert np.array_equal(lab_t.numpy(), lab_r)
        assert np.array_equal(w_t.numpy(), w_r)
        assert np.abs(out_t.numpy() - out_r).max() < 1e-4
