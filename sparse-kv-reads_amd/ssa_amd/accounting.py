"""Bytes the cluster kernels read per decode step, in units of one key row.

Mirrors src/ssa/attn/accounting.py:19-32 (the metric's definition). Per KV head per step, besides
the ``rows`` K and V rows attended over:

  summaries   per cluster in use: its int8 (or fp32) direction plus two fp32 lengths and a count
  centroids   per cluster in use: the centroid the inserted key is compared against; with fixed
              random directions one fp32 table shared by ``heads`` KV heads
  labels      a 16-bit label per cached position, scanned to list the rows
  rows read   a 32-bit position and a 16-bit label per row read
  insertion   the inserted key, and its cluster's fp32 direction sum read and written
"""

from __future__ import annotations


def overhead_rows(*, n, rows, clusters, d: int, summary_bits: int = 8, fitted: bool = True, heads: int = 1,
                  key_bits: int = 16):
    """Key-row equivalents read per KV head per step besides the ``rows`` K and V rows, for
    ``n`` cached positions and ``clusters`` in use; numbers or tensors."""
    row = d * key_bits / 8
    vec = d * summary_bits / 8
    per_cluster = vec + 12 + (vec if fitted else 4 * d / heads)
    return (clusters * per_cluster + 2 * n + 6 * rows + row + 8 * d) / row


def kv_read_fraction(*, n, rows, clusters, d: int, **kw):
    """Fraction of the K+V cache's bytes read per step: ``rows`` rows of each plus the overhead."""
    return (2 * rows + overhead_rows(n=n, rows=rows, clusters=clusters, d=d, **kw)) / (2 * n)


def step_bytes(*, n, rows, clusters, d: int, **kw) -> float:
    """HBM bytes of one KV head's decode step under the same accounting (2-byte key rows)."""
    return (2 * rows + overhead_rows(n=n, rows=rows, clusters=clusters, d=d, **kw)) * d * kw.get("key_bits", 16) / 8
