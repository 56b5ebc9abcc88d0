"""MI355X-native clustered sparse decode attention (the hot path of aaholmes/sparse-kv-reads).

Submodules mirror the reference package's modules for this path:
  ssa_amd.labeled_attn   <- ssa.kernels.labeled_attn   (attention over selected rows, merge, compaction)
  ssa_amd.sphere_fused   <- ssa.kernels.sphere_fused   (the incremental cluster index)
  ssa_amd.graph_kernels  <- ssa.kernels.graph_kernels  (graph-safe step objects, all-layer insertion)
  ssa_amd.patch          <- ssa.models.patch           (the engine's decode_attn_op seam)
  ssa_amd.accounting     <- ssa.attn.accounting        (bytes read per step)
  ssa_amd.graph_decode   <- ssa.models.graph_decode    (the whole decode step in one hipGraph)
  ssa_amd.qwen3          the engine's model surface: a minimal Qwen3 with the decode seam
  ssa_amd.synth          synthetic Qwen3-shaped caches with clustered key directions
All compute runs in libssa_hip.so (HIP, gfx950); nothing falls back to another path.
"""

from ._lib import LIB_PATH, lib  # noqa: F401

__all__ = ["LIB_PATH", "lib"]
