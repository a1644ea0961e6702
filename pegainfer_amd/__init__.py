"""MI355X-native quantized MoE expert path (W4A16, INT4 group-32, bf16 activations).

Public surface:
  * ``pegainfer_amd.ops``   -- host mirror of the reference's Kimi-K2 expert ops
                               (pegainfer-kernels/src/ops/kimi_k2/experts.rs) over the C ABI;
  * ``pegainfer_amd.layer`` -- routed-expert / dense / DeepSeek-V2-Lite-shaped layers;
  * ``pegainfer_amd.synth`` -- seeded synthetic inputs of the benchmark configurations.

The compute runs in ``libpega_moe_hip.so`` (HIP, gfx950), declared in
``include/pega_moe.h``.  There is no CPU fallback.
"""
from . import _lib  # noqa: F401

__all__ = ["ops", "layer", "synth"]


def load():
    """Load the HIP library now (raises ImportError if it was not built)."""
    return _lib.lib()
