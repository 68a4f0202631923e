"""vqlab_amd -- MI355X-native (gfx950) VQ weight-decode path of VQLab.

The HIP kernels live in libvqk.so (C ABI: include/vqk.h). The Python
modules mirror the reference runtime's interface over torch tensors:
  vqlab_amd.vq_pack    -- vq_pack (index packing)
  vqlab_amd.vq_switch  -- vq_switch (VQSwitchLinear, VQPLEEmbedding, kernels)
  vqlab_amd.vq_dense   -- vq_dense (VQLinear, VQEmbedding)
  vqlab_amd.moe        -- fused MoE decode layer (SwitchGLU + routing)
  vqlab_amd.artifact   -- VQLab artifact loader (config.json + safetensors)
"""
from . import _lib

__all__ = ["_lib"]


def load():
    """Load libvqk.so; raises ImportError when it is not built."""
    return _lib.lib()
