"""MI355X-native implementation of the LCT BF16 exponent-Huffman codec.

The public modules mirror the reference package ``LCT``: ``operations``,
``comp_format``, ``comp_tensor``, ``tensor_buffer``, ``LCTensor`` and
``codec``.  All compute runs in ``lib/liblct_hip.so`` (gfx950 HIP kernels).
"""
from .comp_format import Distribution, DistType, NoiseLevel, StorageLayout

__all__ = ["Distribution", "DistType", "NoiseLevel", "StorageLayout"]
