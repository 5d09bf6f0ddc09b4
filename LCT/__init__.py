"""Drop-in module paths of the reference package ``LCT``.

``import LCT.operations`` (and the other reference module paths) resolves to
the MI355X implementation in ``losslessly_compressed_tensors_amd``, so code
written against the reference runs unchanged.
"""
import importlib
import sys

_IMPLEMENTATION = "losslessly_compressed_tensors_amd"
_MODULES = (
    "comp_format",
    "comp_tensor",
    "tensor_buffer",
    "operations",
    "LCTensor",
    "config",
    "codec",
    "codec.geometry",
    "codec.encode",
    "codec.decode",
    "codec.pointwise",
    "compression",
    "compression.probabilities",
    "compression.huffman_tables",
    "components",
    "components.dist_configs",
    "components.ops",
    "components.layers",
    "components.sparse_utils",
)

for _name in _MODULES:
    _module = importlib.import_module(f"{_IMPLEMENTATION}.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _module
    if "." not in _name:
        globals()[_name] = _module
