"""Format settings.

The storage-lane mapping is part of the compressed format
(``LCT/config.py:14-18``); this build implements the default XOR swizzle
``lane ^ (row & 254)`` only.  The reference's backend, autotuning and TileLang
switches have no counterpart: the gfx950 HIP library is the only engine.
"""
from typing import Literal

lane_mapping: Literal["swizzle"] = "swizzle"
