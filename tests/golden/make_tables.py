"""Write golden codebook fixtures from the reference's own table builder.

The codebook (probability model + length-limited Huffman with an escape
cutoff) is the one part of the codec that no invariant pins: its code lengths
come from SciPy QUADPACK integrals and package-merge over ``np.longdouble``
weights, so near-ties could flip lengths in a restatement.  This script is run
by hand in the build container, where the reference is mounted read-only at
``/root/reference``; it imports only the pure NumPy/SciPy modules
``LCT.compression.probabilities`` and ``LCT.compression.huffman_tables``
(``huffman_tables.py:196-242`` and ``probabilities.py:43-158``) and never
touches a GPU.  Only the resulting vectors are committed
(``tests/golden/tables.json``); the reference never travels.

Run:  python tests/golden/make_tables.py [/root/reference]
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

# (family, param, mean, zero_prob): the distributions the benchmark configs and
# the reference's default distribution configs use, plus a few more shapes so a
# wrong probability mapping (mean shift, zero point mass, scale) fails a case.
CASES = [
    ("gaussian", 1.0, 0.0, 0.0),
    ("laplace", 1.0, 0.0, 0.5),
    ("empirical", 1.0, 0.0, 0.0),
    ("laplace", 1.0, 0.0, 0.0),
    ("laplace", 1.0, 0.0, 0.01),
    ("empirical", 1.0, 0.0, 0.02),
    ("empirical", 1.0, 0.0, 0.5),
    ("gamma", 1.0, 0.0, 0.0),
    ("gaussian", 0.25, 0.0, 0.0),
    ("gaussian", 2.0, 0.0, 0.0),
    ("gaussian", 1.0, 0.5, 0.3),
    ("gaussian", 1.0, 50.0, 0.0),
    ("laplace", 1.5, 0.0, 0.0),
    ("empirical", 0.5, 0.0, 0.0),
    ("gaussian", 1.0, 0.0, 0.95),
]

_CHILD = r"""
import json, sys, math
sys.path.insert(0, sys.argv[1])
from LCT.compression.probabilities import (
    _exponent_probabilities, gaussian_probabilities, laplace_probabilities,
    empirical_probabilities, gamma_probabilities,
)
from LCT.compression.huffman_tables import _build_huffman_tables_from_lengths
cases = json.loads(sys.argv[2])
out = []
for family, param, mean, zero_prob in cases:
    if family == "gaussian":
        pdf = gaussian_probabilities(param, mean)
    elif family == "laplace":
        pdf = laplace_probabilities(param, mean)
    elif family == "empirical":
        pdf = empirical_probabilities(param, mean)
    else:
        pdf = gamma_probabilities()
    probs = _exponent_probabilities(pdf, zero_prob)
    enc, dec, rare = _build_huffman_tables_from_lengths(probs, max_length=10, max_esc_length=8)
    out.append({
        "family": family, "param": param, "mean": mean, "zero_prob": zero_prob,
        "probabilities_hex": [float(p).hex() for p in probs],
        "encode": [int(v) for v in enc],
        "decode": [int(v) for v in dec],
        "rare_length": int(rare),
    })
print(json.dumps(out))
"""


def main() -> None:
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    # A child process with only the reference on sys.path, so the build's own
    # ``LCT`` alias package cannot shadow the reference's modules.
    env = dict(os.environ, PYTHONPATH="")
    result = subprocess.run(
        [sys.executable, "-c", _CHILD, ref, json.dumps(CASES)],
        check=True, capture_output=True, text=True, cwd="/tmp", env=env,
    )
    tables = json.loads(result.stdout)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tables.json")
    with open(path, "w") as handle:
        json.dump({"source": "LCT/compression/huffman_tables.py:196-242 via "
                             "probabilities.py:43-158", "cases": tables},
                  handle, indent=0)
    print(f"wrote {len(tables)} cases to {path}")


if __name__ == "__main__":
    main()
