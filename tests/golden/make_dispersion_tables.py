"""Write ``d4_tables_hcnoar.npz`` and ``d3_tables_hcnoar.npz``: the derived D4 and D3
per-element tables (the oracle's restatements of the reference's table setup,
d4.py:444-500 and d3.py:194-219, 617-628) for H, C, N, O and Ar (D4: full-size arrays with
every other element zeroed; D3: compact arrays indexed by species). Run in a container
that holds the reference:

    python tests/golden/make_dispersion_tables.py /path/to/xnn/src/xnn/common/models

The input files (``d4_reference.npz``, ``d3_reference.npz``) are loaded as data
(``allow_pickle=False``); their values derive from dftd4 / multicharge / mctc-lib and
simple-dftd3. The outputs are test fixtures.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.d3 import derive_tables as derive_d3  # noqa: E402
from oracle.d4 import derive_tables, subset_tables  # noqa: E402

ELEMENTS = (1, 6, 7, 8, 18)


def main(models_dir: str) -> None:
    with np.load(os.path.join(models_dir, "d4_reference.npz"), allow_pickle=False) as f:
        raw = {k: f[k] for k in f.files}
    tables = subset_tables(derive_tables(raw), ELEMENTS)
    out = os.path.join(HERE, "d4_tables_hcnoar.npz")
    np.savez_compressed(out, elements=np.array(ELEMENTS), **tables)
    print("wrote", out, os.path.getsize(out), "bytes")
    with np.load(os.path.join(models_dir, "d3_reference.npz"), allow_pickle=False) as f:
        raw3 = {k: f[k] for k in f.files}
    out3 = os.path.join(HERE, "d3_tables_hcnoar.npz")
    np.savez_compressed(out3, **derive_d3(raw3, ELEMENTS))
    print("wrote", out3, os.path.getsize(out3), "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src/xnn/common/models")
