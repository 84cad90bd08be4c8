"""Write ``d4_tables_hcnoar.npz``: the derived D4 per-element tables (the oracle's
restatement of the reference's table setup, d4.py:444-500) for H, C, N, O and Ar,
every other element zeroed. Run in a container that holds the reference:

    python tests/golden/make_dispersion_tables.py /path/to/xnn/src/xnn/common/models

The input file (``d4_reference.npz``) is loaded as data (``allow_pickle=False``); its
values derive from dftd4 / multicharge / mctc-lib. The output is a test fixture.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.d4 import derive_tables, subset_tables  # noqa: E402

ELEMENTS = (1, 6, 7, 8, 18)


def main(models_dir: str) -> None:
    with np.load(os.path.join(models_dir, "d4_reference.npz"), allow_pickle=False) as f:
        raw = {k: f[k] for k in f.files}
    tables = subset_tables(derive_tables(raw), ELEMENTS)
    out = os.path.join(HERE, "d4_tables_hcnoar.npz")
    np.savez_compressed(out, elements=np.array(ELEMENTS), **tables)
    print("wrote", out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src/xnn/common/models")
