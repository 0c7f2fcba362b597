"""Convert the reference's nine spconv golden fixtures into plain .npz files.

The reference ships them as torch-saved dicts under tests/fixtures/ of the
reference tree (made by its tests/generate_spconv_goldens.py with spconv's
ConvAlgo.Native on CPU).  They are data: inputs, weights and spconv's outputs
sorted by coordinate.  This script loads each with ``weights_only=True`` and
writes the same arrays plus a JSON header of the scalar fields, so the test
suite reads them with ``numpy.load`` (no pickle) and the reference tree is not
needed at run time.

Run from the repository root (only where the reference tree is mounted):

    python tests/golden/import_reference_fixtures.py /root/reference/tests/fixtures

Fixture data: Apache-2.0, from the reference project (mrpulford/trispconv).
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).parent


def main(src: str) -> None:
    for p in sorted(Path(src).glob("spconv_golden_*.pt")):
        d = torch.load(p, map_location="cpu", weights_only=True)
        arrays, meta = {}, {}
        for k, v in d.items():
            if torch.is_tensor(v):
                arrays[k] = v.numpy()
            else:
                meta[k] = v
        arrays["meta_json"] = np.frombuffer(json.dumps(meta, sort_keys=True).encode(), dtype=np.uint8)
        name = p.stem.replace("spconv_golden_", "")
        np.savez(OUT / f"spconv_{name}.npz", **arrays)
        print("wrote", OUT / f"spconv_{name}.npz", sorted(arrays))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/fixtures")
