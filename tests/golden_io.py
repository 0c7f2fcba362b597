"""Read the golden fixtures under tests/golden/ (plain .npz, no pickle)."""
from __future__ import annotations

import json
from pathlib import Path
from typing import Dict, List, Tuple

import numpy as np

GOLDEN = Path(__file__).parent / "golden"


def fixture_names() -> List[str]:
    return sorted(p.stem.replace("spconv_", "") for p in GOLDEN.glob("spconv_*.npz"))


def load(name: str) -> Tuple[Dict[str, np.ndarray], Dict]:
    with np.load(GOLDEN / f"spconv_{name}.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files if k != "meta_json"}
        meta = json.loads(bytes(z["meta_json"]).decode())
    return arrays, meta


def encode(idx, shape):
    D, H, W = shape
    i = np.asarray(idx).astype(np.int64)
    return ((i[:, 0] * D + i[:, 1]) * H + i[:, 2]) * W + i[:, 3]


def sort_by_coord(features, indices, shape):
    order = np.argsort(encode(indices, shape), kind="stable")
    return features[order], indices[order]
