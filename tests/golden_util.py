"""Loading the golden fixtures written by tests/golden/make_golden.py (plain .npz data, no pickles)."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def fixtures(kind: str) -> list[Path]:
    return sorted(GOLDEN.glob(f"{kind}_*.npz"))


def load(path: Path) -> dict:
    """Fixture arrays plus its metadata; bf16 inputs come back as float32 holding the bf16 values."""
    with np.load(path, allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    meta = json.loads(str(d.pop("meta")))
    qkv = d["qkv"]
    if qkv.dtype == np.uint16:
        qkv = (qkv.astype(np.uint32) << 16).view(np.float32)
    d["qkv"] = np.asarray(qkv, np.float32)
    d.update(meta)
    if meta["kind"] == "band":
        hd = meta["head_dim"]
        for key, name in (("q_dyt", "q_norm"), ("k_dyt", "k_norm")):
            v = d[key]
            d[name] = {"alpha": np.float32(v[0]), "gamma": v[1:1 + hd].copy(), "beta": v[1 + hd:].copy()}
    return d
