"""Loads tests/golden/golden.npz (written by make_golden.py) as torch tensors."""
import json
from pathlib import Path

import numpy as np
import torch

PATH = Path(__file__).resolve().parent / "golden.npz"


def load():
    data = np.load(PATH, allow_pickle=False)
    out = {}
    for name in data.files:
        a = data[name]
        if name == "manifest":
            out[name] = json.loads(bytes(a).decode())
        elif a.dtype == np.uint16:
            out[name] = torch.from_numpy(a.view(np.int16).copy()).view(torch.float16)
        else:
            out[name] = torch.from_numpy(a.copy())
    return out
