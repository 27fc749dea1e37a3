"""Loads the golden fixtures of tests/golden (safetensors / JSON, no pickles)
and rebuilds the paged pools they describe."""
import hashlib
import json
import os

import torch
from safetensors.torch import load_file

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
HKV, D, P = 8, 128, 256


def load(name: str) -> dict:
    return load_file(os.path.join(GOLDEN, name))


def load_json(name: str) -> dict:
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def sha(t: torch.Tensor) -> str:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def decode_small_pool(f: dict):
    kc = torch.zeros(4, P, HKV, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[:, :16] = f["k_rows"]
    vc[:, :16] = f["v_rows"]
    return kc, vc


def prefill_small_pool(f: dict):
    kc = torch.zeros(2, P, HKV, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[1, :36], vc[1, :36] = f["k0"], f["v0"]
    kc[0, :21], vc[0, :21] = f["k1"], f["v1"]
    return kc, vc
