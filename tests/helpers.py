"""Shared test helpers (seeded inputs, golden loading)."""
import json
from functools import lru_cache
from pathlib import Path

import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


@lru_cache(maxsize=None)
def golden(name: str):
    return json.loads((GOLDEN / name).read_text())


def dev():
    return torch.device("cuda", 0)
