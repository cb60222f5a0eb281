"""Committed golden vectors (inputs and expected outputs) for the parity tests."""

from pathlib import Path

import numpy as np

GOLDEN_DIR = Path(__file__).resolve().parent


def load_golden(name: str):
    return np.load(GOLDEN_DIR / name, allow_pickle=False)
