"""Shared helpers for the tests: seeded inputs and tensor <-> numpy."""

import numpy as np


def rng_normal(seed, *shapes, scale=1.0):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(s, dtype=np.float32) * np.float32(scale) for s in shapes]


def to_np(t):
    return t.detach().float().cpu().numpy()


def to_dev(x, device, dtype):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def max_abs(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b))) if a.size else 0.0
