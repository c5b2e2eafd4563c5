"""Exactly reproducible inputs shared by make_golden.py and the tests.

hash_uniform(n, salt) maps an integer counter through a multiplicative hash to
float32 in [-1, 1): pure integer arithmetic, so every platform and numpy
version produces the same bits, and large inputs need not be stored.
"""
import numpy as np


def hash_uniform(n, salt):
    i = np.arange(n, dtype=np.uint64) + np.uint64(salt) * np.uint64(0x9E3779B9)
    h = (i * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF)
    h ^= h >> np.uint64(15)
    h = (h * np.uint64(2246822519)) & np.uint64(0xFFFFFFFF)
    h ^= h >> np.uint64(13)
    return ((h.astype(np.float64) / 2.0**32) * 2.0 - 1.0).astype(np.float32)


def msdef_value_map(salt=1):
    """(13125, 256) value tokens for the MSDeformAttn fixtures."""
    return hash_uniform(13125 * 256, salt).reshape(13125, 256)
