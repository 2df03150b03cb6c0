"""Readers for the fixtures in tests/golden/data (written by gen_golden.c from the
reference itself).  Floats are stored as their u32 bit patterns."""
import os

import numpy as np

DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "data")


def f32(d, key):
    return np.array(d[key], dtype=np.uint32).view(np.float32)


def binf(name, cols):
    return np.fromfile(os.path.join(DATA, name), dtype=np.float32).reshape(-1, cols)


def same_bits(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))
