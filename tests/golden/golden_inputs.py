"""Closed-form seeded inputs of the golden fixtures (numpy legacy RandomState,
a frozen stream), shared by make_golden.py and the tests."""
import numpy as np

N = 65536


def inputs():
    rs = np.random.RandomState(20261201)
    x = rs.standard_normal((2, N)).astype(np.float32)
    u = rs.standard_normal((2, N)).astype(np.float32)
    return x, u


def cotangents(ncoef):
    rs = np.random.RandomState(777)
    return rs.standard_normal((2, ncoef, 2)).astype(np.float32)


def sliced_input():
    rs = np.random.RandomState(4242)
    return rs.standard_normal((1, 2, 100000)).astype(np.float32)
