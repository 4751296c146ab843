"""RoPE: the oracle restatement pinned by closed forms, and the library's
host inverse-frequency table checked against it (CPU only)."""
import math

import numpy as np
import pytest

from helpers import assert_close


def test_rope_identity_at_position_zero(oracle):
    # rope/tests.rs:92-106: at position 0 every angle is 0
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 2, 64), dtype=np.float32)
    inv = oracle.rope_inv_freq(64, 10000.0)
    y = oracle.rope(x, [0, 0, 0], inv)
    assert np.array_equal(x, y)


def test_rope_position_one_dim_zero(oracle):
    # rope/tests.rs:108-113: pos 1, i 0 -> angle 1.0; x = e_0 -> (cos 1, sin 1)
    x = np.zeros((1, 1, 64), np.float32)
    x[0, 0, 0] = 1.0
    y = oracle.rope(x, [1], oracle.rope_inv_freq(64, 10000.0))
    assert abs(y[0, 0, 0] - math.cos(1.0)) < 1e-6 and abs(y[0, 0, 32] - math.sin(1.0)) < 1e-6
    assert np.count_nonzero(y) == 2


def test_rope_rotation_direction(oracle):
    # D = 2, one frequency theta_0 = 1: q = (1, 0) at m, k = (0, 1) at n gives
    # <R(m) q, R(n) k> = sin((m - n) * 1).  The inverse rotation (the bug
    # fixed as RIL ISS-012 in the reference) gives sin((n - m)).
    inv = np.array([1.0], np.float32)
    for m, n in [(5, 2), (2, 5), (17, 3)]:
        q = oracle.rope(np.array([[[1.0, 0.0]]], np.float32), [m], inv)
        k = oracle.rope(np.array([[[0.0, 1.0]]], np.float32), [n], inv)
        assert abs(float(q.ravel() @ k.ravel()) - math.sin(m - n)) < 1e-5


def test_rope_relative_position_invariance(oracle):
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 1, 128), dtype=np.float32)
    k = rng.standard_normal((1, 1, 128), dtype=np.float32)
    inv = oracle.rope_inv_freq(128, 10000.0)
    d0 = float(oracle.rope(q, [40], inv).ravel() @ oracle.rope(k, [13], inv).ravel())
    d1 = float(oracle.rope(q, [140], inv).ravel() @ oracle.rope(k, [113], inv).ravel())
    assert abs(d0 - d1) < 1e-3


def test_inv_freq_closed_forms(oracle):
    d, theta = 128, 1e6
    i = np.arange(d // 2)
    want = theta ** (-2.0 * i / d)
    base = oracle.rope_inv_freq(d, theta)
    assert_close(base, want, 0, 1e-6, "default")
    assert_close(oracle.rope_inv_freq(d, theta, "linear", 4.0), want / 4.0, 0, 1e-6, "linear")
    yt = theta * 4.0 ** (d / (d - 2))
    assert_close(oracle.rope_inv_freq(d, theta, "yarn", 4.0), yt ** (-2.0 * i / d), 0, 1e-5,
                 "yarn")
    # factor 1 is a no-op for every type; dynamic below the original length too
    for t in ("linear", "yarn", "dynamic"):
        assert np.array_equal(oracle.rope_inv_freq(d, theta, t, 1.0, 4096, 8192), base)
    assert np.array_equal(oracle.rope_inv_freq(d, theta, "dynamic", 4.0, 4096, 2048), base)
    scale = 4.0 * 8192 / 4096 - 3.0
    dt = theta * scale ** (d / (d - 2))
    assert_close(oracle.rope_inv_freq(d, theta, "dynamic", 4.0, 4096, 8192),
                 dt ** (-2.0 * i / d), 0, 1e-5, "dynamic")
    # Su: short factors below the first dim whose wavelength exceeds orig
    sf = np.full(d // 2, 2.0, np.float32)
    lf = np.full(d // 2, 8.0, np.float32)
    got = oracle.rope_inv_freq(d, theta, "su", 1.0, 4096, 0, sf, lf)
    boundary = next(j for j in range(d // 2) if 2 * math.pi / base[j] > 4096)
    assert_close(got[:boundary], base[:boundary] / 2.0, 0, 1e-6, "su short")
    assert_close(got[boundary:], base[boundary:] / 8.0, 0, 1e-6, "su long")


@pytest.mark.parametrize("args", [
    (128, 10000.0, "default"), (64, 1e6, "linear", 8.0), (128, 5e5, "yarn", 4.0),
    (128, 1e6, "dynamic", 4.0, 4096, 9000), (64, 1e4, "su", 1.0, 2048, 0)])
def test_library_inv_freq_matches_oracle(pa, oracle, args):
    kw = {}
    if args[2] == "su":
        kw = {"short_factor": np.linspace(1, 2, args[0] // 2),
              "long_factor": np.linspace(3, 9, args[0] // 2)}
    got = pa.rope_inv_freq(*args, **kw)
    want = oracle.rope_inv_freq(*args, **kw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
