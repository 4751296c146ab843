"""Pins the oracle's FP8-E4M3 codec (the reference's convention,
crates/model/src/components/kv_cache_fp8.rs:143-212).

Independent checks: the reference's own test values
(kv_cache_fp8/tests.rs), torch's float8_e4m3fn conversions wherever that
format and the reference's agree, exhaustive round trips over the byte
codes, and a brute-force nearest-value search for the encoder."""
import os

import numpy as np
import pytest
import torch

ALL = np.arange(256, dtype=np.uint8)
EXP = (ALL >> 3) & 15
MANT = ALL & 7


def test_reference_known_values(oracle):
    # kv_cache_fp8/tests.rs:40-73: round trip within 15% over the normal range
    vals = np.array([1.0, 2.0, 0.5, -3.0, 0.1, -0.1, 100.0, -100.0, 50.0, 0.02, -0.02, 7.5],
                    np.float32)
    rec = oracle.fp8_decode(oracle.fp8_encode(vals))
    assert (np.abs(vals - rec) / np.abs(vals) < 0.15).all()
    # :75-98: values below 2^-6 flush to ~0 instead of saturating
    small = np.array([1e-4, 5e-4, 1e-3, -1e-3], np.float32)
    assert (np.abs(oracle.fp8_decode(oracle.fp8_encode(small))) < 0.02).all()
    # :110-116
    assert oracle.fp8_encode(np.float32(0.0)) == 0
    assert oracle.fp8_encode(np.float32(1.0)) != 0


def test_decode_matches_torch_e4m3fn(oracle):
    # Where the reference's convention and OCP e4m3fn agree: every code
    # except the reference's specials (0x80 NaN, 0x7C / 0xFC inf), OCP's
    # NaNs (0x7F / 0xFF) and exponent-0 codes (subnormal in OCP, never
    # produced by the reference encoder).
    dec = oracle.fp8_decode(ALL)
    ref = torch.from_numpy(ALL.copy()).view(torch.float8_e4m3fn).float().numpy()
    same = (EXP != 0) & ~np.isin(ALL, [0x7C, 0xFC, 0x7F, 0xFF])
    assert same.sum() == 256 - 16 - 4
    assert np.array_equal(dec[same], ref[same])
    assert np.isnan(dec[0x80]) and dec[0x7C] == np.inf and dec[0xFC] == -np.inf
    assert dec[0x38] == 1.0 and dec[0x7B] == 352.0 and dec[0xFB] == -352.0


def test_encode_matches_torch_away_from_ties(oracle):
    rng = np.random.default_rng(0)
    # up to 240, the largest code with exponent field <= 14; from 248 on the
    # reference saturates to 352 where OCP rounds to 256
    mag = np.exp(rng.uniform(np.log(2.0 ** -6), np.log(240.0), 200000)).astype(np.float32)
    x = mag * rng.choice([-1.0, 1.0], mag.size).astype(np.float32)
    # drop exact midpoints (torch rounds ties to even, the reference up)
    m, e = np.frexp(np.abs(x))
    frac = (m * 16.0) % 1.0
    x = x[frac != 0.5]
    ours = oracle.fp8_encode(x)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)


def test_round_trip_every_code(oracle):
    normal = (EXP >= 1) & (EXP <= 14)
    codes = np.concatenate([ALL[normal], np.array([0x00, 0x7B, 0xFB, 0x80, 0x7C, 0xFC],
                                                  np.uint8)])
    assert np.array_equal(oracle.fp8_encode(oracle.fp8_decode(codes)), codes)


def test_encode_is_nearest_with_ties_up(oracle):
    # Brute force: the encoder rounds to the nearest normal with exponent
    # field 1 .. 14 (ties up); a result of 2^8 or more (exponent field 15)
    # saturates to 352 (0x7B), and magnitudes below 2^-6 flush to 0 before
    # rounding.
    codes = ALL[(EXP >= 1) & (EXP <= 14) & (ALL < 0x80)]
    grid = np.sort(np.append(oracle.fp8_decode(codes).astype(np.float64), 256.0))
    rng = np.random.default_rng(1)
    mag = np.concatenate([
        np.exp(rng.uniform(np.log(1e-3), np.log(1e3), 100000)),
        (grid[:-1] + grid[1:]) / 2,          # every midpoint (a tie)
        grid, [2.0 ** -6 * (1 - 1 / 32), 2.0 ** -6]]).astype(np.float32)
    x = np.concatenate([mag, -mag])
    got = oracle.fp8_decode(oracle.fp8_encode(x)).astype(np.float64)
    a = np.abs(x.astype(np.float64))
    want = np.empty_like(a)
    for i, v in enumerate(a):
        if v < 2.0 ** -6:
            want[i] = 0.0          # flushed before rounding
        elif v >= grid[-1]:
            want[i] = 352.0        # saturation
        else:
            k = np.searchsorted(grid, v, side="right")
            lo, hi = grid[k - 1], grid[k]
            want[i] = hi if v - lo >= hi - v else lo
            if want[i] == 256.0:
                want[i] = 352.0
    want = np.where(x < 0, -want, want)
    want = np.where(want == 0, 0.0, want)
    assert np.array_equal(got, want)


def test_fp8_swar_helpers_exhaustive(tmp_path):
    # The integer decode and the exotic-code mask that the FP8 attention
    # kernels use, compiled for the host from pa_common.hpp and checked on
    # every pair of codes / every code in every byte position.
    import shutil
    import subprocess
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = str(tmp_path / "fp8_swar_check")
    subprocess.run([hipcc, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950",
                    "-I", os.path.join(root, "vllm-lite_amd", "csrc"),
                    os.path.join(root, "tests", "native", "fp8_swar_check.cpp"), "-o", exe],
                   check=True, capture_output=True)
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout
