"""GPU parity of the fused RoPE + KV-cache write."""
import numpy as np
import pytest
import torch

from helpers import assert_close
from test_gpu_cache_ops import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu


def bf16_ulps(a, b):
    ia = a.astype(np.int32)
    ib = b.astype(np.int32)
    return np.abs(ia - ib)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hq,hkv,d,theta", [(32, 8, 128, 5e5), (14, 2, 64, 1e6), (4, 4, 2, 1.0)])
def test_rope_reshape_and_cache(pa, oracle, dtype, hq, hkv, d, theta):
    rng = np.random.default_rng(hq + d)
    t, nb = 37, 8
    qkv = rng.standard_normal((t, hq + 2 * hkv, d), dtype=np.float32)
    if dtype == "bf16":
        qkv = oracle.f32_to_bf16(qkv)
    positions = rng.integers(0, 32768, size=t).astype(np.int64)
    positions[:3] = [0, 1, 16383]
    slots = rng.permutation(nb * 16)[:t].astype(np.int64)
    slots[5] = -1
    inv = oracle.rope_inv_freq(d, theta)
    g = to_dev(qkv)  # fused projection output; q/k/v are strided views
    q, k, v = g[:, :hq], g[:, hq:hq + hkv], g[:, hq + hkv:]
    kc, vc = pa.ops.new_cache(nb, hkv, d, torch.bfloat16 if dtype == "bf16" else torch.float32,
                              DEV)
    pa.rope_reshape_and_cache(q, k, v, kc, vc, to_dev(slots), to_dev(positions), to_dev(inv))
    got_q = to_np(g[:, :hq].contiguous())
    want_q = oracle.rope(qkv[:, :hq], positions, inv)
    want_k = oracle.rope(qkv[:, hq:hq + hkv], positions, inv)
    kref = np.zeros((nb, hkv, 16, d), qkv.dtype)
    vref = np.zeros_like(kref)
    oracle.reshape_and_cache(want_k, qkv[:, hq + hkv:], kref, vref, slots)
    got_k, got_v = to_np(kc), oracle.v_to_ref(to_np(vc))
    assert np.array_equal(got_v, vref)  # V is a copy: bit-exact
    if dtype == "bf16":
        # cos/sin of the same f32 angle from two libms: at most 1 bf16 ulp apart
        assert bf16_ulps(got_q, want_q).max() <= 1
        assert bf16_ulps(got_k, kref).max() <= 1
    else:
        assert_close(got_q, want_q, 2e-5, 2e-5, "q")
        assert_close(got_k, kref, 2e-5, 2e-5, "k")
    # k/v inputs untouched, q rows of skipped tokens still rotated
    assert np.array_equal(to_np(g[:, hq:].contiguous()), qkv[:, hq:])
