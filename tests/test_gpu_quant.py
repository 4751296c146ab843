"""GPU parity of the quantised PagedKvCache (int8 values in f32 with one
scale per block, crates/model/src/paged_tensor/tensor_store/buffer.rs:
170-231, 320-331): writes, scales and reads bit-exact against the oracle and
the golden fixtures; attention over a quantised cache against the oracle's
attention over the dequantised cache."""
import numpy as np
import pytest
import torch

from helpers import F32_ATOL, F32_RTOL, assert_close, golden
from test_gpu_cache_ops import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_golden_single_token(pa):
    f = golden("kv_quant.json")["single_token"]
    c = f["cache"]
    cache = pa.PagedKvCache(1, c["num_heads"], c["head_dim"], c["num_blocks"], torch.float32,
                            DEV, quantized=True)
    shape = (c["num_heads"], c["head_dim"])
    k = torch.tensor(f["k"], dtype=torch.float32, device=DEV).reshape(shape)
    v = torch.tensor(f["v"], dtype=torch.float32, device=DEV).reshape(shape)
    cache.write_kv(0, 0, 0, k, v)
    assert to_np(cache.scales(0))[0].view(np.uint32) == f["expect_scale_bits"]
    assert np.all(to_np(cache.key_cache(0))[0, :, 0, :] == f["expect_k_int"])
    assert np.all(to_np(cache.value_cache(0))[0, :, :, 0] == f["expect_v_int"])
    rk, rv = cache.read_kv(0, [0], 1)
    assert np.all(bits(to_np(rk)) == f["expect_k_read_bits"])


def test_golden_per_block_scale(pa, oracle):
    f = golden("kv_quant.json")["per_block_scale"]
    c = f["cache"]
    cache = pa.PagedKvCache(1, 1, 1, c["num_blocks"], torch.float32, DEV, quantized=True)
    vals = np.asarray(f["values"], np.float32)
    for t, x in enumerate(vals):
        xt = torch.tensor([[x]], dtype=torch.float32, device=DEV)
        cache.write_kv(0, f["block_ids"][t // 16], t % 16, xt, xt)
    rk, rv = cache.read_kv(0, f["block_ids"], len(vals))
    rk, rv = to_np(rk), to_np(rv)
    for t, x in enumerate(vals):
        tol = f["tolerance_large"] if x > 50 else f["tolerance_small"]
        assert abs(rk[t, 0, 0] - x) < tol and abs(rv[t, 0, 0] - x) < tol


class QuantOracle:
    def __init__(self, oracle, h, d, nb):
        self.o = oracle
        self.k = np.zeros((nb, h, 16, d), np.float32)
        self.v = np.zeros_like(self.k)
        self.s = np.ones(nb, np.float32)

    def write(self, blk, off, k, v):
        assert self.o.quant_write_kv(self.k, self.v, self.s, blk, off, k, v) == 0


@pytest.mark.parametrize("h,d", [(2, 64), (4, 128), (3, 40)])
def test_write_sequence_bit_exact(pa, oracle, h, d):
    rng = np.random.default_rng(h * d)
    nb = 10
    cache = pa.PagedKvCache(1, h, d, nb, torch.float32, DEV, quantized=True)
    ref = QuantOracle(oracle, h, d, nb)

    def data(t):
        x = (rng.standard_normal((t, h, d)) * rng.choice([0.01, 1.0, 30.0])).astype(np.float32)
        x.reshape(-1)[:: 97] = 0.0
        return x, (rng.standard_normal((t, h, d)) * 3).astype(np.float32)

    # single-token writes, repeatedly into the same block
    for _ in range(12):
        blk, off = int(rng.integers(0, nb)), int(rng.integers(0, 16))
        k, v = data(1)
        cache.write_kv(0, blk, off, to_dev(k[0]), to_dev(v[0]))
        ref.write(blk, off, k[0], v[0])
    # a batch walking across consecutive blocks
    k, v = data(37)
    cache.write_kv_batch(0, 3, 5, to_dev(k), to_dev(v))
    for t in range(37):
        ref.write(3 + (5 + t) // 16, (5 + t) % 16, k[t], v[t])
    # a prefill write with a non-contiguous table, several tokens per block
    ids = [7, 1, 9]
    pos = list(range(3, 40))
    k, v = data(len(pos))
    cache.write_prefill_kv(0, ids, pos, len(pos), to_dev(k), to_dev(v))
    for t, p in enumerate(pos):
        ref.write(ids[p // 16], p % 16, k[t], v[t])

    assert np.array_equal(bits(to_np(cache.scales(0))), bits(ref.s))
    assert np.array_equal(bits(to_np(cache.key_cache(0))), bits(ref.k))
    assert np.array_equal(bits(oracle.v_to_ref(to_np(cache.value_cache(0)))), bits(ref.v))
    blocks = [7, 1, 9, 3, 4, 5]
    rk, rv = cache.read_kv(0, blocks, 90)
    n, ok, ov = oracle.quant_read_kv(ref.k, ref.v, ref.s, blocks, 90)
    assert n == 90
    assert np.array_equal(bits(to_np(rk)), bits(ok))
    assert np.array_equal(bits(to_np(rv)), bits(ov))


def test_attention_over_quantised_cache(pa, oracle):
    rng = np.random.default_rng(3)
    hq, hkv, d, nb = 8, 2, 64, 24
    cache = pa.PagedKvCache(1, hkv, d, nb, torch.float32, DEV, quantized=True)
    ref = QuantOracle(oracle, hkv, d, nb)
    ctx = [40, 77, 5]
    perm = rng.permutation(nb)
    tables, o = [], 0
    for c in ctx:
        n = (c + 15) // 16
        tables.append([int(x) for x in perm[o:o + n]])
        o += n
        k = rng.standard_normal((c, hkv, d)).astype(np.float32)
        v = rng.standard_normal((c, hkv, d)).astype(np.float32)
        cache.write_prefill_kv(0, tables[-1], list(range(c)), c, to_dev(k), to_dev(v))
        for t in range(c):
            ref.write(tables[-1][t // 16], t % 16, k[t], v[t])
    mbs = max(len(t) for t in tables)
    bt = np.zeros((len(ctx), mbs), np.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t)] = t
    deq = lambda c: c * ref.s[:, None, None, None] + np.float32(0.0)
    kf, vf = deq(ref.k), deq(ref.v)
    # decode: the last token of each sequence
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    out = pa.decode(to_dev(q), cache.key_cache(0), cache.value_cache(0), to_dev(bt),
                    to_dev(np.asarray(ctx, np.int32)), max(ctx), block_scales=cache.scales(0))
    want = oracle.paged_attention(q, kf, vf, bt, np.arange(len(ctx) + 1, dtype=np.int32),
                                  np.asarray(ctx, np.int32) - 1)
    assert_close(to_np(out), want, F32_ATOL, F32_RTOL, "quantised decode")
    # prefill: the last 9 / 20 / 5 tokens of each sequence as a chunk
    chunks = [9, 20, 5]
    qp = rng.standard_normal((sum(chunks), hq, d)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    past = np.asarray([c - n for c, n in zip(ctx, chunks)], np.int32)
    outp = pa.prefill(to_dev(qp), cache.key_cache(0), cache.value_cache(0), to_dev(bt),
                      to_dev(cu), to_dev(past), max(chunks), block_scales=cache.scales(0))
    wantp = oracle.paged_attention(qp, kf, vf, bt, cu, past)
    assert_close(to_np(outp), wantp, F32_ATOL, F32_RTOL, "quantised prefill")
