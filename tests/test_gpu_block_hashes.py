"""GPU parity of the cache mirror's block-hash map (PagedKvCache::block_hashes,
crates/model/src/paged_tensor/tensor_store/mod.rs:42): every token a write
stores inserts hash(K block after that token) -> block_id
(tensor_store/buffer.rs:263-264).  The expected map is built by replaying
the same writes token by token on the oracle's caches (write_kv, or the
quantised write for quantised caches) and hashing the block with the
oracle's block_hash after each token, as the reference's per-token loops
(buffer.rs:27-95, paged_gqa.rs:29-63) do.  bit-exact (u64 keys, ids); the
caches' contents too (a prefill write naming one slot twice keeps the
later token, as the per-token loop does)."""
import numpy as np
import pytest
import torch

from test_gpu_cache_ops import DEV, to_dev

pytestmark = pytest.mark.gpu


class Reference:
    """Oracle caches of one layer and the expected map."""

    def __init__(self, oracle, nb, h, d, kind):
        self.o, self.kind = oracle, kind
        self.k = np.zeros((nb, h, 16, d), np.float32)
        self.v = np.zeros((nb, h, 16, d), np.float32)
        self.scales = np.ones(nb, np.float32)
        self.map = {}

    def token(self, block, off, k, v):
        if self.kind == "quant":
            assert self.o.quant_write_kv(self.k, self.v, self.scales, block, off, k, v) == 0
        else:
            assert self.o.write_kv(self.k, self.v, block, off, k, v) == 0
        self.map[self.o.block_hash(self.k[block])] = block


def payload(oracle, rng, t, h, d, kind):
    """Token rows [t, H, D]: device tensor in the cache dtype and the f32
    values the cache stores."""
    x = rng.standard_normal((t, h, d), dtype=np.float32)
    if kind == "bf16":
        b = oracle.f32_to_bf16(x)
        return to_dev(b), oracle.bf16_to_f32(b)
    return to_dev(x), x


@pytest.mark.parametrize("kind", ["f32", "bf16", "quant"])
def test_block_hash_map_follows_every_token(pa, oracle, kind):
    rng = np.random.default_rng({"f32": 1, "bf16": 2, "quant": 3}[kind])
    layers, h, d, nb = 2, 2, 64, 12
    dtype = torch.bfloat16 if kind == "bf16" else torch.float32
    cache = pa.PagedKvCache(layers, h, d, nb, dtype, DEV, quantized=kind == "quant")
    refs = [Reference(oracle, nb, h, d, kind) for _ in range(layers)]
    for step in range(14):
        layer = int(rng.integers(0, layers))
        ref = refs[layer]
        op = step % 3
        if op == 0:  # write_kv: one token
            blk, off = int(rng.integers(0, nb)), int(rng.integers(0, 16))
            (dk, k), (dv, v) = payload(oracle, rng, 1, h, d, kind), payload(oracle, rng, 1, h, d,
                                                                            kind)
            cache.write_kv(layer, blk, off, dk[0], dv[0])
            ref.token(blk, off, k[0], v[0])
        elif op == 1:  # write_kv_batch: a run from (blk, off) into the next blocks
            t = int(rng.integers(1, 40))
            blk, off = int(rng.integers(0, nb - 3)), int(rng.integers(0, 16))
            (dk, k), (dv, v) = payload(oracle, rng, t, h, d, kind), payload(oracle, rng, t, h, d,
                                                                            kind)
            cache.write_kv_batch(layer, blk, off, dk, dv)
            for i in range(t):
                ref.token(blk + (off + i) // 16, (off + i) % 16, k[i], v[i])
        else:  # write_prefill_kv: positions through a table, a position rewritten
            table = [int(x) for x in rng.permutation(nb)[:3]]
            t = int(rng.integers(2, 30))
            pos = [int(p) for p in rng.permutation(48)[:t]]
            pos[-1] = pos[0]  # the same slot twice in one call: the later token wins
            (dk, k), (dv, v) = payload(oracle, rng, t, h, d, kind), payload(oracle, rng, t, h, d,
                                                                            kind)
            cache.write_prefill_kv(layer, table, pos, t, dk, dv)
            for i, p in enumerate(pos):
                ref.token(table[p // 16], p % 16, k[i], v[i])
    for layer in range(layers):
        got = cache.block_hashes(layer)
        assert got == refs[layer].map, f"layer {layer}: {len(got)} vs {len(refs[layer].map)}"
        # the stored K of every block, as the oracle holds it
        kr, _ = cache.read_kv(layer, list(range(nb)), nb * 16)
        want = refs[layer].k.transpose(0, 2, 1, 3).reshape(nb * 16, h, d)
        if kind == "quant":
            want = want * np.repeat(refs[layer].scales, 16)[:, None, None] + 0.0
        assert np.array_equal(kr.float().cpu().numpy(), want)
    some = next(iter(refs[0].map.items()), None)
    if some is not None:
        assert cache.lookup_block_hash(0, some[0]) == some[1]
    absent = next(x for x in range(1, 1 << 20) if x not in refs[0].map)
    assert cache.lookup_block_hash(0, absent) is None
    with pytest.raises(pa.PaError, match="layer_idx"):
        cache.block_hashes(layers)
