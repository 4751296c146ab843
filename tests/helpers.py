"""Shared test helpers: fixture loading, scenario replay and tolerances."""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# bf16 attention bar: |gpu - ref| <= ATOL + RTOL * |ref| elementwise, with the
# reference computed in f32 from the same bf16-rounded inputs.
BF16_ATOL = 2e-2
BF16_RTOL = 1e-2
# f32 attention bar (the reference's own tests use 1e-4).
F32_ATOL = 1e-4
F32_RTOL = 1e-4


def golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def payload(op, key):
    """Float payload of an op as f32, from `key` or `key_bits`."""
    if key + "_bits" in op:
        return np.asarray(op[key + "_bits"], dtype=np.uint32).view(np.float32)
    return np.asarray(op[key], dtype=np.float32)


def expected(op, key):
    return payload(op, "expect_" + key)


def assert_close(got, ref, atol, rtol, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (
        f"{what}: {bad.sum()} / {bad.size} outside tol; max abs err {err.max():.3e} at "
        f"{np.unravel_index(err.argmax(), err.shape)}")


class OracleCache:
    """Scenario target backed by the C oracle (reference [NB, H, 16, D] layout)."""

    def __init__(self, oracle, num_layers, num_heads, head_dim, num_blocks):
        self.o = oracle
        self.h, self.d = num_heads, head_dim
        self.k = [np.zeros((num_blocks, num_heads, 16, head_dim), np.float32)
                  for _ in range(num_layers)]
        self.v = [np.zeros_like(self.k[0]) for _ in range(num_layers)]

    def _layer(self, layer):
        if not 0 <= layer < len(self.k):
            return None
        return self.k[layer], self.v[layer]

    def write_kv(self, layer, block_id, off, k, v):
        kv = self._layer(layer)
        if kv is None:
            return -2
        return self.o.write_kv(kv[0], kv[1], block_id, off, k, v)

    def write_kv_batch(self, layer, block_id, off, k, v):
        kv = self._layer(layer)
        if kv is None:
            return -2
        return self.o.write_kv_batch(kv[0], kv[1], block_id, off, k, v)

    def write_prefill_kv(self, layer, block_ids, positions, seq_len, k, v):
        kv = self._layer(layer)
        return self.o.write_prefill_kv(kv[0], kv[1], block_ids, positions, seq_len, k, v)

    def read_kv(self, layer, block_ids, seq_len):
        kv = self._layer(layer)
        n, k, v = self.o.read_kv(kv[0], kv[1], block_ids, seq_len)
        return k, v

    def read_block(self, layer, block_id):
        kv = self._layer(layer)
        return kv[0][block_id].ravel(), kv[1][block_id].ravel()


def replay(scenario, target):
    """Applies a kv_store_scenarios.json scenario to `target` and checks every
    expectation bit-exactly.  Targets return a nonzero code (or raise) on
    failure."""
    for i, op in enumerate(scenario["ops"]):
        kind = op["op"]
        where = f"{scenario['name']} op {i} ({kind})"
        if kind in ("write_kv", "write_kv_batch", "write_prefill_kv"):
            k, v = payload(op, "k"), payload(op, "v")
            try:
                if kind == "write_kv":
                    rc = target.write_kv(op["layer"], op["block_id"], op["token_offset"], k, v)
                elif kind == "write_kv_batch":
                    rc = target.write_kv_batch(op["layer"], op["block_id"], op["token_offset"],
                                               k, v)
                else:
                    rc = target.write_prefill_kv(op["layer"], op["block_ids"], op["positions"],
                                                 op["seq_len"], k, v)
                failed = rc not in (0, None)
            except Exception:
                failed = True
            assert failed == bool(op.get("expect_error", False)), where
        elif kind == "read_kv":
            k, v = target.read_kv(op["layer"], op["block_ids"], op["seq_len"])
            ek, ev = expected(op, "k"), expected(op, "v")
            assert np.array_equal(np.asarray(k, np.float32).ravel().view(np.uint32),
                                  ek.view(np.uint32)), where + " K"
            assert np.array_equal(np.asarray(v, np.float32).ravel().view(np.uint32),
                                  ev.view(np.uint32)), where + " V"
        elif kind == "read_block":
            k, v = target.read_block(op["layer"], op["block_id"])
            assert np.array_equal(np.asarray(k, np.float32).ravel(), expected(op, "k")), where
            assert np.array_equal(np.asarray(v, np.float32).ravel(), expected(op, "v")), where
        else:
            raise ValueError(kind)


def make_decode_case(rng, B, Hq, Hkv, D, ctx_lens, num_blocks=None, dtype="bf16",
                     kv_scale=1.0, shared_prefix_blocks=0):
    """Synthetic paged decode input.  Returns a dict of numpy arrays:
    q [B, Hq, D], k_cache / v_cache_ref [NB, Hkv, 16, D] (reference layout),
    block_tables [B, MBS] (a random permutation of the pool, optionally with
    the first `shared_prefix_blocks` entries shared by every sequence)."""
    ctx_lens = np.asarray(ctx_lens, np.int32)
    nblk = (ctx_lens + 15) // 16
    mbs = int(nblk.max())
    need = shared_prefix_blocks + int((nblk - shared_prefix_blocks).clip(min=0).sum())
    nb = num_blocks or need + 7
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.full((B, mbs), -1, np.int32)
    shared = perm[:shared_prefix_blocks]
    pos = shared_prefix_blocks
    for b in range(B):
        n = int(nblk[b])
        ns = min(shared_prefix_blocks, n)
        bt[b, :ns] = shared[:ns]
        bt[b, ns:n] = perm[pos:pos + n - ns]
        pos += n - ns
    q = rng.standard_normal((B, Hq, D), dtype=np.float32)
    k = (rng.standard_normal((nb, Hkv, 16, D), dtype=np.float32) * kv_scale)
    v = (rng.standard_normal((nb, Hkv, 16, D), dtype=np.float32) * kv_scale)
    if dtype == "bf16":
        import oracle
        q, k, v = oracle.f32_to_bf16(q), oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
    return {"q": q, "k_cache": k, "v_cache_ref": v, "block_tables": bt, "ctx": ctx_lens,
            "num_blocks": nb}
