"""GPU parity of the KV-cache write / read kernels: bit-exact against the
oracle and the reference's golden scenarios."""
import numpy as np
import pytest
import torch

from helpers import golden, replay

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def to_dev(a):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def to_np(t):
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


class GpuCache:
    """Scenario target backed by the C++ PagedKvCache mirror (f32)."""

    def __init__(self, pa, num_layers, num_heads, head_dim, num_blocks):
        self.c = pa.PagedKvCache(num_layers, num_heads, head_dim, num_blocks, torch.float32, DEV)
        self.h, self.d = num_heads, head_dim

    def _t(self, x):
        return to_dev(np.asarray(x, np.float32).reshape(-1, self.h, self.d))

    def write_kv(self, layer, block_id, off, k, v):
        self.c.write_kv(layer, block_id, off, self._t(k), self._t(v))

    def write_kv_batch(self, layer, block_id, off, k, v):
        self.c.write_kv_batch(layer, block_id, off, self._t(k), self._t(v))

    def write_prefill_kv(self, layer, block_ids, positions, seq_len, k, v):
        self.c.write_prefill_kv(layer, block_ids, positions, seq_len, self._t(k), self._t(v))

    def read_kv(self, layer, block_ids, seq_len):
        k, v = self.c.read_kv(layer, block_ids, seq_len)
        return to_np(k), to_np(v)

    def read_block(self, layer, block_id):
        k = self.c.key_cache(layer)[block_id]
        v = self.c.value_cache(layer)[block_id].transpose(-1, -2)
        return to_np(k.contiguous()).ravel(), to_np(v.contiguous()).ravel()


@pytest.mark.parametrize("scenario", golden("kv_store_scenarios.json"), ids=lambda s: s["name"])
def test_kv_cache_mirror_golden(pa, scenario):
    c = scenario["cache"]
    replay(scenario, GpuCache(pa, c["num_layers"], c["num_heads"], c["head_dim"],
                              c["num_blocks"]))
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("h,d", [(1, 1), (2, 4), (2, 64), (8, 128), (3, 40)])
def test_reshape_and_cache_bit_exact(pa, oracle, dtype, h, d):
    rng = np.random.default_rng(h * 1000 + d)
    nb, t = 9, 70
    k = rng.standard_normal((t, h, d), dtype=np.float32)
    v = rng.standard_normal((t, h, d), dtype=np.float32)
    if dtype == "bf16":
        k, v = oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
    slots = rng.permutation(nb * 16)[:t].astype(np.int64)
    slots[3], slots[11] = -1, nb * 16 + 5  # skipped
    kc = (rng.standard_normal((nb, h, 16, d), dtype=np.float32))
    vc = (rng.standard_normal((nb, h, 16, d), dtype=np.float32))
    if dtype == "bf16":
        kc, vc = oracle.f32_to_bf16(kc), oracle.f32_to_bf16(vc)
    gk, gv = to_dev(kc), to_dev(oracle.v_from_ref(vc))
    pa.reshape_and_cache(to_dev(k), to_dev(v), gk, gv, to_dev(slots))
    oracle.reshape_and_cache(k, v, kc, vc, slots)
    assert np.array_equal(to_np(gk), kc)
    assert np.array_equal(oracle.v_to_ref(to_np(gv)), vc)


def test_reshape_and_cache_strided_source(pa, oracle):
    # K and V as slices of a fused [T, 3, H, D] projection output
    rng = np.random.default_rng(7)
    t, h, d, nb = 33, 4, 64, 5
    qkv = oracle.f32_to_bf16(rng.standard_normal((t, 3, h, d), dtype=np.float32))
    g = to_dev(qkv)
    slots = rng.permutation(nb * 16)[:t].astype(np.int64)
    gk, gv = pa.ops.new_cache(nb, h, d, torch.bfloat16, DEV)
    pa.reshape_and_cache(g[:, 1], g[:, 2], gk, gv, to_dev(slots))
    kc = np.zeros((nb, h, 16, d), np.uint16)
    vc = np.zeros_like(kc)
    oracle.reshape_and_cache(qkv[:, 1], qkv[:, 2], kc, vc, slots)
    assert np.array_equal(to_np(gk), kc)
    assert np.array_equal(oracle.v_to_ref(to_np(gv)), vc)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_read_kv_bit_exact(pa, oracle, dtype):
    rng = np.random.default_rng(8)
    nb, h, d = 12, 2, 64
    kc = rng.standard_normal((nb, h, 16, d), dtype=np.float32)
    vc = rng.standard_normal((nb, h, 16, d), dtype=np.float32)
    if dtype == "bf16":
        kc, vc = oracle.f32_to_bf16(kc), oracle.f32_to_bf16(vc)
    ids = np.array([7, 2, 9, 0], np.int64)
    for seq_len in (1, 16, 17, 50, 64):
        gk, gv = pa.read_kv(to_dev(kc), to_dev(oracle.v_from_ref(vc)),
                            to_dev(ids.astype(np.int32)), seq_len)
        n, ok, ov = oracle.read_kv(kc, vc, ids, seq_len)
        assert n == seq_len
        assert np.array_equal(to_np(gk), ok) and np.array_equal(to_np(gv), ov)


def test_slot_mapping_matches_oracle(pa, oracle):
    rng = np.random.default_rng(9)
    nb, b = 40, 3
    lens = [5, 37, 16]
    bt = rng.permutation(nb).astype(np.int32)[: b * 3].reshape(b, 3)
    positions, cu = [], [0]
    for s, n in enumerate(lens):
        start = [0, 3, 30][s]
        positions += list(range(start, start + n))
        cu.append(cu[-1] + n)
    positions = np.array(positions, np.int64)
    got = to_np(pa.slot_mapping(to_dev(bt), to_dev(positions), to_dev(np.array(cu, np.int32))))
    want = np.concatenate([oracle.slot_mapping(bt[s], positions[cu[s]:cu[s + 1]], lens[s])
                           for s in range(b)])
    # positions past the table map to -1 here (the oracle's block-0 fallback
    # is the reference's; the device kernel skips instead)
    past_table = positions // 16 >= 3
    assert np.array_equal(got[~past_table], want[~past_table])
    assert np.all(got[past_table] == -1)


def test_block_hash(pa, oracle):
    f = golden("block_hash.json")
    rng = np.random.default_rng(10)
    nb, h, d = 6, 2, 32
    kc = rng.standard_normal((nb, h, 16, d), dtype=np.float32) * 3
    kc[2] = 0.0
    kc[3, 0, 0, :4] = [np.nan, np.inf, -1e30, 1e-6]
    ids = np.array([0, 3, 2, 5, 1], np.int32)
    got = to_np(pa.block_hash(to_dev(kc), to_dev(ids))).view(np.uint64)
    want = [oracle.block_hash(kc[i]) for i in ids]
    assert [int(x) for x in got] == want
    # the golden single-block case (1 head, D = 2, one block)
    case = f["cases"][-1]
    blk = np.asarray(case["bits"], np.uint32).view(np.float32).reshape(1, 1, 16, 2)
    got = to_np(pa.block_hash(to_dev(blk), to_dev(np.array([0], np.int32)))).view(np.uint64)
    assert int(got[0]) == int(case["expect"])


def prefill_slots(rng, nb, pasts, chunks):
    """slot_mapping of chunked-prefill rows: sequence s writes positions
    past_s .. past_s + chunk_s - 1 through its own random block table."""
    nblk = [(p + c + 15) // 16 for p, c in zip(pasts, chunks)]
    perm = rng.permutation(nb)
    assert sum(nblk) <= nb
    slots, o = [], 0
    for p, c, n in zip(pasts, chunks, nblk):
        table = perm[o:o + n]
        o += n
        pos = np.arange(p, p + c)
        slots.append(table[pos // 16] * 16 + pos % 16)
    return np.concatenate(slots).astype(np.int64)


# runs of consecutive slots: block-aligned and unaligned starts, chunks
# shorter than a block, a chunk ending mid-block, one slot skipped inside a
# run (its block then goes token by token)
PREFILL_CASES = [([0, 16, 37, 5, 130, 3], [64, 40, 130, 7, 77, 16]),
                 ([0, 0, 8], [15, 17, 300])]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
@pytest.mark.parametrize("h,d", [(8, 128), (2, 64), (1, 512), (3, 40)])
def test_reshape_and_cache_prefill_runs(pa, oracle, dtype, case, h, d):
    # the block-coalesced write path (whole blocks from runs of consecutive
    # slots) and the token-by-token path around it, bit-exact against the
    # oracle's per-token writes; untouched slots keep their contents
    rng = np.random.default_rng(case * 100 + h + d)
    pasts, chunks = PREFILL_CASES[case]
    nb = sum((p + c + 15) // 16 for p, c in zip(pasts, chunks)) + 6
    slots = prefill_slots(rng, nb, pasts, chunks)
    slots[50] = -1
    t = slots.size
    k = rng.standard_normal((t, h, d), dtype=np.float32)
    v = rng.standard_normal((t, h, d), dtype=np.float32)
    kc = rng.standard_normal((nb, h, 16, d), dtype=np.float32)
    vc = rng.standard_normal((nb, h, 16, d), dtype=np.float32)
    if dtype == "bf16":
        k, v, kc, vc = (oracle.f32_to_bf16(x) for x in (k, v, kc, vc))
    gk, gv = to_dev(kc), to_dev(oracle.v_from_ref(vc))
    pa.reshape_and_cache(to_dev(k), to_dev(v), gk, gv, to_dev(slots))
    oracle.reshape_and_cache(k, v, kc, vc, slots)
    assert np.array_equal(to_np(gk), kc)
    assert np.array_equal(oracle.v_to_ref(to_np(gv)), vc)


@pytest.mark.parametrize("src", ["f32", "bf16"])
def test_reshape_and_cache_fp8_prefill_runs(pa, oracle, src):
    rng = np.random.default_rng(31)
    h, d = 8, 128
    pasts, chunks = PREFILL_CASES[0]
    nb = sum((p + c + 15) // 16 for p, c in zip(pasts, chunks)) + 6
    slots = prefill_slots(rng, nb, pasts, chunks)
    t = slots.size
    k = rng.standard_normal((t, h, d), dtype=np.float32) * 3
    v = rng.standard_normal((t, h, d), dtype=np.float32)
    k[3, 0, :3] = [np.nan, np.inf, -np.inf]
    if src == "bf16":
        kb, vb = oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
        k, v = oracle.bf16_to_f32(kb), oracle.bf16_to_f32(vb)
        dk, dv = to_dev(kb), to_dev(vb)
    else:
        dk, dv = to_dev(k), to_dev(v)
    kc, vc = pa.ops.new_cache(nb, h, d, torch.uint8, DEV)
    pa.reshape_and_cache_fp8(dk, dv, kc, vc, to_dev(slots))
    want_k = np.zeros((nb, h, 16, d), np.uint8)
    want_v = np.zeros_like(want_k)
    kq, vq = oracle.fp8_encode(k), oracle.fp8_encode(v)
    for i, s in enumerate(slots):
        want_k[s // 16, :, s % 16, :] = kq[i]
        want_v[s // 16, :, s % 16, :] = vq[i]
    assert np.array_equal(to_np(kc), want_k)
    assert np.array_equal(oracle.v_to_ref(to_np(vc)), want_v)


def test_reshape_and_cache_config3_chunk_strided(pa, oracle):
    # BASELINE config 3's write: 4 x 2048 tokens on pasts 0 / 512 / 1024 /
    # 2048 (every run block-aligned), 8 kv heads x 128, K / V as strided
    # views of a fused projection output
    rng = np.random.default_rng(3)
    h, d = 8, 128
    pasts, chunks = [0, 512, 1024, 2048], [2048] * 4
    nb = sum((p + c + 15) // 16 for p, c in zip(pasts, chunks)) + 16
    slots = prefill_slots(rng, nb, pasts, chunks)
    t = slots.size
    kv = oracle.f32_to_bf16(rng.standard_normal((t, 3, h, d), dtype=np.float32))
    g = to_dev(kv)
    gk, gv = pa.ops.new_cache(nb, h, d, torch.bfloat16, DEV)
    pa.reshape_and_cache(g[:, 1], g[:, 2], gk, gv, to_dev(slots))
    kc = np.zeros((nb, h, 16, d), np.uint16)
    vc = np.zeros_like(kc)
    oracle.reshape_and_cache(kv[:, 1], kv[:, 2], kc, vc, slots)
    assert np.array_equal(to_np(gk), kc)
    assert np.array_equal(oracle.v_to_ref(to_np(gv)), vc)


def test_slot_mapping_offsets_past_num_tokens_stay_in_bounds(pa, oracle):
    """cu_seq_tokens claiming more tokens than num_tokens (a caller error):
    the kernel clamps the offsets, so nothing is written past slot_mapping
    and the tokens inside the call are mapped as usual."""
    rng = np.random.default_rng(10)
    bt = rng.permutation(40).astype(np.int32)[:6].reshape(2, 3)
    positions = np.arange(30, dtype=np.int64)
    cu = np.array([0, 20, 45], np.int32)  # 45 > the 30 tokens of the call
    big = torch.full((64,), 7777, dtype=torch.int64, device=DEV)
    lib = pa._lib.load()
    dbt, dpos, dcu = to_dev(bt), to_dev(positions), to_dev(cu)
    rc = lib.pa_slot_mapping(dbt.data_ptr(), 3, dpos.data_ptr(), dcu.data_ptr(), 2, 30,
                             big.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    got = to_np(big)
    assert np.all(got[30:] == 7777)
    want = np.concatenate([oracle.slot_mapping(bt[0], positions[:20], 20),
                           oracle.slot_mapping(bt[1], positions[20:30], 10)])
    assert np.array_equal(got[:30], want)
