"""GPU parity on cache pools past the 32-bit boundaries.

An MI355X holds 288 GB, so one layer's K (or V) cache can pass 2^31
elements and 4 GiB.  These tests place a case's blocks at the top of such a
pool and check every kernel family that reads or writes the cache there
against the oracle run on the same data in a small pool (block ids
remapped):
  * bf16, Hkv 8 x D 128: 139,264 blocks of 32 KB = 4.25 GiB per cache, so
    element offsets pass 2^31 and byte offsets pass 2^32;
  * FP8: the same block count at 16 KB per block, byte offsets past 2^31;
  * f32: 139,264 blocks of 64 KB (8.5 GiB per cache), element offsets past
    2^31 and byte offsets past 2^33.
Writes (bit-exact), read_kv (bit-exact), block hashes (bit-exact, f32), decode
(partitions merged in the workgroup, the balanced split-K kernel, FP8, f32)
and prefill (tiled bf16 and FP8, generic f32) are covered.  Pools are
allocated uninitialised: only the blocks a table names are ever read.
"""
import math

import numpy as np
import pytest
import torch

from helpers import (BF16_ATOL, BF16_RTOL, F32_ATOL, F32_RTOL, assert_close,
                     make_decode_case)
from test_gpu_cache_ops import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu

NB_BIG = (1 << 17) + 8192  # blocks per cache; the top 8192 start past 2^31 elements
HKV, D = 8, 128


def big_ids(small_nb):
    """Large-pool id of each small-pool id: spread over the top 2 * small_nb
    blocks, every one past the 2^31-element boundary of a bf16 pool."""
    ids = NB_BIG - 1 - 2 * np.arange(small_nb, dtype=np.int64)
    assert ids.min() * HKV * 16 * D > 2 ** 31
    return ids


def remap(bt, ids):
    return np.where(bt < 0, -1, ids[np.clip(bt, 0, None)]).astype(np.int32)


def big_pool(small_k, small_v_tm, dtype):
    """Uninitialised NB_BIG-block pool holding the small pool's blocks at big_ids."""
    nb = small_k.shape[0]
    ids = torch.from_numpy(big_ids(nb)).to(DEV)
    kc = torch.empty((NB_BIG, HKV, 16, D), dtype=dtype, device=DEV)
    vc = torch.empty((NB_BIG, HKV, D, 16), dtype=dtype, device=DEV)
    kc[ids] = to_dev(small_k).view(dtype)
    vc[ids] = to_dev(small_v_tm).view(dtype)
    return kc, vc


@pytest.fixture(autouse=True)
def _free():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("ctx_kind", ["merged", "balanced"])
def test_decode_bf16_past_2g_elements(pa, oracle, ctx_kind):
    rng = np.random.default_rng(11 if ctx_kind == "merged" else 12)
    # merged: partitions one workgroup merges; balanced: long ragged contexts
    # (more partitions than a workgroup merges) through the split-K kernel
    ctx = [1, 17, 300, 1500, 4096] if ctx_kind == "merged" else [9000, 33, 12345, 700]
    case = make_decode_case(rng, len(ctx), 32, HKV, D, ctx, dtype="bf16", kv_scale=0.5)
    ids = big_ids(case["num_blocks"])
    kc, vc = big_pool(case["k_cache"], oracle.v_from_ref(case["v_cache_ref"]), torch.bfloat16)
    bt = remap(case["block_tables"], ids)
    out = pa.decode(to_dev(case["q"]), kc, vc, to_dev(bt), to_dev(case["ctx"]),
                    int(max(ctx)))
    got = oracle.bf16_to_f32(to_np(out))
    B = len(ctx)
    ref = oracle.bf16_to_f32(oracle.paged_attention(
        case["q"], case["k_cache"], case["v_cache_ref"],
        np.where(case["block_tables"] < 0, 0, case["block_tables"]), np.arange(B + 1),
        case["ctx"] - 1, scale=1.0 / math.sqrt(D)))
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, f"large-pool decode ({ctx_kind})")


def test_decode_and_prefill_fp8_past_2g_bytes(pa, oracle):
    rng = np.random.default_rng(13)
    ctx = [5, 200, 2100, 4000]
    case = make_decode_case(rng, len(ctx), 32, HKV, D, ctx, dtype="f32", kv_scale=0.5)
    kcode = oracle.fp8_encode(case["k_cache"])
    vcode = oracle.fp8_encode(case["v_cache_ref"])
    kf, vf = oracle.fp8_decode(kcode), oracle.fp8_decode(vcode)
    ids = big_ids(case["num_blocks"])
    assert ids.min() * HKV * 16 * D > 2 ** 31  # byte offsets of an FP8 pool
    kc, vc = big_pool(kcode, oracle.v_from_ref(vcode), torch.uint8)
    bt = remap(case["block_tables"], ids)
    qb = oracle.f32_to_bf16(case["q"])
    qf = oracle.bf16_to_f32(qb)
    out = pa.decode(to_dev(qb), kc, vc, to_dev(bt), to_dev(case["ctx"]), int(max(ctx)))
    B = len(ctx)
    small_bt = np.where(case["block_tables"] < 0, 0, case["block_tables"])
    ref = oracle.bf16_to_f32(oracle.f32_to_bf16(oracle.paged_attention(
        qf, kf, vf, small_bt, np.arange(B + 1), case["ctx"] - 1, scale=1.0 / math.sqrt(D))))
    assert_close(oracle.bf16_to_f32(to_np(out)), ref, BF16_ATOL, BF16_RTOL,
                 "large-pool FP8 decode")

    # prefill: the last 130 tokens of each sequence as a chunk over the rest
    chunks = np.minimum(np.asarray(ctx), 130)
    pasts = np.asarray(ctx) - chunks
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    q = oracle.f32_to_bf16(rng.standard_normal((int(cu[-1]), 32, D), dtype=np.float32))
    out = pa.prefill(to_dev(q), kc, vc, to_dev(bt), to_dev(cu), to_dev(pasts.astype(np.int32)),
                     int(chunks.max()))
    ref = oracle.paged_attention(oracle.bf16_to_f32(q), kf, vf, small_bt, cu,
                                 pasts.astype(np.int32))
    assert_close(oracle.bf16_to_f32(to_np(out)), ref, BF16_ATOL, BF16_RTOL,
                 "large-pool FP8 prefill")


def test_prefill_bf16_past_2g_elements(pa, oracle):
    rng = np.random.default_rng(14)
    pasts, chunks = [0, 512, 1031, 3000], [300, 257, 64, 1000]
    tot = [p + c for p, c in zip(pasts, chunks)]
    case = make_decode_case(rng, len(tot), 32, HKV, D, tot, dtype="bf16")
    ids = big_ids(case["num_blocks"])
    kc, vc = big_pool(case["k_cache"], oracle.v_from_ref(case["v_cache_ref"]), torch.bfloat16)
    bt = remap(case["block_tables"], ids)
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    q = oracle.f32_to_bf16(rng.standard_normal((int(cu[-1]), 32, D), dtype=np.float32))
    past = np.asarray(pasts, np.int32)
    out = pa.prefill(to_dev(q), kc, vc, to_dev(bt), to_dev(cu), to_dev(past), max(chunks))
    ref = oracle.paged_attention(oracle.as_f32(q), oracle.as_f32(case["k_cache"]),
                                 oracle.as_f32(case["v_cache_ref"]),
                                 np.where(case["block_tables"] < 0, 0, case["block_tables"]),
                                 cu, past)
    assert_close(oracle.bf16_to_f32(to_np(out)), ref, BF16_ATOL, BF16_RTOL,
                 "large-pool bf16 prefill")


def test_f32_decode_and_prefill_past_8g_bytes(pa, oracle):
    rng = np.random.default_rng(15)
    ctx = [40, 700, 1025]
    case = make_decode_case(rng, len(ctx), 16, HKV, D, ctx, dtype="f32")
    ids = big_ids(case["num_blocks"])
    assert ids.min() * HKV * 16 * D * 4 > 2 ** 33
    kc, vc = big_pool(case["k_cache"], oracle.v_from_ref(case["v_cache_ref"]), torch.float32)
    bt = remap(case["block_tables"], ids)
    small_bt = np.where(case["block_tables"] < 0, 0, case["block_tables"])
    B = len(ctx)
    out = pa.decode(to_dev(case["q"]), kc, vc, to_dev(bt), to_dev(case["ctx"]), int(max(ctx)))
    ref = oracle.paged_attention(case["q"], case["k_cache"], case["v_cache_ref"], small_bt,
                                 np.arange(B + 1), case["ctx"] - 1, scale=1.0 / math.sqrt(D))
    assert_close(to_np(out), ref, F32_ATOL, F32_RTOL, "large-pool f32 decode")
    chunks = np.array([40, 33, 100])
    pasts = (np.asarray(ctx) - chunks).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    q = rng.standard_normal((int(cu[-1]), 16, D), dtype=np.float32)
    out = pa.prefill(to_dev(q), kc, vc, to_dev(bt), to_dev(cu), to_dev(pasts), 100)
    ref = oracle.paged_attention(q, case["k_cache"], case["v_cache_ref"], small_bt, cu, pasts)
    assert_close(to_np(out), ref, F32_ATOL, F32_RTOL, "large-pool f32 prefill")
    # block hashes of blocks past the boundary (defined on f32 caches)
    small = np.arange(min(case["num_blocks"], 40))
    got = to_np(pa.block_hash(kc, to_dev(ids[small].astype(np.int32)))).view(np.uint64)
    want = [oracle.block_hash(case["k_cache"][i]) for i in small]
    assert [int(x) for x in got] == want


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_write_read_past_2g_elements(pa, oracle, dtype):
    """The cache write (whole-block runs and single tokens) into blocks past
    the boundary, read back bit-exactly by indexing and by pa_read_kv."""
    rng = np.random.default_rng(16)
    t = 100
    k = rng.standard_normal((t, HKV, D), dtype=np.float32)
    v = rng.standard_normal((t, HKV, D), dtype=np.float32)
    ids = big_ids(8)
    # tokens 0-63: four whole blocks (the block-run path); 64-99: scattered
    slots = np.concatenate([ids[0] * 16 + np.arange(16), ids[3] * 16 + np.arange(16),
                            ids[1] * 16 + np.arange(16), ids[5] * 16 + np.arange(16),
                            ids[2] * 16 + rng.permutation(16)[:12],
                            ids[7] * 16 + rng.permutation(16)[:12],
                            ids[6] * 16 + rng.permutation(16)[:12]]).astype(np.int64)
    touched = [0, 3, 1, 5, 2, 7, 6]
    tdt = torch.bfloat16 if dtype == "bf16" else torch.uint8
    kc = torch.zeros((NB_BIG, HKV, 16, D), dtype=tdt, device=DEV)
    vc = torch.zeros((NB_BIG, HKV, D, 16), dtype=tdt, device=DEV)
    kb, vb = oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
    if dtype == "bf16":
        pa.reshape_and_cache(to_dev(kb), to_dev(vb), kc, vc, to_dev(slots))
        kcode, vcode = kb, vb
    else:
        pa.reshape_and_cache_fp8(to_dev(kb), to_dev(vb), kc, vc, to_dev(slots))
        kcode = oracle.fp8_encode(oracle.bf16_to_f32(kb))
        vcode = oracle.fp8_encode(oracle.bf16_to_f32(vb))
    nbs = len(touched)
    ref_k = np.zeros((nbs, HKV, 16, D), kcode.dtype)
    ref_v = np.zeros((nbs, HKV, 16, D), vcode.dtype)
    where = {int(ids[s]): i for i, s in enumerate(touched)}
    for i, s in enumerate(slots):
        ref_k[where[int(s // 16)], :, s % 16] = kcode[i]
        ref_v[where[int(s // 16)], :, s % 16] = vcode[i]
    big = torch.from_numpy(ids[touched]).to(DEV)
    got_k = to_np(kc[big]) if dtype == "bf16" else kc[big].cpu().numpy()
    got_v = to_np(vc[big]) if dtype == "bf16" else vc[big].cpu().numpy()
    assert np.array_equal(got_k, ref_k)
    assert np.array_equal(oracle.v_to_ref(got_v), ref_v)

    # pa_read_kv walks a table of those blocks (the last one partly read)
    seq_len = 16 * nbs - 5
    rk, rv = pa.read_kv(kc, vc, to_dev(ids[touched].astype(np.int32)), seq_len)
    tok_k = ref_k.transpose(0, 2, 1, 3).reshape(-1, HKV, D)[:seq_len]
    tok_v = ref_v.transpose(0, 2, 1, 3).reshape(-1, HKV, D)[:seq_len]
    if dtype == "bf16":
        assert np.array_equal(to_np(rk), tok_k) and np.array_equal(to_np(rv), tok_v)
    else:
        wk, wv = oracle.fp8_decode(tok_k), oracle.fp8_decode(tok_v)
        assert np.array_equal(to_np(rk).view(np.uint32), wk.view(np.uint32))
        assert np.array_equal(to_np(rv).view(np.uint32), wv.view(np.uint32))

