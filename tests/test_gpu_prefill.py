"""GPU parity of pa_prefill (chunked causal prefill over the paged cache)."""
import math

import numpy as np
import pytest
import torch

from helpers import BF16_ATOL, BF16_RTOL, F32_ATOL, F32_RTOL, assert_close
from test_gpu_cache_ops import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu


def make_prefill_case(oracle, rng, pasts, chunks, hq, hkv, d, dtype, extra_blocks=5):
    B = len(pasts)
    tot = [p + c for p, c in zip(pasts, chunks)]
    nblk = [(t + 15) // 16 for t in tot]
    mbs = max(nblk)
    nb = sum(nblk) + extra_blocks
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((B, mbs), np.int32)
    o = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
    kc = rng.standard_normal((nb, hkv, 16, d), dtype=np.float32)
    vc = rng.standard_normal((nb, hkv, 16, d), dtype=np.float32)
    q = rng.standard_normal((sum(chunks), hq, d), dtype=np.float32)
    if dtype == "bf16":
        q, kc, vc = oracle.f32_to_bf16(q), oracle.f32_to_bf16(kc), oracle.f32_to_bf16(vc)
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    return q, kc, vc, bt, cu, np.asarray(pasts, np.int32)


def run_prefill(pa, oracle, q, kc, vc, bt, cu, past, dtype):
    d = q.shape[-1]
    out = pa.prefill(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt),
                     to_dev(cu), to_dev(past), int(np.diff(cu).max()))
    got = to_np(out)
    if dtype == "bf16":
        got = oracle.bf16_to_f32(got)
    ref = oracle.paged_attention(oracle.as_f32(q), oracle.as_f32(kc), oracle.as_f32(vc), bt,
                                 cu, past)
    return got, ref


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (4, 4, 256), (8, 8, 128),
                                      (16, 8, 64), (16, 2, 128), (28, 4, 128), (12, 4, 64)])
def test_prefill_ragged(pa, oracle, dtype, hq, hkv, d):
    rng = np.random.default_rng(hq + d)
    pasts = [0, 16, 37, 5, 130]
    chunks = [1, 40, 130, 16, 77]
    case = make_prefill_case(oracle, rng, pasts, chunks, hq, hkv, d, dtype)
    got, ref = run_prefill(pa, oracle, *case, dtype)
    tol = (BF16_ATOL, BF16_RTOL) if dtype == "bf16" else (F32_ATOL, F32_RTOL)
    assert_close(got, ref, *tol, f"prefill {dtype} {hq}/{hkv}x{d}")


def test_config3_shape_reduced(pa, oracle):
    # BASELINE config 3 shape (32/8 x 128, past 0/512/1024/2048), chunk 256.
    rng = np.random.default_rng(2)
    case = make_prefill_case(oracle, rng, [0, 512, 1024, 2048], [256] * 4, 32, 8, 128, "bf16")
    got, ref = run_prefill(pa, oracle, *case, "bf16")
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, "config 3 reduced")


def test_chunked_equals_full_on_gpu(pa, oracle):
    # chunked prefill == one-shot prefill (layer_loop.rs:168-236), both on GPU
    rng = np.random.default_rng(3)
    q, kc, vc, bt, cu, past = make_prefill_case(oracle, rng, [0], [200], 8, 2, 128, "bf16")
    dk, dv, dbt = to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt)
    full = pa.prefill(to_dev(q), dk, dv, dbt, to_dev(cu), to_dev(past), 200)
    a = pa.prefill(to_dev(q[:77]), dk, dv, dbt, to_dev(np.array([0, 77], np.int32)),
                   to_dev(np.array([0], np.int32)), 77)
    b = pa.prefill(to_dev(q[77:]), dk, dv, dbt, to_dev(np.array([0, 123], np.int32)),
                   to_dev(np.array([77], np.int32)), 123)
    chunked = torch.cat([a, b]).float()
    assert_close(chunked.cpu().numpy(), full.float().cpu().numpy(), 1e-2, 1e-2, "chunked")


def test_decode_equals_last_prefill_row(pa, oracle):
    rng = np.random.default_rng(4)
    q, kc, vc, bt, cu, past = make_prefill_case(oracle, rng, [300], [50], 32, 8, 128, "bf16")
    dk, dv, dbt = to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt)
    pf = pa.prefill(to_dev(q), dk, dv, dbt, to_dev(cu), to_dev(past), 50)
    dec = pa.decode(to_dev(q[-1:]), dk, dv, dbt, to_dev(np.array([350], np.int32)), 350)
    assert_close(dec.float().cpu().numpy(), pf[-1:].float().cpu().numpy(), 1e-2, 1e-2,
                 "decode vs prefill")


def test_prefill_long_chunk_many_tiles(pa, oracle):
    # several 64-key LDS tiles, query tiles of every wavefront, ragged end
    rng = np.random.default_rng(5)
    case = make_prefill_case(oracle, rng, [0, 333], [700, 290], 32, 8, 128, "bf16")
    got, ref = run_prefill(pa, oracle, *case, "bf16")
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, "long chunk")


def test_prefill_stale_nan_beyond_context(pa, oracle):
    # keys past past+qlen in the last block hold NaN: must not leak
    rng = np.random.default_rng(6)
    q, kc, vc, bt, cu, past = make_prefill_case(oracle, rng, [7], [30], 8, 2, 128, "bf16")
    last = bt[0, (7 + 30 - 1) // 16]
    kc[last, :, (37 % 16):, :] = 0x7FC0
    vc[last, :, (37 % 16):, :] = 0x7FC0
    got, ref = run_prefill(pa, oracle, q, kc, vc, bt, cu, past, "bf16")
    assert np.isfinite(got).all()
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, "stale NaN")


def compact(bt, past, drop):
    """The table without the entries `drop[b]` (whole blocks of the past) and
    the past length without their 16 keys each."""
    rows = [[x for i, x in enumerate(bt[b]) if i not in drop[b]] for b in range(len(bt))]
    out = np.zeros_like(bt)
    for b, r in enumerate(rows):
        out[b, :len(r)] = r
    return out, (past - 16 * np.asarray([len(d) for d in drop])).astype(np.int32)


@pytest.mark.parametrize("dtype,hq,hkv,d", [("bf16", 32, 8, 128), ("bf16", 14, 2, 64),
                                            ("f32", 8, 2, 64)])
def test_prefill_ids_outside_pool_are_absent_keys(pa, oracle, dtype, hq, hkv, d):
    # A table entry outside [0, num_blocks) contributes no keys.  With such
    # entries only among the past blocks every query row sees all of them,
    # so the result equals attention over the table without those entries
    # and a past shorter by 16 keys per entry (key order and the causal
    # relation of the remaining keys are unchanged).
    rng = np.random.default_rng(d + hq)
    pasts, chunks = [200, 100, 0], [150, 33, 20]
    q, kc, vc, bt, cu, past = make_prefill_case(oracle, rng, pasts, chunks, hq, hkv, d, dtype)
    nb = kc.shape[0]
    drop = [{1, 5, 6}, {0}, set()]
    bad = bt.copy()
    bad[0, 1], bad[0, 5], bad[0, 6], bad[1, 0] = nb + 3, -1, nb, -7
    out = pa.prefill(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bad),
                     to_dev(cu), to_dev(past), int(np.diff(cu).max()))
    got = oracle.bf16_to_f32(to_np(out)) if dtype == "bf16" else to_np(out)
    bt_c, past_c = compact(bt, past, drop)
    ref = oracle.paged_attention(oracle.as_f32(q), oracle.as_f32(kc), oracle.as_f32(vc), bt_c,
                                 cu, past_c)
    assert np.isfinite(got).all()
    tol = (BF16_ATOL, BF16_RTOL) if dtype == "bf16" else (F32_ATOL, F32_RTOL)
    assert_close(got, ref, *tol, f"prefill with out-of-pool ids {dtype} {hq}/{hkv}x{d}")


def test_config3_full_size(pa, oracle):
    # BASELINE config 3 at full size: 4 x 2048 new tokens on past
    # 0 / 512 / 1024 / 2048, 32 / 8 x 128, bf16; the persistent grid's
    # rounds and snake order run exactly as in the benchmark.
    #  (1) Whole 64-row query tiles (a workgroup's tile) against the oracle:
    #      per sequence the first and the last tile and every eighth tile
    #      (offset by the sequence), 6 of its 32 tiles, so every diagonal
    #      position within the 64-key LDS tiles and both 32-row wavefront
    #      halves are covered; 1536 rows in all.  Each tile is a 64-row
    #      sequence with past P_s + 64 t over the same block table.
    #  (2) Every row against pa_decode over context P_s + i + 1 (the decode
    #      kernel is itself checked against the oracle): all 8192 x 32 rows.
    rng = np.random.default_rng(2)
    pasts, chunk = [0, 512, 1024, 2048], 2048
    q, kc, vc, bt, cu, past = make_prefill_case(oracle, rng, pasts, [chunk] * 4, 32, 8, 128,
                                                "bf16")
    dk, dv, dbt = to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt)
    out = pa.prefill(to_dev(q), dk, dv, dbt, to_dev(cu), to_dev(past), chunk)
    got = oracle.bf16_to_f32(to_np(out))

    tiles = []  # (sequence, tile)
    for s in range(4):
        pick = {0, chunk // 64 - 1} | {t for t in range(chunk // 64) if t % 8 == s + 1}
        tiles += [(s, t) for t in sorted(pick)]
    sel = np.concatenate([cu[s] + 64 * t + np.arange(64) for s, t in tiles])
    bt1 = bt[[s for s, _ in tiles]]
    past1 = np.array([pasts[s] + 64 * t for s, t in tiles], np.int32)
    ref = oracle.paged_attention(oracle.as_f32(q[sel]), oracle.as_f32(kc), oracle.as_f32(vc),
                                 bt1, np.arange(0, 64 * len(tiles) + 1, 64), past1,
                                 scale=1 / math.sqrt(128))
    assert len(sel) == 1536
    assert_close(got[sel], ref, BF16_ATOL, BF16_RTOL, "config 3 full, 64-row tiles vs oracle")

    seq = np.repeat(np.arange(4), chunk)
    ctx = (np.asarray(pasts)[seq] + np.tile(np.arange(chunk), 4) + 1).astype(np.int32)
    dec = pa.decode(to_dev(q), dk, dv,
                    to_dev(bt[seq]), to_dev(ctx), int(ctx.max()))
    assert_close(got, oracle.bf16_to_f32(to_np(dec)), 2e-2, 1e-2,
                 "config 3 full, all rows vs pa_decode")


@pytest.mark.parametrize("seed", range(8))
def test_prefill_random_sweep(pa, oracle, seed):
    # Seeded random shapes on the tiled kernel (bf16, D 64 / 128) and its
    # persistent schedule: group sizes 1-8 (head groups of at most four per
    # workgroup), 1-7 sequences with 1-400 new tokens on 0-800 past tokens,
    # every row against the oracle.
    rng = np.random.default_rng(900 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 3, 4, 7, 8]))
    hq, d = hkv * g, int(rng.choice([64, 128]))
    b = int(rng.integers(1, 8))
    chunks = [int(x) for x in rng.integers(1, 401, b)]
    pasts = [int(x) for x in rng.integers(0, 801, b)]
    if b > 2:
        pasts[0] = 0
    print(f"prefill sweep seed {seed}: {hq}/{hkv} x {d}, chunks {chunks}, pasts {pasts}",
          flush=True)
    case = make_prefill_case(oracle, rng, pasts, chunks, hq, hkv, d, "bf16")
    got, ref = run_prefill(pa, oracle, *case, "bf16")
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, f"prefill sweep seed {seed}")


@pytest.mark.parametrize("dtype,hq,hkv,d", [("bf16", 32, 8, 128), ("bf16", 4, 4, 256),
                                            ("f32", 8, 2, 64)])
def test_inconsistent_offsets_stay_in_bounds(pa, oracle, dtype, hq, hkv, d):
    """cu_q_lens past total_q and a sequence longer than max_q_len (caller
    errors): the kernels (tiled, D 256, generic) clamp the offsets, so
    nothing is written past `out`; a consistent sequence is unaffected."""
    rng = np.random.default_rng(hq + d + 5)
    q, kc, vc, bt, cu, past = make_prefill_case(oracle, rng, [37, 0], [50, 70], hq, hkv, d, dtype)
    total = 100  # the call owns 100 rows; the offsets claim 120
    canary = 3.0  # exact in bf16 and f32
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    big = torch.full((total + 40, hq, d), canary, dtype=tdt, device=DEV)
    out = big[:total]
    qd = to_dev(q)[:total]
    pa.prefill(qd, to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt), to_dev(cu),
               to_dev(past), 60, out=out)  # max_q_len 60 < the second sequence's 70
    torch.cuda.synchronize()
    assert bool((big[total:].float() == canary).all()), "write past out"
    got = to_np(out)[:50]
    if dtype == "bf16":
        got = oracle.bf16_to_f32(got)
    ref = oracle.paged_attention(oracle.as_f32(q[:50]), oracle.as_f32(kc), oracle.as_f32(vc),
                                 bt[:1], cu[:2], past[:1])
    tol = (BF16_ATOL, BF16_RTOL) if dtype == "bf16" else (F32_ATOL, F32_RTOL)
    assert_close(got, ref, *tol, "consistent sequence")


@pytest.mark.parametrize("dtype,hq,hkv,d", [("bf16", 32, 8, 128), ("bf16", 14, 2, 64),
                                            ("fp8", 32, 8, 128)])
def test_prefill_keys_past_64_tiles(pa, oracle, dtype, hq, hkv, d):
    """Items whose keys span more than 64 LDS tiles (4096 keys): the
    wavefront's block ids are loaded 64 tiles at a time, so pasts of 6000
    and 9000 keys cross one and two reloads."""
    rng = np.random.default_rng(d + hq)
    pasts, chunks = [6000, 9000, 100], [200, 65, 300]
    q, kc, vc, bt, cu, past = make_prefill_case(oracle, rng, pasts, chunks, hq, hkv, d,
                                                "f32" if dtype == "fp8" else dtype)
    if dtype == "fp8":
        kcode, vcode = oracle.fp8_encode(kc * 0.5), oracle.fp8_encode(vc * 0.5)
        qb = oracle.f32_to_bf16(q)
        out = pa.prefill(to_dev(qb), to_dev(kcode), to_dev(oracle.v_from_ref(vcode)), to_dev(bt),
                         to_dev(cu), to_dev(past), max(chunks))
        got = oracle.bf16_to_f32(to_np(out))
        ref = oracle.paged_attention(oracle.bf16_to_f32(qb), oracle.fp8_decode(kcode),
                                     oracle.fp8_decode(vcode), bt, cu, past)
    else:
        got, ref = run_prefill(pa, oracle, q, kc, vc, bt, cu, past, dtype)
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, f"prefill past 64 tiles {dtype} {hq}/{hkv}x{d}")
