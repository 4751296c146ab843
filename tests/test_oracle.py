"""Pins the C oracle (CPU) before it is trusted as the checker.

Every oracle function is checked against the reference's own known-answer
tests (golden fixtures) and against facts the mathematics fixes (closed
forms, invariants, an independent float64 implementation), chosen so that a
dropped term, a wrong index or a transposed operand fails at least one.
"""
import numpy as np
import pytest

from helpers import OracleCache, assert_close, golden, replay


@pytest.mark.parametrize("scenario", golden("kv_store_scenarios.json"), ids=lambda s: s["name"])
def test_kv_store_scenarios(oracle, scenario):
    c = scenario["cache"]
    replay(scenario, OracleCache(oracle, c["num_layers"], c["num_heads"], c["head_dim"],
                                 c["num_blocks"]))


def test_slot_mapping_closed_form(oracle):
    # block_ids[pos // 16] * 16 + pos % 16 over non-contiguous tables.
    ids = [7, 3, 11, 0]
    pos = np.arange(64)
    got = oracle.slot_mapping(ids, pos, 64)
    want = np.array([ids[p // 16] * 16 + p % 16 for p in range(64)])
    assert np.array_equal(got, want)
    # positions shorter than T fall back to the token index (paged_gqa.rs:40)
    got = oracle.slot_mapping(ids, [20], 3)
    assert list(got) == [3 * 16 + 4, 7 * 16 + 1, 7 * 16 + 2]
    # a missing table entry falls back to block 0 (paged_gqa.rs:51)
    assert list(oracle.slot_mapping([5], [16], 1)) == [0 * 16 + 0]


def test_reshape_and_cache_matches_write_kv(oracle):
    rng = np.random.default_rng(0)
    nb, h, d, t = 6, 3, 8, 40
    k = rng.standard_normal((t, h, d), dtype=np.float32)
    v = rng.standard_normal((t, h, d), dtype=np.float32)
    slots = rng.permutation(nb * 16)[:t].astype(np.int64)
    slots[5] = -1
    slots[9] = nb * 16  # out of range: skipped
    kc = np.zeros((nb, h, 16, d), np.float32)
    vc = np.zeros_like(kc)
    assert oracle.reshape_and_cache(k, v, kc, vc, slots) == 2
    kc2 = np.zeros_like(kc)
    vc2 = np.zeros_like(kc)
    for i, s in enumerate(slots):
        if 0 <= s < nb * 16:
            assert oracle.write_kv(kc2, vc2, int(s) // 16, int(s) % 16, k[i], v[i]) == 0
            # and the slot holds exactly the token (index arithmetic pinned)
            assert np.array_equal(kc[s // 16, :, s % 16, :], k[i])
            assert np.array_equal(vc[s // 16, :, s % 16, :], v[i])
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)


def test_bf16_copy_is_bit_exact(oracle):
    rng = np.random.default_rng(1)
    k = oracle.f32_to_bf16(rng.standard_normal((5, 2, 16), dtype=np.float32))
    kc = np.zeros((4, 2, 16, 16), np.uint16)
    vc = np.zeros_like(kc)
    assert oracle.write_kv_batch(kc, vc, 1, 3, k, k) == 0
    n, rk, rv = oracle.read_kv(kc, vc, [1], 8)
    assert n == 8
    assert np.array_equal(rk[3:8], k) and np.array_equal(rv[3:8], k)


def test_bf16_rounding_known_values(oracle):
    # 1.0 = 0x3F80, pi -> 0x4049 (3.140625), round-to-even ties, NaN stays NaN.
    x = np.array([1.0, np.pi, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, np.nan], np.float32)
    b = oracle.f32_to_bf16(x)
    assert list(b[:4]) == [0x3F80, 0x4049, 0x3F80, 0x3F82]
    assert np.isnan(oracle.bf16_to_f32(b[4:]))[0]


def test_expand_kv_blocked(oracle):
    f = golden("attention_fixtures.json")["expand_kv_blocked"]
    kv = np.asarray(f["kv"], np.float32).reshape(f["seq"], f["num_kv_heads"], f["head_dim"])
    out = oracle.expand_kv(kv, f["num_q_heads"])
    assert out.ravel().tolist() == f["expect"]


def test_gqa_single_token_outputs_v(oracle):
    f = golden("attention_fixtures.json")["gqa_single_token"]
    hq, hkv, d = f["num_q_heads"], f["num_kv_heads"], f["head_dim"]
    q = np.asarray(f["q"], np.float32).reshape(1, hq, d)
    k = np.asarray(f["k"], np.float32).reshape(1, hkv, d)
    v = np.asarray(f["v"], np.float32).reshape(1, hkv, d)
    out = oracle.attention(q, k, v, past=0)
    assert out.ravel().tolist() == f["expect"]


def test_gqa_naive_reference_fixture(oracle):
    f = golden("attention_fixtures.json")["gqa_naive_reference"]
    hq, hkv, s, d = f["num_q_heads"], f["num_kv_heads"], f["seq"], f["head_dim"]
    # fixture is head-first [H, S, D]; the oracle takes token-major [S, H, D]
    q = np.asarray(f["q"], np.float32).reshape(hq, s, d).transpose(1, 0, 2)
    k = np.asarray(f["k"], np.float32).reshape(hkv, s, d).transpose(1, 0, 2)
    v = np.asarray(f["v"], np.float32).reshape(hkv, s, d).transpose(1, 0, 2)
    want = np.asarray(f["expect"]).reshape(hq, s, d).transpose(1, 0, 2)
    for f64 in (False, True):
        out = oracle.attention(q, k, v, past=0, f64=f64)
        assert_close(out, want, f["tolerance"], 0, "naive GQA fixture")


def test_uniform_keys_give_mean_of_values(oracle):
    rng = np.random.default_rng(2)
    L, hq, hkv, d = 37, 6, 2, 16
    q = rng.standard_normal((1, hq, d), dtype=np.float32)
    k = np.tile(rng.standard_normal((1, hkv, d), dtype=np.float32), (L, 1, 1))
    v = rng.standard_normal((L, hkv, d), dtype=np.float32)
    out = oracle.attention(q, k, v, past=L - 1)
    want = np.repeat(v.mean(axis=0), hq // hkv, axis=0)[None]
    assert_close(out, want, 1e-5, 1e-5, "uniform keys")


def test_mask_and_scale_against_independent_f64(oracle):
    # Independent numpy float64 restatement with a rectangular (chunked) mask.
    rng = np.random.default_rng(3)
    past, C, hq, hkv, d = 11, 9, 8, 2, 32
    q = rng.standard_normal((C, hq, d), dtype=np.float32)
    k = rng.standard_normal((past + C, hkv, d), dtype=np.float32)
    v = rng.standard_normal((past + C, hkv, d), dtype=np.float32)
    out = oracle.attention(q, k, v, past=past)
    g = hq // hkv
    want = np.zeros((C, hq, d))
    for h in range(hq):
        s = q[:, h, :].astype(np.float64) @ k[:, h // g, :].T.astype(np.float64) / np.sqrt(d)
        keep = np.arange(past + C)[None, :] <= (past + np.arange(C))[:, None]
        s = np.where(keep, s, -np.inf)
        p = np.exp(s - s.max(1, keepdims=True))
        want[:, h, :] = (p / p.sum(1, keepdims=True)) @ v[:, h // g, :].astype(np.float64)
    assert_close(out, want, 1e-5, 1e-5, "chunked mask vs f64")
    # a transposed mask (j >= past + i) or a missing scale fails this bar
    bad = oracle.attention(q, k, v, past=past, scale=1.0)
    assert np.abs(bad - want).max() > 1e-2


def test_chunked_equals_full_prefill(oracle):
    # crates/model/src/causal_lm/layer_loop.rs:168-236: chunked == full.
    rng = np.random.default_rng(4)
    T, hq, hkv, d = 40, 4, 2, 8
    q = rng.standard_normal((T, hq, d), dtype=np.float32)
    k = rng.standard_normal((T, hkv, d), dtype=np.float32)
    v = rng.standard_normal((T, hkv, d), dtype=np.float32)
    full = oracle.attention(q, k, v, past=0)
    first = oracle.attention(q[:17], k[:17], v[:17], past=0)
    second = oracle.attention(q[17:], k, v, past=17)
    assert_close(np.concatenate([first, second]), full, 1e-6, 1e-6, "chunked")
    # decode of the last token == last prefill row
    last = oracle.attention(q[-1:], k, v, past=T - 1)
    assert_close(last, full[-1:], 1e-6, 1e-6, "decode row")


def test_paged_attention_equals_dense(oracle):
    # gather through a shuffled block table == dense attention on the tokens
    rng = np.random.default_rng(5)
    hq, hkv, d, nb = 4, 2, 16, 12
    ctx = [5, 33, 16]
    kc = rng.standard_normal((nb, hkv, 16, d), dtype=np.float32)
    vc = rng.standard_normal((nb, hkv, 16, d), dtype=np.float32)
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.full((3, 3), -1, np.int32)
    bt[0, :1], bt[1, :3], bt[2, :1] = perm[0:1], perm[1:4], perm[4:5]
    q = rng.standard_normal((3, hq, d), dtype=np.float32)
    out = oracle.paged_attention(q, kc, vc, bt, [0, 1, 2, 3], [c - 1 for c in ctx])
    for b, L in enumerate(ctx):
        ids = [int(x) for x in bt[b] if x >= 0]
        n, kd, vd = oracle.read_kv(kc, vc, ids, L)
        assert n == L
        want = oracle.attention(q[b:b + 1], kd, vd, past=L - 1)
        assert_close(out[b:b + 1], want, 1e-6, 1e-6, "paged vs dense")
    # f64 mode agrees with f32
    out64 = oracle.paged_attention(q, kc, vc, bt, [0, 1, 2, 3], [c - 1 for c in ctx], f64=True)
    assert_close(out, out64, 1e-5, 1e-5, "f32 vs f64")


def test_block_hash_fixtures(oracle):
    f = golden("block_hash.json")
    assert oracle.block_hash(np.array([1.0], np.float32)) == f["hand_checked"]["[1.0]"]
    assert oracle.block_hash(np.array([1.0, 2.0], np.float32)) == f["hand_checked"]["[1.0, 2.0]"]
    for case in f["cases"]:
        data = np.asarray(case["bits"], np.uint32).view(np.float32)
        assert oracle.block_hash(data) == int(case["expect"])


def test_quant_single_token_closed_form(oracle):
    f = golden("kv_quant.json")["single_token"]
    c = f["cache"]
    kc = np.zeros((c["num_blocks"], c["num_heads"], 16, c["head_dim"]), np.float32)
    vc = np.zeros_like(kc)
    scales = np.ones(c["num_blocks"], np.float32)
    k = np.asarray(f["k"], np.float32)
    v = np.asarray(f["v"], np.float32)
    assert oracle.quant_write_kv(kc, vc, scales, 0, 0, k, v) == 0
    assert scales[0].view(np.uint32) == f["expect_scale_bits"]
    assert np.all(kc[0, :, 0, :] == f["expect_k_int"]) and np.all(vc[0, :, 0, :] == f["expect_v_int"])
    n, rk, rv = oracle.quant_read_kv(kc, vc, scales, [0], 1)
    assert n == 1
    assert np.all(rk.view(np.uint32) == f["expect_k_read_bits"])
    assert np.abs(rk - 10.0).max() < f["tolerance_vs_input"]
    assert np.abs(rv - 20.0).max() < f["tolerance_vs_input"]


def test_quant_per_block_scale(oracle):
    f = golden("kv_quant.json")["per_block_scale"]
    c = f["cache"]
    kc = np.zeros((c["num_blocks"], 1, 16, 1), np.float32)
    vc = np.zeros_like(kc)
    scales = np.ones(c["num_blocks"], np.float32)
    vals = np.asarray(f["values"], np.float32)
    for t, x in enumerate(vals):
        blk = f["block_ids"][t // 16]
        assert oracle.quant_write_kv(kc, vc, scales, blk, t % 16, x[None], x[None]) == 0
    n, rk, rv = oracle.quant_read_kv(kc, vc, scales, f["block_ids"], len(vals))
    assert n == len(vals)
    for t, x in enumerate(vals):
        tol = f["tolerance_large"] if x > 50 else f["tolerance_small"]
        assert abs(rk[t, 0, 0] - x) < tol and abs(rv[t, 0, 0] - x) < tol
    # values sit on the int8 grid of their own block's scale
    assert np.all(np.abs(kc) <= 127) and np.all(kc == np.round(kc))


def test_quant_read_is_affine_plus_zero(oracle):
    # buffer.rs:320-331 reads a quantised block through candle's
    # affine(scale, 0.0): x * scale + 0.0, so a stored -0 (round(-0.3) in the
    # write) reads back as +0
    kc = np.zeros((1, 1, 16, 2), np.float32)
    vc = np.zeros_like(kc)
    scales = np.ones(1, np.float32)
    k = np.array([[-0.3, 100.0]], np.float32)  # scale 100/127: -0.3 -> round(-0.38) = -0
    assert oracle.quant_write_kv(kc, vc, scales, 0, 0, k, k) == 0
    assert np.signbit(kc[0, 0, 0, 0]) and kc[0, 0, 0, 0] == 0.0
    n, rk, rv = oracle.quant_read_kv(kc, vc, scales, [0], 1)
    assert rk[0, 0, 0].view(np.uint32) == 0 and rk[0, 0, 1] == np.float32(127.0) * scales[0]


def test_argmax_logits_known_answers(oracle):
    # crates/traits/src/sampling.rs:468-490
    assert oracle.argmax_logits(np.array([1.0, 2.0, 3.0, 2.0, 1.0])) == 2
    assert oracle.argmax_logits(np.array([-3.0, -1.0, -2.0])) == 1
    assert oracle.argmax_logits(np.array([1.0, 1.0, 1.0, 1.0])) == 0
    assert oracle.argmax_logits(np.zeros(0, np.float32)) == 0
    assert oracle.argmax_logits(np.array([42.0])) == 0


def test_argmax_logits_against_numpy(oracle):
    # numpy's argmax takes the first maximum; with NaN mapped to -inf it is
    # the reference's fold (NaN never compares greater, all -inf gives 0)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((40, 1000)).astype(np.float32)
    x[1, 500] = x[1, 7] = x[1].max() + 1          # a tie: the first wins
    x[2, :] = np.nan
    x[3, :] = -np.inf
    x[4, ::3] = np.nan
    x[5, 0] = np.nan
    x[6, :] = 0.0
    x[6, 9] = -0.0                                 # -0 == +0: index 0 stays
    x[7, 999] = np.inf
    x[8] = np.round(x[8])                          # many ties
    expect = np.argmax(np.where(np.isnan(x), -np.inf, x), axis=1)
    np.testing.assert_array_equal(oracle.argmax_logits(x), expect)
