"""Writes the golden fixtures under tests/golden/ from the reference's own
known-answer tests.

The reference (Rust + candle) cannot run in this image, so nothing here
executes it.  Each scenario restates one reference test: its inputs are the
test's inputs, and its expected outputs are the values the test asserts
(or, where the test only compares two paths, values fixed independently:
float64 numpy for attention, exact integer arithmetic for hashes and the
int8 grid).  Source citations are paths in the vllm-lite repository.

Run:  python tests/golden/make_golden.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def dump(name, obj):
    with open(os.path.join(HERE, name), "w") as f:
        json.dump(obj, f, sort_keys=True, separators=(",", ":"))
        f.write("\n")


def lcg_values(seed, n):
    """crates/model/src/paged_tensor/tensor_store/mod.rs:458-471:
    state = seed + 1; state = state * 1664525 + 1013904223 (u32 wrapping);
    f = (state as f32) * 1e-9 (f32 multiply).  Returned as f32 bit patterns."""
    state = (seed + 1) & 0xFFFFFFFF
    out = np.zeros(n, dtype=np.float32)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(state) * np.float32(1e-9)
    return [int(b) for b in out.view(np.uint32)]


def kv_scenarios():
    sc = []
    # paged_gqa.rs:269-313 — non-contiguous blocks [5, 9], K[i] = V[i] = i.
    vals = [float(i) for i in range(20)]
    b9 = [16.0, 17.0, 18.0, 19.0, 20.0] + [0.0] * 11
    sc.append({
        "name": "multi_block_roundtrip_non_contiguous",
        "source": "crates/model/src/components/attention/paged_gqa.rs:269-313",
        "cache": {"num_layers": 1, "num_heads": 1, "head_dim": 1, "num_blocks": 20},
        "ops": [
            {"op": "write_prefill_kv", "layer": 0, "block_ids": [5, 9],
             "positions": list(range(20)), "seq_len": 20, "k": vals, "v": vals},
            {"op": "read_kv", "layer": 0, "block_ids": [5, 9], "seq_len": 20,
             "expect_k": vals, "expect_v": vals},
            # decode token 20 -> block_ids[20 / 16] = 9, slot 20 % 16 = 4
            {"op": "write_prefill_kv", "layer": 0, "block_ids": [5, 9], "positions": [20],
             "seq_len": 1, "k": [20.0], "v": [20.0]},
            {"op": "read_kv", "layer": 0, "block_ids": [9], "seq_len": 16,
             "expect_k": b9, "expect_v": b9},
        ]})
    # tensor_store/mod.rs:333-368 — [head][token][dim] block layout.
    k_blk = [0.0] * 128
    v_blk = [0.0] * 128
    k_blk[0:4] = [1.0, 2.0, 3.0, 4.0]
    k_blk[64:68] = [5.0, 6.0, 7.0, 8.0]
    v_blk[0:4] = [10.0, 20.0, 30.0, 40.0]
    v_blk[64:68] = [50.0, 60.0, 70.0, 80.0]
    sc.append({
        "name": "block_layout_head_token_dim",
        "source": "crates/model/src/paged_tensor/tensor_store/mod.rs:333-368",
        "cache": {"num_layers": 2, "num_heads": 2, "head_dim": 4, "num_blocks": 4},
        "ops": [
            {"op": "write_kv", "layer": 0, "block_id": 0, "token_offset": 0,
             "k": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0],
             "v": [10.0, 20.0, 30.0, 40.0, 50.0, 60.0, 70.0, 80.0]},
            {"op": "read_block", "layer": 0, "block_id": 0, "expect_k": k_blk,
             "expect_v": v_blk},
            {"op": "read_block", "layer": 1, "block_id": 0, "expect_k": [0.0] * 128,
             "expect_v": [0.0] * 128},
        ]})
    # buffer/tests.rs:111-128 — headroom blocks beyond seq_len are ignored.
    sc.append({
        "name": "read_kv_headroom_blocks",
        "source": "crates/model/src/paged_tensor/tensor_store/buffer/tests.rs:111-128",
        "cache": {"num_layers": 1, "num_heads": 2, "head_dim": 4, "num_blocks": 4},
        "ops": [
            {"op": "write_kv_batch", "layer": 0, "block_id": 0, "token_offset": 0,
             "num_tokens": 4, "k": [1.0] * 32, "v": [1.0] * 32},
            {"op": "read_kv", "layer": 0, "block_ids": [0, 1], "seq_len": 4,
             "expect_k": [1.0] * 32, "expect_v": [1.0] * 32},
        ]})
    # buffer/tests.rs:442-510 — writes at num_blocks 64 stay in their block.
    exp5_k = [0.0] * (16 * 2 * 64)
    exp5_v = [0.0] * (16 * 2 * 64)
    for i in range(3 * 128, 4 * 128):
        exp5_k[i] = 7.5
        exp5_v[i] = 11.25
    exp7_k = [-3.0] * 128 + [0.0] * (15 * 128)
    exp7_v = [2.5] * 128 + [0.0] * (15 * 128)
    sc.append({
        "name": "write_kv_block_isolation_64_blocks",
        "source": "crates/model/src/paged_tensor/tensor_store/buffer/tests.rs:442-510",
        "cache": {"num_layers": 1, "num_heads": 2, "head_dim": 64, "num_blocks": 64},
        "ops": [
            {"op": "write_kv", "layer": 0, "block_id": 5, "token_offset": 3,
             "k": [7.5] * 128, "v": [11.25] * 128},
            {"op": "write_kv", "layer": 0, "block_id": 7, "token_offset": 0,
             "k": [-3.0] * 128, "v": [2.5] * 128},
            {"op": "read_kv", "layer": 0, "block_ids": [5], "seq_len": 16,
             "expect_k": exp5_k, "expect_v": exp5_v},
            {"op": "read_kv", "layer": 0, "block_ids": [7], "seq_len": 16,
             "expect_k": exp7_k, "expect_v": exp7_v},
        ]})
    # buffer/tests.rs:516-560 — a second write to the same block keeps slot 0.
    ek = [1.0] * 8 + [0.0] * 32 + [3.0] * 8 + [0.0] * (10 * 8)
    ev = [2.0] * 8 + [0.0] * 32 + [4.0] * 8 + [0.0] * (10 * 8)
    sc.append({
        "name": "write_kv_preserves_other_tokens",
        "source": "crates/model/src/paged_tensor/tensor_store/buffer/tests.rs:516-560",
        "cache": {"num_layers": 1, "num_heads": 2, "head_dim": 4, "num_blocks": 4},
        "ops": [
            {"op": "write_kv", "layer": 0, "block_id": 0, "token_offset": 0,
             "k": [1.0] * 8, "v": [2.0] * 8},
            {"op": "write_kv", "layer": 0, "block_id": 0, "token_offset": 5,
             "k": [3.0] * 8, "v": [4.0] * 8},
            {"op": "read_kv", "layer": 0, "block_ids": [0], "seq_len": 16,
             "expect_k": ek, "expect_v": ev},
        ]})
    # buffer/tests.rs:133-170, :370-383 — bounds errors.
    sc.append({
        "name": "write_bounds_errors",
        "source": "crates/model/src/paged_tensor/tensor_store/buffer/tests.rs:133-170,370-383",
        "cache": {"num_layers": 1, "num_heads": 2, "head_dim": 4, "num_blocks": 4},
        "ops": [
            {"op": "write_kv", "layer": 1, "block_id": 0, "token_offset": 0,
             "k": [1.0] * 8, "v": [1.0] * 8, "expect_error": True},
            {"op": "write_kv", "layer": 0, "block_id": 4, "token_offset": 0,
             "k": [1.0] * 8, "v": [1.0] * 8, "expect_error": True},
            {"op": "write_kv", "layer": 0, "block_id": 0, "token_offset": 16,
             "k": [1.0] * 8, "v": [1.0] * 8, "expect_error": True},
            {"op": "write_kv_batch", "layer": 0, "block_id": 3, "token_offset": 10,
             "num_tokens": 7, "k": [1.0] * 56, "v": [1.0] * 56, "expect_error": True},
            {"op": "read_kv", "layer": 0, "block_ids": [0], "seq_len": 16,
             "expect_k": [0.0] * 128, "expect_v": [0.0] * 128},
        ]})
    # tensor_store/mod.rs:458-483 — LCG payload, bit-exact round trip.
    kb = lcg_values(0xDEADBEEF, 32)
    vb = lcg_values(0xCAFEF00D, 32)
    sc.append({
        "name": "lcg_bit_exact_roundtrip",
        "source": "crates/model/src/paged_tensor/tensor_store/mod.rs:458-483",
        "cache": {"num_layers": 1, "num_heads": 1, "head_dim": 2, "num_blocks": 2},
        "ops": [
            {"op": "write_kv_batch", "layer": 0, "block_id": 1, "token_offset": 0,
             "num_tokens": 16, "k_bits": kb, "v_bits": vb},
            {"op": "read_kv", "layer": 0, "block_ids": [1], "seq_len": 16,
             "expect_k_bits": kb, "expect_v_bits": vb},
        ]})
    # buffer/tests.rs:354-368 — a batch run crossing into the next block
    # (the reference feeds randn; an LCG payload pins the same walk).
    kb = lcg_values(7, 20 * 2 * 8)
    vb = lcg_values(8, 20 * 2 * 8)
    sc.append({
        "name": "write_kv_batch_crosses_block_boundary",
        "source": "crates/model/src/paged_tensor/tensor_store/buffer/tests.rs:354-368",
        "cache": {"num_layers": 1, "num_heads": 2, "head_dim": 8, "num_blocks": 4},
        "ops": [
            {"op": "write_kv_batch", "layer": 0, "block_id": 0, "token_offset": 0,
             "num_tokens": 20, "k_bits": kb, "v_bits": vb},
            {"op": "read_kv", "layer": 0, "block_ids": [0, 1], "seq_len": 20,
             "expect_k_bits": kb, "expect_v_bits": vb},
        ]})
    # crates/model/tests/kv_write_path.rs:66-112 — blocks not given stay zero.
    kb = lcg_values(11, 20 * 4 * 32)
    sc.append({
        "name": "prefill_leaves_other_blocks_zero",
        "source": "crates/model/tests/kv_write_path.rs:66-112",
        "cache": {"num_layers": 2, "num_heads": 4, "head_dim": 32, "num_blocks": 4},
        "ops": [
            {"op": "write_prefill_kv", "layer": 0, "block_ids": [0, 1],
             "positions": list(range(20)), "seq_len": 20, "k_bits": kb, "v_bits": kb},
            {"op": "read_kv", "layer": 0, "block_ids": [0, 1], "seq_len": 20,
             "expect_k_bits": kb, "expect_v_bits": kb},
            {"op": "read_kv", "layer": 0, "block_ids": [2], "seq_len": 16,
             "expect_k": [0.0] * (16 * 128), "expect_v": [0.0] * (16 * 128)},
        ]})
    return sc


def naive_attention_f64(q, k, v, hq, hkv, seq, d):
    """Textbook masked softmax attention in float64, written independently of
    the oracle (crates/model/src/components/attention/util/tests.rs:347-392
    states the definition): head-first q [Hq, S, D], k/v [Hkv, S, D]."""
    q = np.asarray(q, np.float64).reshape(hq, seq, d)
    k = np.asarray(k, np.float64).reshape(hkv, seq, d)
    v = np.asarray(v, np.float64).reshape(hkv, seq, d)
    g = hq // hkv
    out = np.zeros((hq, seq, d))
    for h in range(hq):
        s = q[h] @ k[h // g].T / np.sqrt(d)
        s = np.where(np.tril(np.ones((seq, seq), bool)), s, -np.inf)
        e = np.exp(s - s.max(axis=1, keepdims=True))
        out[h] = (e / e.sum(axis=1, keepdims=True)) @ v[h // g]
    return out


def attention_fixtures():
    hq, hkv, seq, d = 4, 2, 3, 4
    q = [float((i * 7 + 3) % 11 - 5) for i in range(hq * seq * d)]
    k = [float((i * 5 + 1) % 9 - 4) for i in range(hkv * seq * d)]
    v = [float((i * 3 + 2) % 13 - 6) for i in range(hkv * seq * d)]
    expect = naive_attention_f64(q, k, v, hq, hkv, seq, d)
    return {
        "expand_kv_blocked": {
            "source": "crates/model/src/components/attention/util/tests.rs:296-313",
            "kv": [0.0, 1.0], "seq": 1, "num_kv_heads": 2, "num_q_heads": 8, "head_dim": 1,
            "expect": [0.0, 0.0, 0.0, 0.0, 1.0, 1.0, 1.0, 1.0]},
        "gqa_single_token": {
            "source": "crates/model/src/components/attention/util/tests.rs:316-339",
            "num_q_heads": 4, "num_kv_heads": 2, "head_dim": 2,
            "q": [0.0] * 8, "k": [0.0] * 4, "v": [1.0, 0.0, 0.0, 1.0],
            "expect": [1.0, 0.0, 1.0, 0.0, 0.0, 1.0, 0.0, 1.0]},
        "gqa_naive_reference": {
            "source": "crates/model/src/components/attention/util/tests.rs:394-458",
            "num_q_heads": hq, "num_kv_heads": hkv, "seq": seq, "head_dim": d,
            "layout": "head-first [H, S, D]", "tolerance": 1e-4,
            "q": q, "k": k, "v": v, "expect": [float(x) for x in expect.ravel()]},
    }


def rust_as_u64(x32):
    """`(x.abs() * 1000.0) as u64` with f32 arithmetic and Rust's saturating
    float -> int cast."""
    y = np.float32(abs(np.float32(x32))) * np.float32(1000.0)
    if np.isnan(y) or y <= 0:
        return 0
    if y >= np.float32(2.0 ** 64):
        return 2 ** 64 - 1
    return int(y)


def hash_fixtures():
    """crates/model/src/paged_tensor/tensor_store/layout.rs:51-58."""
    cases = [
        [1.0],
        [1.0, 2.0],
        [0.001, -0.002, 0.5],
        [float("nan"), 1.0e30, -0.0, 3.25],
        [1.0e19, 1.0e16, 0.0],
    ]
    out = []
    for data in cases:
        acc = 0
        for x in data:
            acc = (acc * 31 + rust_as_u64(x)) % (2 ** 64)
        bits = [int(b) for b in np.asarray(data, np.float32).view(np.uint32)]
        out.append({"bits": bits, "expect": str(acc)})
    # a 1-head, D=2 block of the LCG stream, the size a hash of a block sees
    bits = lcg_values(3, 32)
    data = np.asarray(bits, np.uint32).view(np.float32)
    acc = 0
    for x in data:
        acc = (acc * 31 + rust_as_u64(x)) % (2 ** 64)
    out.append({"bits": bits, "expect": str(acc)})
    return {"source": "crates/model/src/paged_tensor/tensor_store/layout.rs:51-58",
            "hand_checked": {"[1.0]": 1000, "[1.0, 2.0]": 1000 * 31 + 2000},
            "cases": out}


def quant_fixtures():
    """buffer.rs:184-231 closed form: scale = max(max|K|, max|V|) / 127,
    q = round(x / scale) (half away from zero), read = q * scale."""
    def round_half_away(x):
        return np.float32(np.sign(x) * np.floor(np.abs(x) + np.float32(0.5)))

    s = np.float32(20.0) / np.float32(127.0)
    kq = round_half_away(np.float32(10.0) / s)
    vq = round_half_away(np.float32(20.0) / s)
    return {
        "single_token": {
            "source": "crates/model/src/paged_tensor/tensor_store/buffer/tests.rs:198-222",
            "cache": {"num_heads": 2, "head_dim": 4, "num_blocks": 4},
            "k": [10.0] * 8, "v": [20.0] * 8,
            "expect_scale_bits": int(np.float32(s).view(np.uint32)),
            "expect_k_int": float(kq), "expect_v_int": float(vq),
            "expect_k_read_bits": int(np.float32(kq * s).view(np.uint32)),
            "tolerance_vs_input": 0.1},
        "per_block_scale": {
            "source": "crates/model/src/paged_tensor/tensor_store/buffer/tests.rs:284-320",
            "cache": {"num_heads": 1, "head_dim": 1, "num_blocks": 4},
            "block_ids": [0, 1], "values": [100.0] * 16 + [1.0] * 4,
            "tolerance_large": 5.0, "tolerance_small": 0.5},
    }


if __name__ == "__main__":
    dump("kv_store_scenarios.json", kv_scenarios())
    dump("attention_fixtures.json", attention_fixtures())
    dump("block_hash.json", hash_fixtures())
    dump("kv_quant.json", quant_fixtures())
    print("wrote fixtures to", HERE)
