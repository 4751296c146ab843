"""GPU parity of pa_decode against the oracle's paged attention.

bf16 cases run the MFMA kernel; f32 and unusual shapes run the generic
kernel.  Tolerances: bf16 |gpu - ref| <= 2e-2 + 1e-2 |ref| with the
reference computed in f32 from the same bf16 inputs; f32 1e-4 / 1e-4.
"""
import math

import numpy as np
import pytest
import torch

from helpers import (BF16_ATOL, BF16_RTOL, F32_ATOL, F32_RTOL, assert_close, golden,
                     make_decode_case)
from test_gpu_cache_ops import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu


def run_decode(pa, oracle, case, dtype, scale=None, check_split=True):
    q, kc, vc = case["q"], case["k_cache"], case["v_cache_ref"]
    bt, ctx = case["block_tables"], case["ctx"]
    B, Hq, D = q.shape
    scale = scale if scale is not None else 1.0 / math.sqrt(D)
    out = pa.decode(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt),
                    to_dev(ctx), int(ctx.max()), scale=scale)
    got = to_np(out)
    got = oracle.bf16_to_f32(got) if dtype == "bf16" else got
    ref = oracle.paged_attention(q, kc, vc, np.where(bt < 0, 0, bt), np.arange(B + 1),
                                 ctx - 1, scale=scale)
    ref = oracle.bf16_to_f32(ref) if dtype == "bf16" else ref
    return got, ref


def ref_f32(oracle, case, scale=None):
    """Reference on the same inputs but computed without bf16 output rounding."""
    q, kc, vc = case["q"], case["k_cache"], case["v_cache_ref"]
    B = q.shape[0]
    qf, kf, vf = (oracle.as_f32(x) for x in (q, kc, vc))
    return oracle.paged_attention(qf, kf, vf, np.where(case["block_tables"] < 0, 0,
                                                       case["block_tables"]),
                                  np.arange(B + 1), case["ctx"] - 1, scale=scale)


def test_config1_qwen_f32(pa, oracle):
    # B 8, Hq 14, Hkv 2, D 64, ctx ~ U[128, 1024], f32,
    # block tables = disjoint slices of a permutation of a 1024-block pool.
    rng = np.random.default_rng(0)
    ctx = rng.integers(128, 1025, size=8)
    case = make_decode_case(rng, 8, 14, 2, 64, ctx, num_blocks=1024, dtype="f32")
    got, ref = run_decode(pa, oracle, case, "f32")
    assert_close(got, ref, F32_ATOL, F32_RTOL, "config 1")


@pytest.mark.parametrize("b,hq,hkv,d", [(16, 32, 8, 128), (2, 16, 1, 64), (3, 8, 4, 32)])
def test_f32_group_partition_lengths(pa, oracle, b, hq, hkv, d):
    # The f32 group kernel takes 128-token partitions when 256-token ones
    # give fewer workgroups than CUs and the group has at most 8 heads:
    # B 16 x 8 kv heads x 4 partitions = 512 workgroups (256 tokens); a group
    # of 16 heads (256 tokens); 3 x 4 x up to 8 (128 tokens).
    rng = np.random.default_rng(b * 100 + hq)
    ctx = rng.integers(600, 1025, size=b)
    case = make_decode_case(rng, b, hq, hkv, d, ctx, dtype="f32")
    got, ref = run_decode(pa, oracle, case, "f32")
    assert_close(got, ref, F32_ATOL, F32_RTOL, f"f32 group {b}x{hq}/{hkv}x{d}")


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (8, 8, 128), (16, 2, 256),
                                      (8, 4, 64), (16, 1, 128)])
def test_bf16_mfma_shapes(pa, oracle, hq, hkv, d):
    rng = np.random.default_rng(hq * 10 + d)
    ctx = [1, 15, 16, 17, 31, 32, 33, 255, 256, 257, 600]
    case = make_decode_case(rng, len(ctx), hq, hkv, d, ctx, dtype="bf16", kv_scale=0.5)
    got, _ = run_decode(pa, oracle, case, "bf16")
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, f"bf16 {hq}/{hkv}x{d}")


def test_config2_llama_shape_small_batch(pa, oracle):
    # BASELINE config 2 shape (32/8 x 128, ctx 4096, K/V 0.5 N(0,1)) at B = 4.
    rng = np.random.default_rng(1)
    case = make_decode_case(rng, 4, 32, 8, 128, [4096] * 4, dtype="bf16", kv_scale=0.5)
    got, _ = run_decode(pa, oracle, case, "bf16")
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, "config 2 shape")


def test_config2_full_batch_long_partitions(pa, oracle):
    # BASELINE config 2 at full size (B 64, ctx 4096): the launch uses
    # 2048-token partitions.
    rng = np.random.default_rng(11)
    case = make_decode_case(rng, 64, 32, 8, 128, [4096] * 64, dtype="bf16", kv_scale=0.5)
    got, _ = run_decode(pa, oracle, case, "bf16")
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, "config 2 full")


@pytest.mark.parametrize("b,hkv,ctx_max,waves", [(32, 2, 760, 8), (2, 8, 1024, 8),
                                                 (32, 8, 900, 4), (16, 8, 1500, 1)])
def test_partitions_merged_in_workgroup(pa, oracle, b, hkv, ctx_max, waves):
    # decode launches whose partitions one workgroup merges in LDS: 128-token
    # partitions, up to 8 (small batches, contexts <= 1024: the engine's
    # decode step), 256-token partitions, up to 4; and more than 8 partitions
    # (the reduce kernel), all with ragged contexts including 1 and 128 / 129
    rng = np.random.default_rng(b * hkv + ctx_max)
    ctx = rng.integers(1, ctx_max + 1, size=b)
    ctx[0], ctx[1] = ctx_max, 1
    if b > 3:
        ctx[2], ctx[3] = 128, 129
    case = make_decode_case(rng, b, 4 * hkv, hkv, 128 if hkv == 8 else 64, ctx, dtype="bf16",
                            kv_scale=0.5)
    got, _ = run_decode(pa, oracle, case, "bf16")
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, f"merge {waves}")


def test_long_ragged_contexts_512_partitions(pa, oracle):
    # contexts past 8k with enough work items: 512-token partitions
    rng = np.random.default_rng(12)
    ctx = [9000, 8193, 5000, 1, 700, 8800, 9001, 4097]
    case = make_decode_case(rng, 8, 32, 8, 128, ctx, dtype="bf16")
    got, _ = run_decode(pa, oracle, case, "bf16")
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, "512 partitions")


def test_config4_shared_prefix_long_context(pa, oracle):
    # BASELINE config 4 pattern: log-uniform long contexts sharing a
    # 4096-token prefix (the same physical blocks in every table); B = 3.
    rng = np.random.default_rng(3)
    ctx = np.exp(rng.uniform(np.log(8192), np.log(32768), size=3)).astype(np.int32)
    case = make_decode_case(rng, 3, 32, 8, 128, ctx, dtype="bf16", shared_prefix_blocks=256)
    assert np.all(case["block_tables"][:, :256] == case["block_tables"][0, :256])
    got, _ = run_decode(pa, oracle, case, "bf16")
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, "config 4 pattern")


def test_config4_full_batch(pa, oracle):
    # BASELINE config 4 at full size: B 16, contexts log-uniform in
    # [8192, 32768] (seed 3), the first 256 blocks (4096 tokens) of every
    # table the same physical blocks, N(0, 1) K/V.  At this size the launch
    # runs 512-token partitions and decode_reduce_kernel merges up to 64
    # partitions per head.
    rng = np.random.default_rng(3)
    ctx = np.exp(rng.uniform(np.log(8192), np.log(32768), size=16)).astype(np.int32)
    case = make_decode_case(rng, 16, 32, 8, 128, ctx, dtype="bf16", shared_prefix_blocks=256)
    assert np.all(case["block_tables"][:, :256] == case["block_tables"][0, :256])
    out = pa.decode(to_dev(case["q"]), to_dev(case["k_cache"]),
                    to_dev(oracle.v_from_ref(case["v_cache_ref"])), to_dev(case["block_tables"]),
                    to_dev(ctx), int(ctx.max()), scale=1 / math.sqrt(128))
    got = oracle.bf16_to_f32(to_np(out))
    assert_close(got, ref_f32(oracle, case, scale=1 / math.sqrt(128)), BF16_ATOL, BF16_RTOL,
                 "config 4 full")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_split_equals_single_pass(pa, oracle, dtype):
    # A sequence long enough to split must match the same keys attended in
    # one partition: compare ctx = 256 (one pass) against the prefix of a
    # split launch by masking -- here via two independent launches.
    rng = np.random.default_rng(4)
    case = make_decode_case(rng, 2, 8, 2, 128, [256, 1000], dtype=dtype)
    got, ref = run_decode(pa, oracle, case, dtype)
    tol = (BF16_ATOL, BF16_RTOL) if dtype == "bf16" else (F32_ATOL, F32_RTOL)
    assert_close(got, ref_f32(oracle, case), *tol, "split")


def test_stale_nan_beyond_context_is_ignored(pa, oracle):
    # Cache slots past each context hold NaN; masking must keep them out.
    rng = np.random.default_rng(5)
    ctx = [5, 21, 300]
    case = make_decode_case(rng, 3, 8, 2, 128, ctx, dtype="bf16")
    kc, vc, bt = case["k_cache"], case["v_cache_ref"], case["block_tables"]
    for b, L in enumerate(ctx):
        last = bt[b, (L - 1) // 16]
        kc[last, :, (L - 1) % 16 + 1:, :] = 0x7FC0
        vc[last, :, (L - 1) % 16 + 1:, :] = 0x7FC0
    got, _ = run_decode(pa, oracle, case, "bf16")
    assert np.isfinite(got).all()
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, "stale NaN")


def test_gqa_grouping_single_key(pa, oracle):
    # util/tests.rs:316-339 on the GPU: one key, so out = V of the paired
    # kv head; blocked grouping [V0, V0, V1, V1].
    f = golden("attention_fixtures.json")["gqa_single_token"]
    for dtype, tdt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        d = 64  # padded head dim so both kernels run; extra dims zero
        kc, vc = pa.ops.new_cache(2, 2, d, tdt, DEV)
        v_ref = np.zeros((2, 2, 16, d), np.float32)
        v_ref[1, :, 0, :2] = np.asarray(f["v"], np.float32).reshape(2, 2)
        vc.copy_(torch.from_numpy(oracle.v_from_ref(v_ref)).to(tdt))
        q = torch.zeros(1, 4, d, dtype=tdt, device=DEV)
        out = pa.decode(q, kc, vc, torch.tensor([[1]], dtype=torch.int32, device=DEV),
                        torch.tensor([1], dtype=torch.int32, device=DEV), 1)
        got = out[0, :, :2].float().cpu().numpy().ravel().tolist()
        assert got == f["expect"], (dtype, got)


def test_scale_and_attn_factor(pa, oracle):
    # scale folds attn_factor / sqrt(D) (gqa/forward.rs:38-43)
    rng = np.random.default_rng(6)
    case = make_decode_case(rng, 2, 8, 2, 128, [100, 700], dtype="bf16")
    s = 1.7 / math.sqrt(128)
    got, _ = run_decode(pa, oracle, case, "bf16", scale=s)
    assert_close(got, ref_f32(oracle, case, scale=s), BF16_ATOL, BF16_RTOL, "scale")


def test_empty_context_gives_zeros(pa, oracle):
    kc, vc = pa.ops.new_cache(4, 2, 128, torch.bfloat16, DEV)
    q = torch.randn(2, 8, 128, device=DEV).to(torch.bfloat16)
    out = torch.full_like(q, 7.0)
    pa.decode(q, kc, vc, torch.tensor([[0], [1]], dtype=torch.int32, device=DEV),
              torch.tensor([0, 0], dtype=torch.int32, device=DEV), 0, out=out)
    # max_context_len 0 is a no-op launch: out untouched
    assert torch.all(out == 7.0)
    pa.decode(q, kc, vc, torch.tensor([[0], [1]], dtype=torch.int32, device=DEV),
              torch.tensor([0, 3], dtype=torch.int32, device=DEV), 3, out=out)
    assert torch.all(out[0] == 0)


@pytest.mark.parametrize("dtype,hq,hkv,d", [("bf16", 32, 8, 128), ("f32", 14, 2, 64)])
def test_ids_outside_pool_are_absent_keys(pa, oracle, dtype, hq, hkv, d):
    # A table entry outside [0, num_blocks) contributes no keys; decode
    # attention does not depend on key order, so the result equals attention
    # over the table without those entries and a context shorter by their
    # 16 keys each.
    rng = np.random.default_rng(5)
    case = make_decode_case(rng, 3, hq, hkv, d, [100, 300, 40], dtype=dtype)
    q, kc, vc = case["q"], case["k_cache"], case["v_cache_ref"]
    bt, ctx = case["block_tables"], case["ctx"]
    nb = kc.shape[0]
    drop = [{2, 4}, {0, 9, 10, 17}, set()]
    bad = bt.copy()
    for b, ds in enumerate(drop):
        for i, x in enumerate(sorted(ds)):
            bad[b, x] = nb + i if i % 2 else -1 - i
    out = pa.decode(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bad),
                    to_dev(ctx), int(ctx.max()))
    got = oracle.bf16_to_f32(to_np(out)) if dtype == "bf16" else to_np(out)
    rows = [[x for i, x in enumerate(bt[b]) if i not in drop[b]] for b in range(len(bt))]
    bt_c = np.zeros_like(bt)
    for b, r in enumerate(rows):
        bt_c[b, :len(r)] = r
    ctx_c = (ctx - 16 * np.asarray([len(ds) for ds in drop])).astype(np.int32)
    B = q.shape[0]
    ref = oracle.paged_attention(oracle.as_f32(q), oracle.as_f32(kc), oracle.as_f32(vc), bt_c,
                                 np.arange(B + 1), ctx_c - 1)
    assert np.isfinite(got).all()
    tol = (BF16_ATOL, BF16_RTOL) if dtype == "bf16" else (F32_ATOL, F32_RTOL)
    assert_close(got, ref, *tol, f"decode with out-of-pool ids {dtype} {hq}/{hkv}x{d}")


@pytest.mark.parametrize("hq,hkv,d,seed", [(32, 8, 128, 0), (8, 8, 64, 1), (16, 2, 256, 2),
                                           (28, 4, 128, 3)])
def test_balanced_split_ragged(pa, oracle, hq, hkv, d, seed):
    # Long, ragged contexts (the balanced split-K launch: the work cut
    # evenly over the wavefronts, a wavefront's range crossing sequence and
    # kv-head boundaries): empty contexts, a single token, block edges and
    # long sequences side by side, more than 64 sequences.
    rng = np.random.default_rng(40 + seed)
    b = 70 if d <= 128 else 9
    ctx = rng.integers(1, 12000, b)
    ctx[::7] = rng.integers(9000, 16000, len(ctx[::7]))
    ctx[3], ctx[5], ctx[8] = 0, 1, 32
    case = make_decode_case(rng, b, hq, hkv, d, np.maximum(ctx, 1), dtype="bf16")
    case["ctx"] = ctx.astype(np.int32)
    out = pa.decode(to_dev(case["q"]), to_dev(case["k_cache"]),
                    to_dev(oracle.v_from_ref(case["v_cache_ref"])), to_dev(case["block_tables"]),
                    to_dev(case["ctx"]), int(ctx.max()))
    got = oracle.bf16_to_f32(to_np(out))
    live = ctx > 0
    ref = np.zeros_like(got)
    sub = {k: (v[live] if k in ("q", "block_tables", "ctx") else v) for k, v in case.items()}
    ref[live] = ref_f32(oracle, sub)
    assert np.all(got[~live] == 0)
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, f"balanced {hq}/{hkv}x{d}")


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (8, 8, 64), (16, 8, 256),
                                      (16, 4, 128)])
def test_balanced_shared_prefix_groups(pa, oracle, hq, hkv, d):
    # Long contexts whose tables share prefixes in some sequence groups (the
    # balanced launch attends a group's common prefix once for all its
    # members): a 50-block prefix (odd: it ends inside a 2-block unit) shared
    # by most sequences, a member that diverges after 7 blocks, a member
    # shorter than the prefix, a group with nothing shared, and a
    # sequence count that leaves a partial last group.
    rng = np.random.default_rng(hq + hkv + d)
    b = 13
    ctx = rng.integers(3000, 9000, b).astype(np.int32)
    ctx[4] = 500          # shorter than the shared prefix
    case = make_decode_case(rng, b, hq, hkv, d, ctx, dtype="bf16", shared_prefix_blocks=50)
    bt = case["block_tables"]
    nb = case["num_blocks"]
    extra = rng.permutation(np.arange(nb, nb + 200)).astype(np.int32)
    bt[2, 7:50] = extra[:43]              # diverges after 7 blocks
    bt[9:12, :50] = extra[43:193].reshape(3, 50)  # a group without a common prefix
    grow = 200
    for key in ("k_cache", "v_cache_ref"):
        pad = rng.standard_normal((grow,) + case[key].shape[1:], dtype=np.float32)
        case[key] = np.concatenate([case[key], oracle.f32_to_bf16(pad)])
    out = pa.decode(to_dev(case["q"]), to_dev(case["k_cache"]),
                    to_dev(oracle.v_from_ref(case["v_cache_ref"])), to_dev(bt),
                    to_dev(ctx), int(ctx.max()))
    got = oracle.bf16_to_f32(to_np(out))
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL,
                 f"balanced shared prefix {hq}/{hkv}x{d}")


@pytest.mark.parametrize("seed", range(10))
def test_balanced_random_sweep(pa, oracle, seed):
    # Seeded random shapes on the balanced launch: group sizes 1-8, head
    # dims 64 / 128, up to 24 sequences of 1-6000 tokens, and block tables
    # whose prefixes are shared by random runs of sequences up to random
    # divergence points (some shorter than the shared part), against the
    # oracle.
    rng = np.random.default_rng(700 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 7, 8]))
    hq, d = hkv * g, int(rng.choice([64, 128]))
    b = int(rng.integers(2, 25))
    ctx = rng.integers(1, 6000, b).astype(np.int32)
    ctx[rng.integers(0, b)] = int(rng.integers(4200, 6000))   # at least one long row
    if b > 3:
        ctx[rng.integers(0, b)] = int(rng.integers(1, 40))    # and a short one
    prefix = int(rng.integers(0, 120))
    case = make_decode_case(rng, b, hq, hkv, d, ctx, dtype="bf16", shared_prefix_blocks=prefix)
    bt = case["block_tables"]
    nb = case["num_blocks"]
    # private copies of the prefix for some sequences, diverging at random
    extra = rng.permutation(np.arange(nb, nb + prefix * b + 1)).astype(np.int32)
    used = 0
    for s_ in range(b):
        if prefix and rng.random() < 0.3:
            cut = int(rng.integers(0, prefix))
            n = min(prefix, (int(ctx[s_]) + 15) // 16) - cut
            if n > 0:
                bt[s_, cut:cut + n] = extra[used:used + n]
                used += n
    grow = len(extra) if used else 0   # the pool grows by every id `extra` may hold
    if grow:
        for key in ("k_cache", "v_cache_ref"):
            pad = rng.standard_normal((grow,) + case[key].shape[1:], dtype=np.float32)
            case[key] = np.concatenate([case[key], oracle.f32_to_bf16(pad)])
    print(f"sweep seed {seed}: B {b}, {hq}/{hkv} x {d}, prefix {prefix}, max ctx {ctx.max()}",
          flush=True)
    out = pa.decode(to_dev(case["q"]), to_dev(case["k_cache"]),
                    to_dev(oracle.v_from_ref(case["v_cache_ref"])), to_dev(bt),
                    to_dev(ctx), int(ctx.max()))
    got = oracle.bf16_to_f32(to_np(out))
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, f"sweep seed {seed}")


def test_negative_context_in_shared_prefix_group(pa, oracle):
    """A negative context_lens entry (a caller error) inside a sequence
    group whose tables share a prefix: the group shares nothing, the row
    attends no keys (zeros, as a zero length does) and the other members
    match the oracle.  Before the common-prefix kernel clamped its result,
    -1000 gave a negative shared length, so every member of the group also
    attended the unit before its first token (the entry before its table
    row)."""
    rng = np.random.default_rng(91)
    ctx = np.array([5000, 7000, 6000, 4500, 8000, 3000], np.int32)
    case = make_decode_case(rng, len(ctx), 32, 8, 128, ctx, dtype="bf16",
                            shared_prefix_blocks=100)
    bad = ctx.copy()
    bad[0] = -1000  # first member of the first group (4 sequences at 4:1 GQA)
    out = pa.decode(to_dev(case["q"]), to_dev(case["k_cache"]),
                    to_dev(oracle.v_from_ref(case["v_cache_ref"])), to_dev(case["block_tables"]),
                    to_dev(bad), int(ctx.max()))
    got = oracle.bf16_to_f32(to_np(out))
    ref = ref_f32(oracle, case)
    assert np.all(got[0] == 0)
    assert_close(got[1:], ref[1:], BF16_ATOL, BF16_RTOL, "members beside a negative length")


def test_context_above_max_context_len_stays_in_bounds(pa, oracle):
    """A context_lens entry above the max_context_len argument (a caller
    error) must not write outside the workspace pa_decode_workspace_size
    sized for max_context_len: the balanced split-K launch clamps lengths to
    it.  The other sequences' results are unaffected; a canary after the
    sized workspace stays intact."""
    rng = np.random.default_rng(77)
    ctx = np.array([9000, 12000, 300, 5000], np.int32)
    case = make_decode_case(rng, len(ctx), 32, 8, 128, ctx, dtype="bf16", kv_scale=0.5)
    max_ctx = 6000  # below the first two sequences' lengths
    need = pa.ops.decode_workspace_size(len(ctx), 32, 128, max_ctx)
    assert need > 0
    ws = torch.full((need + 65536,), 0x5A, dtype=torch.uint8, device=DEV)
    out = pa.decode(to_dev(case["q"]), to_dev(case["k_cache"]),
                    to_dev(oracle.v_from_ref(case["v_cache_ref"])), to_dev(case["block_tables"]),
                    to_dev(ctx), max_ctx, workspace=ws)
    torch.cuda.synchronize()
    assert bool((ws[need:] == 0x5A).all()), "write past the sized workspace"
    got = oracle.bf16_to_f32(to_np(out))
    ref = oracle.bf16_to_f32(oracle.paged_attention(
        case["q"], case["k_cache"], case["v_cache_ref"],
        np.where(case["block_tables"] < 0, 0, case["block_tables"]), np.arange(len(ctx) + 1),
        ctx - 1, scale=1.0 / math.sqrt(128)))
    assert_close(got[2:], ref[2:], BF16_ATOL, BF16_RTOL, "sequences within max_context_len")
    assert np.isfinite(got[:2]).all()


def _balanced_groups(ws, b, hq, d, max_ctx):
    """The shared-prefix group record a balanced launch leaves in its
    workspace (after the b * hq * slots partial results): group count,
    members of each group (batch indices) and their shared 32-token units."""
    units = (max_ctx + 31) // 32
    slots = (units + 7) // 8 + 3
    off = b * hq * slots * (d + 2) * 4
    rec = ws[off:off + (6 * b + 2) * 4].cpu().numpy().view(np.int32)
    ng = int(rec[0])
    order, gstart, lcp = rec[1:1 + b], rec[1 + b:2 + 2 * b], rec[2 + 4 * b:2 + 5 * b]
    return [sorted(order[gstart[g]:gstart[g + 1]].tolist()) for g in range(ng)], lcp[:ng]


def test_config4_sharers_shuffled_among_private_sequences(pa, oracle):
    # Config 4's 16 sharers of a 4096-token prefix, randomly permuted and
    # interleaved with 8 sequences that share nothing: the groups of four
    # sharers (16 / G MFMA columns) must still form and attend the prefix
    # once, wherever the sharers sit in the batch.
    rng = np.random.default_rng(33)
    n_sh, n_pr = 16, 8
    ctx = np.exp(rng.uniform(np.log(8192), np.log(32768), size=n_sh + n_pr)).astype(np.int32)
    case = make_decode_case(rng, n_sh + n_pr, 32, 8, 128, ctx, dtype="bf16",
                            shared_prefix_blocks=256)
    bt = case["block_tables"]
    nb = case["num_blocks"]
    extra = rng.permutation(np.arange(nb, nb + 256 * n_pr)).astype(np.int32)
    bt[n_sh:, :256] = extra.reshape(n_pr, 256)          # private prefixes
    for key in ("k_cache", "v_cache_ref"):
        pad = rng.standard_normal((len(extra),) + case[key].shape[1:], dtype=np.float32)
        case[key] = np.concatenate([case[key], oracle.f32_to_bf16(pad)])
    perm = rng.permutation(n_sh + n_pr)
    for key in ("q", "block_tables", "ctx"):
        case[key] = np.ascontiguousarray(case[key][perm])
    b, max_ctx = n_sh + n_pr, int(case["ctx"].max())
    ws = torch.zeros(pa.decode_workspace_size(b, 32, 128, max_ctx), dtype=torch.uint8,
                     device=DEV)
    out = pa.decode(to_dev(case["q"]), to_dev(case["k_cache"]),
                    to_dev(oracle.v_from_ref(case["v_cache_ref"])),
                    to_dev(case["block_tables"]), to_dev(case["ctx"]), max_ctx, workspace=ws)
    got = oracle.bf16_to_f32(to_np(out))
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, "config 4 shuffled")
    groups, lcp = _balanced_groups(ws, b, 32, 128, max_ctx)
    sharers = set(np.nonzero(perm < n_sh)[0].tolist())
    shared_groups = [g for g in groups if len(g) > 1]
    assert sorted(sum(shared_groups, [])) == sorted(sharers)
    assert all(len(g) == 4 for g in shared_groups)
    assert all(l == 128 for g, l in zip(groups, lcp) if len(g) > 1)   # 4096 tokens


def test_balanced_row_needing_plus_three_slots(pa, oracle):
    # A layout whose row needs ceil(units / 8) + 3 partial-result slots (32 /
    # 8 x 128, contexts 4007 / 4096 / 1087, sequences 0 and 1 sharing 182
    # blocks): the slot sizing must hold it (the former + 2 sizing wrote one
    # slot past the row).
    rng = np.random.default_rng(19)
    ctx = np.array([4007, 4096, 1087], np.int32)
    case = make_decode_case(rng, 3, 32, 8, 128, ctx, dtype="bf16", shared_prefix_blocks=182)
    case["block_tables"][2, :68] = np.arange(case["num_blocks"], case["num_blocks"] + 68)
    for key in ("k_cache", "v_cache_ref"):
        pad = rng.standard_normal((68,) + case[key].shape[1:], dtype=np.float32)
        case[key] = np.concatenate([case[key], oracle.f32_to_bf16(pad)])
    got, _ = run_decode(pa, oracle, case, "bf16")
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, "plus-three slots")


def _host_groups(ctx, tables, g_):
    """The grouping decode_group_kernel forms, restated on the host: sequences
    with at least one full 32-token unit, ordered by (first block id, batch
    index), cut into runs of one first block and at most 16 / G members; a
    group's shared units are the common table prefix in whole units, capped
    by its shortest member."""
    b = len(ctx)
    none = 1 << 40
    keys = sorted(((int(tables[s, 0]) if ctx[s] // 32 > 0 else none), s) for s in range(b))
    groups, cur, prev = [], [], None
    for hi, s in keys:
        if cur and (hi == none or hi != prev or len(cur) == 16 // g_):
            groups.append(cur)
            cur = []
        cur.append(s)
        prev = hi
    groups.append(cur)
    out = {}
    for grp in groups:
        if len(grp) < 2:
            continue
        lim = min(int(ctx[s]) // 32 for s in grp)
        rows = tables[grp][:, :2 * lim]
        same = (rows == rows[0]).all(axis=0)
        diff = int(np.argmin(same)) if not same.all() else 2 * lim
        out[tuple(sorted(grp))] = min(lim, diff // 2)
    return out


@pytest.mark.parametrize("b", [1024, 1025])
def test_balanced_group_capacity_edge(pa, oracle, b):
    # The shared-prefix grouping handles up to 1024 sequences (one
    # workgroup per possible group); 1025 run ungrouped.  Tables from 30
    # prefix families (a random share of each family's 40 blocks, then
    # blocks drawn with repetition from a pool whose first blocks also
    # collide at random), contexts up to ~8300 so the balanced launch runs.
    rng = np.random.default_rng(5000 + b)
    hq, hkv, d = 2, 1, 64
    ctx = rng.integers(1, 3000, b).astype(np.int32)
    ctx[rng.choice(b, 6, replace=False)] = rng.integers(8200, 8400, 6)
    mbs = int((ctx.max() + 15) // 16)
    fam = rng.permutation(1200).astype(np.int32).reshape(30, 40)
    bt = rng.integers(1200, 3200, (b, mbs)).astype(np.int32)
    for s_ in range(b):
        if rng.random() < 0.6:
            n = int(rng.integers(1, 41))
            bt[s_, :n] = fam[rng.integers(0, 30), :n]
        bt[s_, (ctx[s_] + 15) // 16:] = -1
    q = oracle.f32_to_bf16(rng.standard_normal((b, hq, d), dtype=np.float32))
    kc = oracle.f32_to_bf16(rng.standard_normal((3200, hkv, 16, d), dtype=np.float32))
    vr = oracle.f32_to_bf16(rng.standard_normal((3200, hkv, 16, d), dtype=np.float32))
    case = {"q": q, "k_cache": kc, "v_cache_ref": vr, "block_tables": bt, "ctx": ctx,
            "num_blocks": 3200}
    max_ctx = int(ctx.max())
    print(f"group capacity edge: B {b}, max ctx {max_ctx}", flush=True)
    ws = torch.zeros(pa.decode_workspace_size(b, hq, d, max_ctx), dtype=torch.uint8, device=DEV)
    out = pa.decode(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vr)), to_dev(bt),
                    to_dev(ctx), max_ctx, workspace=ws)
    got = oracle.bf16_to_f32(to_np(out))
    assert_close(got, ref_f32(oracle, case), BF16_ATOL, BF16_RTOL, f"group capacity B {b}")
    if b <= 1024:
        groups, lcp = _balanced_groups(ws, b, hq, d, max_ctx)
        dev = {tuple(g): int(l) for g, l in zip(groups, lcp) if len(g) > 1}
        host = _host_groups(ctx, bt, hq // hkv)
        assert len(host) > 30 and dev == host
