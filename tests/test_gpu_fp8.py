"""GPU parity of the FP8-E4M3 KV path (the reference's codes,
crates/model/src/components/kv_cache_fp8.rs): the quantising cache write is
bit-exact against the oracle encoder, read_kv against the oracle decoder, and
decode / prefill over FP8 caches match the oracle's attention over the
dequantised caches within the bf16 tolerance."""
import math

import numpy as np
import pytest
import torch

from helpers import BF16_ATOL, BF16_RTOL, assert_close, make_decode_case
from test_gpu_cache_ops import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu


def wide_values(rng, shape):
    """Magnitudes across and beyond the E4M3 range, exact ties, specials."""
    n = int(np.prod(shape))
    x = np.exp(rng.uniform(np.log(1e-5), np.log(2e3), n)).astype(np.float32)
    x *= rng.choice([-1.0, 1.0], n).astype(np.float32)
    k = n // 8
    grid = np.ldexp(1.0 + rng.integers(0, 8, k) / 8.0, rng.integers(-6, 8, k))
    x[:k] = (grid + np.ldexp(1.0 / 16.0, np.frexp(grid)[1] - 1)).astype(np.float32)  # ties
    specials = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1e-40, 240.0, 247.9, 248.0,
                         352.0, 1e30, 2.0 ** -6, 2.0 ** -6 * 0.99], np.float32)
    x[k:k + specials.size] = specials
    return x.reshape(shape)


def ref_scatter(codes, slots, nb):
    """Reference-layout scatter of per-token codes [T, H, D] (uint8)."""
    t, h, d = codes.shape
    cache = np.zeros((nb, h, 16, d), np.uint8)
    for i, s in enumerate(slots):
        if 0 <= s < nb * 16:
            cache[s // 16, :, s % 16, :] = codes[i]
    return cache


@pytest.mark.parametrize("src", ["f32", "bf16"])
@pytest.mark.parametrize("h,d", [(8, 128), (2, 64), (3, 40)])
def test_reshape_and_cache_fp8_bit_exact(pa, oracle, src, h, d):
    rng = np.random.default_rng(h * d)
    t, nb = 77, 12
    k = wide_values(rng, (t, h, d))
    v = wide_values(rng, (t, h, d))
    if src == "bf16":
        kb, vb = oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
        k, v = oracle.bf16_to_f32(kb), oracle.bf16_to_f32(vb)  # the values the GPU sees
        dk, dv = to_dev(kb), to_dev(vb)
    else:
        dk, dv = to_dev(k), to_dev(v)
    slots = rng.permutation(nb * 16)[:t].astype(np.int64)
    slots[3] = -1
    slots[9] = nb * 16
    kc, vc = pa.ops.new_cache(nb, h, d, torch.uint8, DEV)
    pa.reshape_and_cache_fp8(dk, dv, kc, vc, to_dev(slots))
    kref = ref_scatter(oracle.fp8_encode(k), slots, nb)
    vref = ref_scatter(oracle.fp8_encode(v), slots, nb)
    assert np.array_equal(to_np(kc), kref)
    assert np.array_equal(oracle.v_to_ref(to_np(vc)), vref)


def test_read_kv_fp8_every_code(pa, oracle):
    rng = np.random.default_rng(5)
    nb, h, d = 9, 2, 64
    kref = rng.integers(0, 256, (nb, h, 16, d)).astype(np.uint8)
    vref = rng.integers(0, 256, (nb, h, 16, d)).astype(np.uint8)
    kref.reshape(-1)[:256] = np.arange(256)
    ids = np.array([4, 0, 7, 2, 8], np.int32)
    seq_len = 70
    k, v = pa.read_kv(to_dev(kref), to_dev(oracle.v_from_ref(vref)), to_dev(ids), seq_len)
    want_k = oracle.fp8_decode(kref[ids].transpose(0, 2, 1, 3).reshape(-1, h, d)[:seq_len])
    want_v = oracle.fp8_decode(vref[ids].transpose(0, 2, 1, 3).reshape(-1, h, d)[:seq_len])
    got_k, got_v = to_np(k), to_np(v)
    # bit-exact, NaN codes included
    assert np.array_equal(got_k.view(np.uint32), want_k.view(np.uint32))
    assert np.array_equal(got_v.view(np.uint32), want_v.view(np.uint32))


def fp8_decode_case(oracle, rng, B, hq, hkv, d, ctx, shared=0):
    case = make_decode_case(rng, B, hq, hkv, d, ctx, dtype="bf16", shared_prefix_blocks=shared)
    kf = oracle.bf16_to_f32(case["k_cache"])
    vf = oracle.bf16_to_f32(case["v_cache_ref"])
    kc, vc = oracle.fp8_encode(kf), oracle.fp8_encode(vf)
    return case, kc, vc


def run_fp8_decode(pa, oracle, case, kc, vc):
    q, bt, ctx = case["q"], case["block_tables"], case["ctx"]
    out = pa.decode(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt),
                    to_dev(ctx), int(ctx.max()))
    got = oracle.bf16_to_f32(to_np(out))
    b = q.shape[0]
    qs = np.arange(b + 1, dtype=np.int32)
    past = (ctx - 1).astype(np.int32)
    ref = oracle.paged_attention(oracle.bf16_to_f32(q), oracle.fp8_decode(kc),
                                 oracle.fp8_decode(vc), np.where(bt < 0, 0, bt), qs, past)
    return got, ref


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (14, 2, 64), (8, 1, 256), (16, 16, 128),
                                      (28, 4, 64), (64, 4, 128), (12, 4, 96)])
def test_decode_fp8(pa, oracle, hq, hkv, d):
    # (64, 4): group 16; (12, 4, 96): the generic kernel
    rng = np.random.default_rng(hq * d)
    ctx = [1, 15, 16, 17, 33, 255, 256, 257, 700, 1500]
    case, kc, vc = fp8_decode_case(oracle, rng, len(ctx), hq, hkv, d, ctx)
    got, ref = run_fp8_decode(pa, oracle, case, kc, vc)
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, f"fp8 decode {hq}/{hkv}x{d}")


def test_decode_fp8_long_split_and_stale_codes(pa, oracle):
    rng = np.random.default_rng(9)
    ctx = [5000, 12003, 200]
    case, kc, vc = fp8_decode_case(oracle, rng, len(ctx), 32, 8, 128, ctx, shared=8)
    # codes past each context (in its last block) are 0x7F, NaN to the
    # hardware conversion; they must be masked, not multiplied by 0
    bt = case["block_tables"]
    for b, c in enumerate(ctx):
        last = bt[b, (c - 1) // 16]
        if c % 16 and (c - 1) // 16 >= 8:  # not a shared prefix block
            kc[last, :, c % 16:, :] = 0x7F
            vc[last, :, c % 16:, :] = 0x7F
    got, ref = run_fp8_decode(pa, oracle, case, kc, vc)
    assert np.isfinite(got).all()
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, "fp8 decode long")


def test_prefill_fp8(pa, oracle):
    rng = np.random.default_rng(11)
    hq, hkv, d = 8, 2, 128
    pasts, chunks = [0, 37, 100], [20, 45, 3]
    nblk = [(p + c + 15) // 16 for p, c in zip(pasts, chunks)]
    nb = sum(nblk) + 3
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((3, max(nblk)), np.int32)
    o = 0
    for b in range(3):
        bt[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
    kc = oracle.fp8_encode(rng.standard_normal((nb, hkv, 16, d), dtype=np.float32))
    vc = oracle.fp8_encode(rng.standard_normal((nb, hkv, 16, d), dtype=np.float32))
    q = oracle.f32_to_bf16(rng.standard_normal((sum(chunks), hq, d), dtype=np.float32))
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    past = np.asarray(pasts, np.int32)
    out = pa.prefill(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt),
                     to_dev(cu), to_dev(past), max(chunks))
    got = oracle.bf16_to_f32(to_np(out))
    ref = oracle.paged_attention(oracle.bf16_to_f32(q), oracle.fp8_decode(kc),
                                 oracle.fp8_decode(vc), bt, cu, past)
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, "fp8 prefill")


@pytest.mark.parametrize("hq,hkv,d,pasts,chunks", [
    (32, 8, 128, [0, 512, 130], [300, 200, 77]),   # config 3 heads, several tiles
    (14, 2, 64, [0, 37, 1000], [129, 64, 5]),
    (8, 8, 128, [16, 0], [1, 90]),
])
def test_prefill_fp8_tiled_shapes(pa, oracle, hq, hkv, d, pasts, chunks):
    # the LDS-tiled kernel on FP8 caches: K / V tiles copied as FP8 and
    # converted to bf16 per operand fragment
    rng = np.random.default_rng(hq * d + len(pasts))
    B = len(pasts)
    nblk = [(p + c + 15) // 16 for p, c in zip(pasts, chunks)]
    nb = sum(nblk) + 5
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((B, max(nblk)), np.int32)
    o = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
    kc = oracle.fp8_encode(rng.standard_normal((nb, hkv, 16, d), dtype=np.float32) * 2)
    vc = oracle.fp8_encode(rng.standard_normal((nb, hkv, 16, d), dtype=np.float32))
    q = oracle.f32_to_bf16(rng.standard_normal((sum(chunks), hq, d), dtype=np.float32))
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    past = np.asarray(pasts, np.int32)
    out = pa.prefill(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt),
                     to_dev(cu), to_dev(past), max(chunks))
    got = oracle.bf16_to_f32(to_np(out))
    ref = oracle.paged_attention(oracle.bf16_to_f32(q), oracle.fp8_decode(kc),
                                 oracle.fp8_decode(vc), bt, cu, past)
    assert np.isfinite(got).all()
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, f"fp8 prefill {hq}/{hkv}x{d}")


def assert_same_specials(got, ref, what):
    """NaN where the reference is NaN, the same signed infinities, and the
    finite entries within the bf16 bar."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), (
        f"{what}: NaN pattern differs ({np.isnan(got).sum()} vs {np.isnan(ref).sum()})")
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)), f"{what}: +inf pattern"
    assert np.array_equal(np.isneginf(got), np.isneginf(ref)), f"{what}: -inf pattern"
    fin = np.isfinite(ref)
    assert_close(got[fin], ref[fin], BF16_ATOL, BF16_RTOL, what)


def plant_codes(rng, kc, vc, bt, ctx, hkv, d):
    """Writes the reference's special and off-OCP codes into visible cache
    entries, one pattern per sequence (sequences 0-5), and NaN / inf codes
    past the context of sequence 6.  kc / vc: reference-layout codes."""
    def at(b, tok):
        return bt[b, tok // 16], tok % 16
    blk, off = at(0, ctx[0] // 3)
    kc[blk, 1, off, 5] = 0x80                       # K NaN: every head of kv head 1
    blk, off = at(1, ctx[1] - 1)
    kc[blk, 0, off, 7] = 0x7C                       # K +inf: NaN where q[7] > 0
    blk, off = at(2, 10)
    vc[blk, hkv - 1, off, d - 1] = 0xFC             # V -inf in one dim
    blk, off = at(3, ctx[3] // 2)
    vc[blk, 0, off, 0] = 0x80                       # V NaN in one dim
    blk, off = at(3, ctx[3] // 2 + 1)
    vc[blk, 0, off, 1] = 0x7C                       # and V +inf in another
    # off-OCP finite codes: subnormal-field codes in K, every one in V
    sub = np.array([1, 2, 3, 4, 5, 6, 7, 0x81, 0x82, 0x83, 0x84, 0x85, 0x86, 0x87], np.uint8)
    big = np.array([0x7F, 0xFF, 0x78, 0xF8, 0x7B, 0xFB, 0x7D, 0xFD, 0x7E, 0xFE], np.uint8)
    for b, codes_k, codes_v in ((4, sub, np.concatenate([sub, big])), (5, sub, sub)):
        n = int(ctx[b])
        for tok in rng.choice(n, min(n, 40), replace=False):
            blk, off = at(b, int(tok))
            h = rng.integers(0, hkv)
            kc[blk, h, off, rng.integers(0, d)] = rng.choice(codes_k)
            vc[blk, h, off, rng.integers(0, d)] = rng.choice(codes_v)
    n = int(ctx[6])
    if n % 16:
        blk = bt[6, (n - 1) // 16]
        kc[blk, :, n % 16:, 0] = 0x80
        vc[blk, :, n % 16:, 1] = 0x7C


@pytest.mark.parametrize("B,ctx_hi", [(7, 3000), (64, 2048), (24, 6000)])
def test_decode_fp8_special_codes(pa, oracle, B, ctx_hi):
    # The reference decodes 0x80 as NaN and 0x7C / 0xFC as +-inf, and
    # 0x01-0x07 / 0x7F as finite values the OCP conversion reads otherwise
    # (kv_cache_fp8.rs:188-212).  Attention over such codes equals the
    # oracle's attention over the reference-decoded caches: NaN / inf where
    # it has them, the finite entries within the bf16 bar, codes past the
    # context ignored.  B 7: partitions merged by the reduce kernel; B 64:
    # 512-token partitions merged inside the workgroup; B 24 past 4096
    # tokens: 1024-token partitions merged inside the workgroup.  Any
    # wavefront that meets such a code runs the out-of-line exact pass.
    rng = np.random.default_rng(B)
    hq, hkv, d = 32, 8, 128
    ctx = rng.integers(ctx_hi // 2, ctx_hi + 1, B).astype(np.int32)
    ctx[6] = ctx_hi - 5
    case, kc, vc = fp8_decode_case(oracle, rng, B, hq, hkv, d, ctx)
    plant_codes(rng, kc, vc, case["block_tables"], ctx, hkv, d)
    got, ref = run_fp8_decode(pa, oracle, case, kc, vc)
    assert np.isnan(ref[0]).any() and np.isinf(ref[2]).any()
    assert_same_specials(got, ref, f"fp8 decode specials B {B}")


def test_prefill_fp8_special_codes(pa, oracle):
    # The same codes under the chunked-prefill mask: a code among the past
    # keys reaches every query row, one among the new keys only the rows at
    # or after it.
    rng = np.random.default_rng(77)
    hq, hkv, d = 32, 8, 128
    pasts, chunks = [100, 0, 64, 300, 17, 250, 33], [150, 200, 70, 20, 90, 64, 50]
    B = len(pasts)
    ctx = np.array([p + c for p, c in zip(pasts, chunks)], np.int32)
    nblk = [(int(c) + 15) // 16 for c in ctx]
    nb = sum(nblk) + 5
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((B, max(nblk)), np.int32)
    o = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
    kc = oracle.fp8_encode(rng.standard_normal((nb, hkv, 16, d), dtype=np.float32))
    vc = oracle.fp8_encode(rng.standard_normal((nb, hkv, 16, d), dtype=np.float32))
    plant_codes(rng, kc, vc, bt, ctx, hkv, d)
    q = oracle.f32_to_bf16(rng.standard_normal((sum(chunks), hq, d), dtype=np.float32))
    cu = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    past = np.asarray(pasts, np.int32)
    out = pa.prefill(to_dev(q), to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(bt),
                     to_dev(cu), to_dev(past), max(chunks))
    got = oracle.bf16_to_f32(to_np(out))
    ref = oracle.paged_attention(oracle.bf16_to_f32(q), oracle.fp8_decode(kc),
                                 oracle.fp8_decode(vc), bt, cu, past)
    assert np.isnan(ref).any() and np.isinf(ref).any() and np.isfinite(ref).any()
    assert_same_specials(got, ref, "fp8 prefill specials")


def test_prefill_fp8_config3_full_size(pa, oracle):
    # The config-3 workload over an FP8-E4M3 cache at full size (the
    # prefill-fp8 benchmark): 4 x 2048 new tokens on past 0 / 512 / 1024 /
    # 2048, 32 / 8 x 128.  Sampled query rows against the oracle over the
    # decoded cache (row i of sequence s as a one-row sequence with past
    # P_s + i: tile diagonal edges, both wavefront halves, the first and last
    # rows, random rows), then every row against pa_decode over the same
    # FP8 cache (the FP8 decode kernel is itself checked against the oracle).
    from test_gpu_prefill import make_prefill_case
    rng = np.random.default_rng(3)
    pasts, chunk = [0, 512, 1024, 2048], 2048
    q, kc, vc, bt, cu, past = make_prefill_case(oracle, rng, pasts, [chunk] * 4, 32, 8, 128,
                                                "f32")
    q = oracle.f32_to_bf16(q)
    kc8, vc8 = oracle.fp8_encode(kc), oracle.fp8_encode(vc)
    dk, dv, dbt = to_dev(kc8), to_dev(oracle.v_from_ref(vc8)), to_dev(bt)
    out = pa.prefill(to_dev(q), dk, dv, dbt, to_dev(cu), to_dev(past), chunk)
    got = oracle.bf16_to_f32(to_np(out))

    rows = []
    for s in range(4):
        pick = {0, 1, 31, 32, 33, 2047, 2046}
        pick |= {i for i in range(chunk) if i % 64 in (0, 63) and i % 512 < 64}
        pick |= set(rng.integers(0, chunk, 8).tolist())
        rows += [(s, i) for i in sorted(pick)]
    sel = np.array([cu[s] + i for s, i in rows])
    past1 = np.array([pasts[s] + i for s, i in rows], np.int32)
    ref = oracle.paged_attention(oracle.bf16_to_f32(q[sel]), oracle.fp8_decode(kc8),
                                 oracle.fp8_decode(vc8), bt[[s for s, _ in rows]],
                                 np.arange(len(rows) + 1), past1, scale=1 / math.sqrt(128))
    assert_close(got[sel], ref, BF16_ATOL, BF16_RTOL, "fp8 config 3 full, sampled rows")

    seq = np.repeat(np.arange(4), chunk)
    ctx = (np.asarray(pasts)[seq] + np.tile(np.arange(chunk), 4) + 1).astype(np.int32)
    dec = pa.decode(to_dev(q), dk, dv, to_dev(bt[seq]), to_dev(ctx), int(ctx.max()))
    assert_close(got, oracle.bf16_to_f32(to_np(dec)), 2e-2, 1e-2,
                 "fp8 config 3 full, all rows vs pa_decode")


def test_decode_fp8_config2_full_size(pa, oracle):
    # The config-2 shape over an FP8-E4M3 cache at full size (the
    # decode-fp8 benchmark: B 64, ctx 4096, 32 / 8 x 128; 512-token
    # partitions merged eight per workgroup) against the oracle over the
    # decoded cache.
    rng = np.random.default_rng(12)
    case, kc, vc = fp8_decode_case(oracle, rng, 64, 32, 8, 128, [4096] * 64)
    got, ref = run_fp8_decode(pa, oracle, case, kc, vc)
    assert_close(got, ref, BF16_ATOL, BF16_RTOL, "fp8 config 2 full")


def exotic_codes(c):
    """Codes the hardware E4M3 conversion reads differently from the
    reference's decode: exponent field 15, or exponent field 0 and a
    nonzero byte."""
    e = (c >> 3) & 0xF
    return (e == 15) | ((e == 0) & (c != 0))


@pytest.mark.parametrize("src", ["f32", "bf16"])
@pytest.mark.parametrize("h,d", [(8, 128), (3, 40)])
def test_reshape_and_cache_fp8_flagged(pa, oracle, src, h, d):
    # The flagged writer stores the same bytes as pa_reshape_and_cache_fp8
    # and sets exactly the flags of the blocks that received a NaN / inf
    # code (the values wide_values plants), leaving flags already set.
    # (8, 128): the block-coalesced kernel, with one whole-block run of
    # slots; (3, 40): the per-token kernel.
    rng = np.random.default_rng(h + d)
    t, nb = 77, 12
    k = wide_values(rng, (t, h, d))
    v = wide_values(rng, (t, h, d))
    if src == "bf16":
        dk, dv = to_dev(oracle.f32_to_bf16(k)), to_dev(oracle.f32_to_bf16(v))
        k, v = oracle.bf16_to_f32(oracle.f32_to_bf16(k)), oracle.bf16_to_f32(oracle.f32_to_bf16(v))
    else:
        dk, dv = to_dev(k), to_dev(v)
    slots = rng.permutation(nb * 16)[:t].astype(np.int64)
    slots[16:32] = 5 * 16 + np.arange(16)      # tokens 16-31 fill block 5 in order
    slots[3] = -1
    run = (np.arange(t) >= 16) & (np.arange(t) < 32)
    slots = np.where(np.isin(slots, slots[16:32]) & ~run, -1, slots)
    kc, vc = pa.ops.new_cache(nb, h, d, torch.uint8, DEV)
    kc2, vc2 = pa.ops.new_cache(nb, h, d, torch.uint8, DEV)
    flags = torch.zeros(nb, dtype=torch.uint8, device=DEV)
    flags[11] = 1                               # set before: stays set
    pa.reshape_and_cache_fp8(dk, dv, kc, vc, to_dev(slots), block_flags=flags)
    pa.reshape_and_cache_fp8(dk, dv, kc2, vc2, to_dev(slots))
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    codes_k, codes_v = oracle.fp8_encode(k), oracle.fp8_encode(v)
    want = np.zeros(nb, np.uint8)
    want[11] = 1
    for i, s in enumerate(slots):
        if 0 <= s < nb * 16 and (exotic_codes(codes_k[i]).any() or exotic_codes(codes_v[i]).any()):
            want[s // 16] = 1
    assert want.sum() >= 3
    assert np.array_equal(to_np(flags), want)


@pytest.mark.parametrize("B,ctx_hi", [(7, 3000), (64, 2048), (24, 6000)])
def test_decode_fp8_flagged(pa, oracle, B, ctx_hi):
    # pa_decode_fp8_flagged over the special-code caches of
    # test_decode_fp8_special_codes with the flags of the blocks that hold
    # them: bit-identical to pa_decode (whose per-code test finds the same
    # partitions), hence the reference's NaN / inf pattern; with one more,
    # needless flag the output is still the same.
    rng = np.random.default_rng(B)
    hq, hkv, d = 32, 8, 128
    ctx = rng.integers(ctx_hi // 2, ctx_hi + 1, B).astype(np.int32)
    ctx[6] = ctx_hi - 5
    case, kc, vc = fp8_decode_case(oracle, rng, B, hq, hkv, d, ctx)
    plant_codes(rng, kc, vc, case["block_tables"], ctx, hkv, d)
    nb = kc.shape[0]
    flags = (exotic_codes(kc).reshape(nb, -1).any(1) |
             exotic_codes(vc).reshape(nb, -1).any(1)).astype(np.uint8)
    assert flags.sum() > 0
    q, bt = to_dev(case["q"]), to_dev(case["block_tables"])
    dk, dv, dctx = to_dev(kc), to_dev(oracle.v_from_ref(vc)), to_dev(ctx)
    plain = pa.decode(q, dk, dv, bt, dctx, int(ctx.max()))
    flagged = pa.decode(q, dk, dv, bt, dctx, int(ctx.max()), block_flags=to_dev(flags))
    assert torch.equal(plain.view(torch.int16), flagged.view(torch.int16))
    _, ref = run_fp8_decode(pa, oracle, case, kc, vc)
    assert_same_specials(oracle.bf16_to_f32(to_np(flagged)), ref, f"fp8 flagged B {B}")
    flags[case["block_tables"][1, 0]] = 1
    again = pa.decode(q, dk, dv, bt, dctx, int(ctx.max()), block_flags=to_dev(flags))
    assert torch.equal(plain.view(torch.int16), again.view(torch.int16))
