"""GPU parity of the batched step (pa_batch_*): an engine loop of mixed
prefill chunks and decodes over several layers, each step's attention
checked against the oracle run on its own cache."""
import numpy as np
import pytest
import torch

from helpers import BF16_ATOL, BF16_RTOL, F32_ATOL, F32_RTOL, assert_close
from test_gpu_cache_ops import DEV, to_dev, to_np

pytestmark = pytest.mark.gpu

# (sequence -> tokens fed) per step; a sequence's first step is its prefill
# (chunked when it spans several steps), later single tokens are decodes.
STEPS = [
    {0: 40, 1: 20},
    {0: 1, 1: 30},
    {0: 1, 1: 1},
    {0: 1, 1: 1, 2: 70},
    {2: 1, 0: 1},
]


# long contexts over few sequences (the engine's decode shape): several
# partitions per (sequence, kv head) merged in the workgroup, two decode
# steps in a row
LONG_STEPS = [
    {0: 700, 1: 1000, 2: 333, 3: 129},
    {0: 1, 1: 1, 2: 1, 3: 1},
    {0: 1, 1: 1, 2: 1, 3: 1},
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rope", [True, False])
def test_engine_loop(pa, oracle, dtype, rope):
    run_loop(pa, oracle, dtype, rope, STEPS, 128, 48)


@pytest.mark.parametrize("d", [64, 128])
def test_engine_loop_long_decode(pa, oracle, d):
    run_loop(pa, oracle, "bf16", True, LONG_STEPS, d, 160)


def run_loop(pa, oracle, dtype, rope, steps, d, nb):
    rng = np.random.default_rng(11 + rope + d)
    layers, hq, hkv = 2, 8, 2
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    cache = pa.PagedKvCache(layers, hkv, d, nb, tdt, DEV)
    pool = list(rng.permutation(nb))
    tables, computed = {}, {}
    inv = oracle.rope_inv_freq(d, 1e4)
    ref_k = [np.zeros((nb, hkv, 16, d), np.uint16 if dtype == "bf16" else np.float32)
             for _ in range(layers)]
    ref_v = [np.zeros_like(ref_k[0]) for _ in range(layers)]
    batch = pa.StepBatch()
    for step in steps:
        seqs = list(step)
        for s in seqs:
            computed.setdefault(s, 0)
            tables.setdefault(s, [])
            while len(tables[s]) * 16 < computed[s] + step[s]:
                tables[s].append(int(pool.pop()))
        batch.prepare(cache, [step[s] for s in seqs], [computed[s] for s in seqs],
                      [tables[s] for s in seqs])
        t = sum(step.values())
        assert batch.num_tokens() == t
        assert batch.is_decode() == all(step[s] == 1 and computed[s] > 0 for s in seqs)
        positions = np.concatenate([np.arange(computed[s], computed[s] + step[s])
                                    for s in seqs]).astype(np.int64)
        slots = np.concatenate([[tables[s][p // 16] * 16 + p % 16
                                 for p in range(computed[s], computed[s] + step[s])]
                                for s in seqs]).astype(np.int64)
        mbs = max(len(tables[s]) for s in seqs)
        bt = np.zeros((len(seqs), mbs), np.int32)
        for i, s in enumerate(seqs):
            bt[i, :len(tables[s])] = tables[s]
        q_start = np.concatenate([[0], np.cumsum([step[s] for s in seqs])]).astype(np.int32)
        past = np.array([computed[s] for s in seqs], np.int32)
        for layer in range(layers):
            qkv = rng.standard_normal((t, hq + 2 * hkv, d), dtype=np.float32)
            if dtype == "bf16":
                qkv = oracle.f32_to_bf16(qkv)
            g = to_dev(qkv)
            # layer 1: q as a strided view of the fused QKV rows
            q = g[:, :hq] if layer == 1 else g[:, :hq].contiguous()
            out = batch.attention(cache, layer, q, g[:, hq:hq + hkv], g[:, hq + hkv:],
                                  to_dev(inv) if rope else None)
            qr, kr = qkv[:, :hq], qkv[:, hq:hq + hkv]
            if rope:
                qr, kr = oracle.rope(qr, positions, inv), oracle.rope(kr, positions, inv)
            oracle.reshape_and_cache(kr, qkv[:, hq + hkv:], ref_k[layer], ref_v[layer], slots)
            want = oracle.paged_attention(np.ascontiguousarray(qr), ref_k[layer], ref_v[layer],
                                          bt, q_start, past)
            tol = (BF16_ATOL, BF16_RTOL) if dtype == "bf16" else (F32_ATOL, F32_RTOL)
            got = to_np(out.float()) if dtype == "bf16" else to_np(out)
            if dtype == "bf16":
                want = oracle.bf16_to_f32(want)
            assert_close(got, want, *tol, f"step {steps.index(step)} layer {layer}")
            if not rope:
                # the cache holds exactly what the oracle wrote
                assert np.array_equal(to_np(cache.key_cache(layer)), ref_k[layer])
                assert np.array_equal(oracle.v_to_ref(to_np(cache.value_cache(layer))),
                                      ref_v[layer])
        for s in seqs:
            computed[s] += step[s]


def test_prepare_rejects_bad_tables(pa):
    cache = pa.PagedKvCache(1, 2, 64, 8, torch.bfloat16, DEV)
    batch = pa.StepBatch()
    with pytest.raises(pa.PaError, match="out of bounds"):
        batch.prepare(cache, [3], [0], [[8]])
    with pytest.raises(pa.PaError, match="table holds"):
        batch.prepare(cache, [20], [0], [[1]])
    batch.prepare(cache, [17], [0], [[1, 2]])
    # a prepare rejected by validation leaves the prepared step as it was
    with pytest.raises(pa.PaError, match="out of bounds"):
        batch.prepare(cache, [1, 1], [3, 3], [[1], [9]])
    assert batch.num_tokens() == 17
    q = torch.zeros(17, 4, 64, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(17, 2, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(pa.PaError, match="layer_idx"):
        batch.attention(cache, 1, q, kv, kv)
    with pytest.raises(pa.PaError, match="multiple"):
        batch.attention(cache, 0, torch.zeros(17, 3, 64, dtype=torch.bfloat16, device=DEV),
                        kv, kv)
    # attention only (the step's K / V already written): no inv_freq then, and
    # key and value both or neither
    inv = torch.ones(32, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):
        batch.attention(cache, 0, q, None, None, inv)
    with pytest.raises(ValueError):
        batch.attention(cache, 0, q, kv, None)
    import ctypes as C
    lib = pa._lib.load()
    out = torch.empty_like(q)
    rc = lib.pa_batch_attention(batch._h, cache._h, 0, 4, C.c_void_p(q.data_ptr()), 0, None, 0,
                                None, 0, C.c_void_p(inv.data_ptr()), 0.125,
                                C.c_void_p(out.data_ptr()), cache._stream())
    assert rc == -1 and b"inv_freq" in lib.pa_last_error()
    # the attention-only call itself runs (zero caches: zero output)
    out = batch.attention(cache, 0, q, None, None)
    assert out.shape == q.shape and not torch.isnan(out.float()).any()


def test_decode_workspace_growth_refused_under_capture(pa):
    # A decode step whose workspace would have to grow inside a stream
    # capture returns an error (hipMalloc cannot be captured) instead of
    # allocating; after one eager step of the shape the capture succeeds.
    hq, hkv, d, nb = 8, 2, 128, 512
    cache = pa.PagedKvCache(1, hkv, d, nb, torch.bfloat16, DEV)
    batch = pa.StepBatch()
    blocks = [list(range(i * 128, (i + 1) * 128)) for i in range(4)]
    batch.set_capacity(2048)
    batch.prepare(cache, [1] * 4, [1500] * 4, blocks)
    q = torch.randn(4, hq, d, device=DEV).to(torch.bfloat16)
    k = torch.randn(4, hkv, d, device=DEV).to(torch.bfloat16)
    v = torch.randn(4, hkv, d, device=DEV).to(torch.bfloat16)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="capturing"):
        with torch.cuda.graph(g, stream=stream):
            batch.attention(cache, 0, q, k, v)
    torch.cuda.synchronize()
    eager = batch.attention(cache, 0, q, k, v)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=stream):
        captured = batch.attention(cache, 0, q, k, v)
    for _ in range(2):
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
    batch.close()
    cache.close()


def _advance_case(pa, rng, seqs_ctx, d=64, nb=64):
    hq, hkv = 8, 2
    caches = []
    k0 = torch.from_numpy(rng.standard_normal((nb, hkv, 16, d), dtype=np.float32))
    for _ in range(2):
        c = pa.PagedKvCache(1, hkv, d, nb, torch.bfloat16, DEV)
        c.key_cache(0).copy_(k0.to(torch.bfloat16).to(DEV))
        c.value_cache(0).copy_(k0.transpose(-1, -2).to(torch.bfloat16).to(DEV) * 0.5)
        caches.append(c)
    pool = list(rng.permutation(nb))
    tables = [[int(pool.pop()) for _ in range((n + 8 + 15) // 16)] for n in seqs_ctx]
    return caches, tables, hq, hkv


def test_advance_equals_prepare(pa):
    # pa_batch_advance from a prepared decode step gives the same positions,
    # slots and context lengths as preparing the next step on the host:
    # attention (with RoPE and the KV write) and the caches agree bit for bit
    # over several steps, across block boundaries
    rng = np.random.default_rng(21)
    ctx = [15, 30, 47, 1]  # first decode tokens at positions 15, 30, 47, 1
    (ca, cb), tables, hq, hkv = _advance_case(pa, rng, ctx)
    d = 64
    inv = torch.from_numpy(np.ascontiguousarray(
        1e4 ** (-np.arange(0, d, 2, dtype=np.float32) / d))).to(DEV)
    adv, ref = pa.StepBatch(), pa.StepBatch()
    adv.prepare(ca, [1] * 4, ctx, tables)
    for step in range(8):
        if step:
            adv.advance(ca)
        ref.prepare(cb, [1] * 4, [n + step for n in ctx], tables)
        assert adv.is_decode() and adv.num_tokens() == 4
        q = torch.randn(4, hq, d, device=DEV).to(torch.bfloat16)
        k = torch.randn(4, hkv, d, device=DEV).to(torch.bfloat16)
        v = torch.randn(4, hkv, d, device=DEV).to(torch.bfloat16)
        oa = adv.attention(ca, 0, q.clone(), k, v, inv)
        ob = ref.attention(cb, 0, q.clone(), k, v, inv)
        assert torch.equal(oa, ob), f"step {step}"
    assert torch.equal(ca.key_cache(0), cb.key_cache(0))
    assert torch.equal(ca.value_cache(0), cb.value_cache(0))
    adv.close()
    ref.close()


def test_advance_rejects(pa):
    rng = np.random.default_rng(3)
    (c, _), tables, hq, hkv = _advance_case(pa, rng, [20, 5])
    b = pa.StepBatch()
    b.prepare(c, [5, 1], [0, 5], tables)  # a prefill chunk: not a decode step
    with pytest.raises(pa.PaError, match="not a prepared decode step"):
        b.advance(c)
    # the first table holds 2 blocks (32 tokens), the second 1 (16)
    b.prepare(c, [1, 1], [30, 5], [tables[0], tables[1]])
    b.advance(c)  # 32 tokens: the last slot of the first table
    with pytest.raises(pa.PaError, match="table holds"):
        b.advance(c)
    b.close()


def test_captured_advance_replays_match_prepared_steps(pa):
    # a captured [advance + attention] step, replayed with eager work and
    # synchronisations between the replays, equals the host-prepared steps
    rng = np.random.default_rng(8)
    ctx = [14, 33, 3]
    (ca, cb), tables, hq, hkv = _advance_case(pa, rng, ctx)
    d = 64
    adv, ref = pa.StepBatch(), pa.StepBatch()
    cap = 16 * max(len(t) for t in tables)  # the widest table's tokens
    adv.set_capacity(cap)
    ref.set_capacity(cap)
    qs = [torch.randn(3, hq, d, device=DEV).to(torch.bfloat16) for _ in range(6)]
    ks = [torch.randn(3, hkv, d, device=DEV).to(torch.bfloat16) for _ in range(6)]
    # step 0 eager on both (also sizes the decode workspace)
    adv.prepare(ca, [1] * 3, ctx, tables)
    ref.prepare(cb, [1] * 3, ctx, tables)
    assert torch.equal(adv.attention(ca, 0, qs[0], ks[0], ks[0]),
                       ref.attention(cb, 0, qs[0], ks[0], ks[0]))
    torch.cuda.synchronize()
    q_in = torch.empty_like(qs[0])
    k_in = torch.empty_like(ks[0])
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        adv.advance(ca)
        out = adv.attention(ca, 0, q_in, k_in, k_in)
    for step in range(1, 6):
        q_in.copy_(qs[step])
        k_in.copy_(ks[step])
        g.replay()
        torch.cuda.synchronize()
        ref.prepare(cb, [1] * 3, [n + step for n in ctx], tables)
        want = ref.attention(cb, 0, qs[step], ks[step], ks[step])
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {step}"
    assert torch.equal(ca.key_cache(0), cb.key_cache(0))
    adv.close()
    ref.close()


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_captured_advance_needs_capacity(pa):
    rng = np.random.default_rng(4)
    (c, _), tables, hq, hkv = _advance_case(pa, rng, [10, 20])
    b = pa.StepBatch()
    b.prepare(c, [1, 1], [10, 20], tables)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(pa.PaError, match="capacity"):
        with torch.cuda.graph(g, stream=torch.cuda.Stream()):
            b.advance(c)
    torch.cuda.synchronize()
    b.close()
