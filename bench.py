"""Benchmark of the paged-attention hot path on one MI355X.

Default workload: Llama-3-8B-shaped decode in bf16,
batch 64, 32 query / 8 KV heads, head_dim 128, every context 4096 tokens,
block tables a seeded random permutation of a 16384-block pool, K/V
0.5 * N(0, 1), Q N(0, 1), scale 1/sqrt(128).  One step = one decode step of
one layer: scatter the new token's K/V (pa_reshape_and_cache) and attend
over the 4096-token paged context (pa_decode).  Inputs are resident in HBM
before timing starts.

Prints ONE JSON line (the driver's contract) with a roofline object for the
dominant launch (pa_decode, timed with HIP events on its stream) and the
CPU baseline (the C oracle restating the reference's CPU path, timed on a
bounded sample on the host cores).

Other workloads for profiling: --config prefill (config 3, MFMA-bound),
--config splitk (config 4), --config qwen (config 1, f32).
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
from __graft_entry__ import _package  # noqa: E402

METRIC = ("paged-attn decode tokens/s + achieved HBM GB/s (% peak), Llama-3-8B shape, 1 GPU")
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_VALU_PEAK_TFLOPS = 157.3
DEV = "cuda:0"


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


def make_tables(gen, B, blocks_per_seq, pool, shared_prefix=0):
    perm = torch.randperm(pool, generator=gen)
    bt = torch.empty(B, blocks_per_seq, dtype=torch.int32)
    shared = perm[:shared_prefix]
    o = shared_prefix
    for b in range(B):
        bt[b, :shared_prefix] = shared
        n = blocks_per_seq - shared_prefix
        bt[b, shared_prefix:] = perm[o:o + n]
        o += n
    return bt


class Workload:
    """Synthetic inputs resident on the GPU plus the step closure."""

    def __init__(self, pa, name):
        self.pa = pa
        self.name = name
        g = torch.Generator().manual_seed({"decode": 1, "decode-fp8": 1, "prefill": 2,
                                           "prefill-fp8": 2, "splitk": 3, "qwen": 0}[name])
        dg = torch.Generator(device=DEV).manual_seed(1234)
        self.kind = "decode"
        self.fp8 = name in ("decode-fp8", "prefill-fp8")
        if name in ("decode", "decode-fp8"):
            B, hq, hkv, d, ctx = 64, 32, 8, 128, 4096
            self.dtype = torch.bfloat16
            nblk = ctx // 16
            pool = B * nblk  # 16384 blocks
            self.ctx = torch.full((B,), ctx, dtype=torch.int32)
            bt = make_tables(g, B, nblk, pool)
            kv_scale = 0.5
            self.workload = ("config 2: Llama-3-8B decode bf16, B 64, 32/8 heads x 128, "
                             "ctx 4096, block 16, random block tables over 16384 blocks")
            if self.fp8:
                self.workload = ("config 2 shape over an FP8-E4M3 KV cache (reference codes), "
                                 "q/out bf16, B 64, 32/8 heads x 128, ctx 4096, 16384 blocks")
        elif name == "splitk":
            B, hq, hkv, d = 16, 32, 8, 128
            self.dtype = torch.bfloat16
            lens = torch.exp(torch.empty(B).uniform_(math.log(8192), math.log(32768),
                                                     generator=g)).to(torch.int32)
            self.ctx = lens
            nblk = int((lens.max() + 15) // 16)
            pool = 256 + int(((lens + 15) // 16 - 256).sum()) + 16
            perm = torch.randperm(pool, generator=g)
            bt = torch.zeros(B, nblk, dtype=torch.int32)
            o = 256
            for b in range(B):
                n = int((lens[b] + 15) // 16)
                bt[b, :256] = perm[:256]
                bt[b, 256:n] = perm[o:o + n - 256]
                o += n - 256
            kv_scale = 1.0
            # a second 4096-token prefix (blocks past the pool) for the
            # batch-order check: two prefixes, each shared by 8 sequences
            self.extra_blocks = 256
            self.workload = ("config 4: long-context split-K decode bf16, B 16, 32/8 x 128, "
                             "ctx log-U[8k, 32k], 4096-token shared prefix")
        elif name == "qwen":
            B, hq, hkv, d = 8, 14, 2, 64
            self.dtype = torch.float32
            lens = torch.randint(128, 1025, (B,), generator=g, dtype=torch.int32)
            self.ctx = lens
            nblk = int((lens.max() + 15) // 16)
            pool = 1024
            perm = torch.randperm(pool, generator=g)
            bt = torch.zeros(B, nblk, dtype=torch.int32)
            o = 0
            for b in range(B):
                n = int((lens[b] + 15) // 16)
                bt[b, :n] = perm[o:o + n]
                o += n
            kv_scale = 1.0
            self.workload = ("config 1: Qwen2.5-0.5B decode f32, B 8, 14/2 x 64, "
                             "ctx U[128, 1024], pool 1024 blocks")
        elif name in ("prefill", "prefill-fp8"):
            self.kind = "prefill"
            hq, hkv, d = 32, 8, 128
            self.dtype = torch.bfloat16
            pasts = [0, 512, 1024, 2048]
            chunk = 2048
            B = 4
            nblks = [(p + chunk + 15) // 16 for p in pasts]
            nblk = max(nblks)
            pool = sum(nblks) + 16
            perm = torch.randperm(pool, generator=g)
            bt = torch.zeros(B, nblk, dtype=torch.int32)
            o = 0
            for b in range(B):
                bt[b, :nblks[b]] = perm[o:o + nblks[b]]
                o += nblks[b]
            self.past = torch.tensor(pasts, dtype=torch.int32, device=DEV)
            self.cu = torch.tensor([0, chunk, 2 * chunk, 3 * chunk, 4 * chunk],
                                   dtype=torch.int32, device=DEV)
            self.max_q = chunk
            self.q = torch.randn(B * chunk, hq, d, generator=dg, device=DEV).to(self.dtype)
            kv_scale = 1.0
            self.pairs = sum(chunk * p + chunk * (chunk + 1) // 2 for p in pasts)
            self.flops = 4.0 * self.pairs * hq * d
            self.workload = ("config 3: Llama-3-8B chunked causal prefill bf16, 4 x 2048 new "
                             "tokens on past 0/512/1024/2048, 32/8 x 128")
            if self.fp8:
                self.workload = ("config 3 shape over an FP8-E4M3 KV cache (reference codes), "
                                 "q/out bf16, 4 x 2048 new tokens on past 0/512/1024/2048, "
                                 "32/8 x 128")
        else:
            raise SystemExit(f"unknown config {name}")
        self.B, self.hq, self.hkv, self.d = B, hq, hkv, d
        self.scale = 1.0 / math.sqrt(d)
        self.bt = bt.to(DEV)
        self.pool = pool
        if self.fp8:
            # quantise N(0, 0.5) K/V into the pool with the library's encoder
            self.kc, self.vc = pa.ops.new_cache(pool, hkv, d, torch.uint8, DEV)
            chunk = 16384
            for t0 in range(0, pool * 16, chunk):
                n = min(chunk, pool * 16 - t0)
                kk = (torch.randn(n, hkv, d, generator=dg, device=DEV) * kv_scale).to(self.dtype)
                vv = (torch.randn(n, hkv, d, generator=dg, device=DEV) * kv_scale).to(self.dtype)
                sl = torch.arange(t0, t0 + n, dtype=torch.int64, device=DEV)
                pa.reshape_and_cache_fp8(kk, vv, self.kc, self.vc, sl)
            del kk, vv, sl
        else:
            nbk = pool + getattr(self, "extra_blocks", 0)
            self.kc = (torch.randn(nbk, hkv, 16, d, generator=dg, device=DEV) * kv_scale).to(
                self.dtype)
            self.vc = (torch.randn(nbk, hkv, d, 16, generator=dg, device=DEV) * kv_scale).to(
                self.dtype)
        self.ctx_dev = self.ctx.to(DEV) if self.kind == "decode" else None
        es = torch.empty(0, dtype=self.dtype).element_size()
        if self.kind == "decode":
            self.q = torch.randn(B, hq, d, generator=dg, device=DEV).to(self.dtype)
            self.out = torch.empty_like(self.q)
            self.max_ctx = int(self.ctx.max())
            self.ws = torch.empty(max(1, pa.decode_workspace_size(B, hq, d, self.max_ctx)),
                                  dtype=torch.uint8, device=DEV)
            # new token of each sequence = its last position
            pos = (self.ctx - 1).to(torch.int64)
            slots = bt[torch.arange(B), (pos // 16)].to(torch.int64) * 16 + pos % 16
            self.slots = slots.to(DEV)
            self.k_new = torch.randn(B, hkv, d, generator=dg, device=DEV).to(self.dtype)
            self.v_new = torch.randn(B, hkv, d, generator=dg, device=DEV).to(self.dtype)
            tokens = int(self.ctx.sum())
            # algorithmic bytes per pa_decode launch: K and V of every context
            # token at Hkv heads, q in, out, block tables, context lengths.
            kv_es = 1 if self.fp8 else es
            self.kv_bytes = 2 * tokens * hkv * d * kv_es
            self.alg_bytes = (self.kv_bytes + 2 * B * hq * d * es +
                              int(((self.ctx + 15) // 16).sum()) * 4 + B * 4)
            uniq = len(set(bt[:, :].flatten().tolist()))
            self.unique_kv_bytes = 2 * min(uniq * 16, tokens) * hkv * d * kv_es
        else:
            self.out = torch.empty_like(self.q)
            tokens_all = sum(p + 2048 for p in [0, 512, 1024, 2048])
            kv_es = 1 if self.fp8 else es
            self.alg_bytes = (2 * tokens_all * hkv * d * kv_es + 2 * self.q.numel() * es)

    def two_prefix_tables(self, interleaved):
        """Config 4's tables with two 4096-token prefixes, each shared by 8
        sequences: A by sequences 0-7 and B by 8-15 (ordered), or A by the
        even and B by the odd batch slots (interleaved).  Same contexts,
        same bytes and the same sharing in both; only the batch order of
        the sharers differs."""
        bt = self.bt.clone()
        other = torch.arange(self.pool, self.pool + 256, dtype=torch.int32, device=DEV)
        for b in range(self.B):
            if (b % 2 == 1) if interleaved else (b >= self.B // 2):
                bt[b, :256] = other
        return bt

    def write_step(self):
        if self.fp8:
            self.pa.reshape_and_cache_fp8(self.k_new, self.v_new, self.kc, self.vc, self.slots)
        else:
            self.pa.reshape_and_cache(self.k_new, self.v_new, self.kc, self.vc, self.slots)

    def attend(self):
        if self.kind == "decode":
            self.pa.decode(self.q, self.kc, self.vc, self.bt, self.ctx_dev, self.max_ctx,
                           scale=self.scale, out=self.out, workspace=self.ws)
        else:
            self.pa.prefill(self.q, self.kc, self.vc, self.bt, self.cu, self.past, self.max_q,
                            scale=self.scale, out=self.out)

    def step(self):
        if self.kind == "decode":
            self.write_step()
        self.attend()


def measured_traffic(config):
    """HBM bytes per launch of the dominant call as measured with rocprofv3
    --pmc FETCH_SIZE / WRITE_SIZE (scaled by the copy calibration), read from
    profiles/hbm_traffic.txt, with where they come from: (bytes, source) or
    (None, None) when that file has no entry.  The run does not measure
    them itself (counters need a profiler pass of their own); the source
    names the commit and the kernel duration of that pass, so a bench line
    whose avg_launch_us has moved away from it shows that the byte count may
    be stale."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        kv = dict(x.split("=", 1) for x in line.split() if "=" in x)
        if kv.get("config") == config:
            src = {"file": "profiles/hbm_traffic.txt",
                   "method": "rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE; copy-calibrated",
                   "commit": kv.get("commit"),
                   "profiled_launch_us": float(kv["launch_us"]) if "launch_us" in kv else None}
            return int(kv["fetch_bytes"]) + int(kv["write_bytes"]), src
    return None, None


def time_attend(w, iters):
    """Average duration of the dominant launch (pa_decode / pa_prefill),
    HIP events on the stream the library launches on (torch's current)."""
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        w.attend()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / iters / 1e3  # seconds


def time_attend_flushed(w, iters, flush_bytes=512 << 20, dirty=False):
    """Median duration of the dominant launch with the caches flushed before
    each one: 512 MiB (larger than L2 + MALL) of scratch is streamed between
    launches, and HIP events bracket each launch on its own.  By default
    the scratch is read (a sum), which leaves the caches full of clean lines
    of other data: a cold start.  dirty=True writes it instead (a fill), so
    the launch also runs while that much dirty data is being written back."""
    scratch = torch.ones(flush_bytes // 4, dtype=torch.float32, device=DEV)
    sink = torch.empty((), dtype=torch.float32, device=DEV)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(iters)]
    torch.cuda.synchronize()
    for a, b in ev:
        if dirty:
            scratch.fill_(1.0)
        else:
            torch.sum(scratch, dim=0, out=sink)
        a.record()
        w.attend()
        b.record()
    torch.cuda.synchronize()
    return float(np.median([a.elapsed_time(b) for a, b in ev])) / 1e3


def flushed_legs(roof, w, iters, frac_of, no_flush):
    """Adds the cache-flushed timing legs to a roofline dict: read flush
    (cold, clean caches) as flushed_launch_us / flushed_frac, write flush
    (dirty lines draining meanwhile) as flushed_dirty_launch_us / _frac."""
    if no_flush:
        return
    for key, dirty in (("flushed", False), ("flushed_dirty", True)):
        t = time_attend_flushed(w, iters, dirty=dirty)
        roof[key + "_launch_us"] = round(t * 1e6, 2)
        roof[key + "_frac"] = round(frac_of(t), 4)


def gemm_ceiling(n=8192, iters=10):
    """Measured bf16 MFMA ceiling of this GPU: a square hipBLASLt GEMM
    (torch.matmul) of side n, in TFLOP/s.  The datasheet's 2.5 PFLOP/s is
    the roofline peak; this is what a tuned GEMM sustains on the same box."""
    a = torch.randn(n, n, device=DEV, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=DEV, dtype=torch.bfloat16)
    for _ in range(2):
        a @ b
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        a @ b
    stop.record()
    torch.cuda.synchronize()
    t = start.elapsed_time(stop) / iters / 1e3
    return 2.0 * n ** 3 / t / 1e12


def cpu_baseline(w, budget_s=12.0):
    """Times the C oracle (restated reference CPU path: gather blocks to dense
    f32, expand KV to all query heads, full softmax, OpenMP over heads) on a
    bounded sample of the same workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    threads = cpu_threads()
    if w.kind != "decode":
        return cpu_baseline_prefill(w, oracle, threads, budget_s)
    nseq = min(8, w.B)
    bt = w.bt[:nseq].cpu().numpy()
    ctx = w.ctx[:nseq].numpy()
    used = sorted(set(int(x) for b in range(nseq) for x in bt[b, :(ctx[b] + 15) // 16]))
    remap = {blk: i for i, blk in enumerate(used)}
    bt_c = np.vectorize(lambda x: remap.get(int(x), 0))(bt).astype(np.int32)
    idx = torch.tensor(used, device=DEV)

    def host(t):
        if t.dtype == torch.bfloat16:
            return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        return t.contiguous().cpu().numpy()

    kc = host(w.kc[idx])
    vc = host(w.vc[idx].transpose(-1, -2))
    q = host(w.q[:nseq])
    if w.fp8:
        # the reference dequantises FP8 blocks (Fp8Quantizer::dequantize) before
        # attending in f32; the dequantisation is part of each timed pass
        q = oracle.bf16_to_f32(q)

        def attend(qq, bts, qs, past):
            oracle.paged_attention(qq, oracle.fp8_decode(kc), oracle.fp8_decode(vc), bts, qs,
                                   past, scale=w.scale, threads=threads)
    else:
        def attend(qq, bts, qs, past):
            oracle.paged_attention(qq, kc, vc, bts, qs, past, scale=w.scale, threads=threads)
    attend(q[:1], bt_c[:1], [0, 1], ctx[:1] - 1)  # warm
    t0 = time.perf_counter()
    reps = 0
    while True:
        attend(q, bt_c, np.arange(nseq + 1), ctx - 1)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 50:
            break
    return {"value": round(nseq * reps / el, 2), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"{nseq} sequences of the same workload x {reps} passes "
                      f"({el:.1f} s): oracle {'FP8 dequantisation + ' if w.fp8 else ''}"
                      "gather + expand_kv + dense f32 softmax attention, OpenMP"}


def cpu_baseline_prefill(w, oracle, threads, budget_s):
    """Config 3 on the C oracle (the reference's chunked-prefill path
    restated: per 16-row query tile, gather the tile's visible keys to dense
    f32, expand KV to every query head, masked dense softmax attention,
    OpenMP over heads), timed on a bounded sample of the same workload: 8
    query tiles of 16 rows spread evenly over each sequence's 2048-row chunk
    (32 tiles), each attending its past + causal keys.  The rate is the
    sample's causal (query, key) pairs x 4 Hq D FLOP per second, the unit of
    the GPU figure."""
    pasts = w.past.cpu().tolist()
    cu = w.cu.cpu().tolist()
    bt_all = w.bt.cpu().numpy()
    tiles = []
    for b, past in enumerate(pasts):
        for t0 in np.linspace(0, w.max_q - 16, 8).astype(int).tolist():
            tiles.append((b, past + t0, cu[b] + t0))
    # the blocks the sample reads, remapped into a compact host pool
    used = sorted({int(x) for b, p, _ in tiles for x in bt_all[b, :(p + 16 + 15) // 16]})
    remap = np.zeros(int(bt_all.max()) + 1, np.int32)
    remap[used] = np.arange(len(used), dtype=np.int32)
    idx = torch.tensor(used, device=DEV)

    def host(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    if w.fp8:
        kc = oracle.fp8_decode(host8(w.kc[idx]))
        vc = oracle.fp8_decode(host8(w.vc[idx].transpose(-1, -2)))
        q = oracle.bf16_to_f32(host(w.q))
    else:
        kc = host(w.kc[idx])
        vc = host(w.vc[idx].transpose(-1, -2))
        q = host(w.q)
    bt = np.stack([remap[bt_all[b]] for b, _, _ in tiles]).astype(np.int32)
    qs = np.concatenate([q[r0:r0 + 16] for _, _, r0 in tiles])
    past = np.array([p for _, p, _ in tiles], np.int32)
    qstart = np.arange(0, 16 * len(tiles) + 1, 16, dtype=np.int32)
    pairs = sum(16 * p + 16 * 17 // 2 for p in past.tolist())
    flops = 4.0 * pairs * w.hq * w.d
    oracle.paged_attention(qs[:16], kc, vc, bt[:1], qstart[:2], past[:1], scale=w.scale,
                           threads=threads)  # warm
    t0 = time.perf_counter()
    reps = 0
    while True:
        oracle.paged_attention(qs, kc, vc, bt, qstart, past, scale=w.scale, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 50:
            break
    return {"value": round(flops * reps / el / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{len(tiles)} query tiles of 16 rows spread over the 4 chunks "
                      f"({pairs} causal pairs) x {reps} passes ({el:.1f} s): oracle "
                      f"{'FP8 dequantisation (outside the timing) + ' if w.fp8 else ''}"
                      "gather + expand_kv + masked dense f32 softmax attention, OpenMP"}


def host8(t):
    return t.contiguous().cpu().numpy()


def run_kv_rw(pa, args):
    """The reference's own published microbenchmark on this path,
    paged_kv_cache/read_write (crates/model/benches/paged_kv_cache.rs:69-103):
    a 1-layer f32 cache of 2 heads x 64 dims and 64 / 256 / 1024 blocks; each
    iteration is one write_kv of one token into (block 0, offset 0) and one
    read_kv of 1 token over block 0, here pa_kv_cache_write_kv +
    pa_kv_cache_read_kv through the cache mirror (both synchronise, as the
    reference's host copies do), timed end to end in ns per iteration.  The
    reference's figures (docs/perf/v27-after.md:61-63) were taken on an
    unnamed CUDA GPU.  The oracle's write_kv + read_kv on the same sizes is
    timed on the host beside it."""
    import ctypes as C
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    ref_ns = {64: 393358, 256: 712714, 1024: 1847365}
    lib = pa._lib.load()
    h, d = 2, 64
    g = torch.Generator(device=DEV).manual_seed(7)
    for nb in (64, 256, 1024):
        cache = pa.PagedKvCache(1, h, d, nb, dtype=torch.float32, device=DEV)
        k = torch.randn(1, h, d, generator=g, device=DEV)
        v = torch.randn(1, h, d, generator=g, device=DEV)
        out_k = torch.empty(1, h, d, device=DEV)
        out_v = torch.empty_like(out_k)
        ids = (C.c_int64 * 1)(0)
        n = C.c_int32(0)
        stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        hnd = cache._h
        kp, vp = C.c_void_p(k.data_ptr()), C.c_void_p(v.data_ptr())
        okp, ovp = C.c_void_p(out_k.data_ptr()), C.c_void_p(out_v.data_ptr())

        def it():
            rc = lib.pa_kv_cache_write_kv(hnd, 0, 0, 0, kp, vp, stream)
            rc |= lib.pa_kv_cache_read_kv(hnd, 0, ids, 1, 1, okp, ovp, C.byref(n), stream)
            return rc
        for _ in range(max(args.warmup, 20)):
            assert it() == 0
        torch.cuda.synchronize()
        iters = max(args.steps, 200)
        t0 = time.perf_counter()
        for _ in range(iters):
            it()
        torch.cuda.synchronize()
        ns = (time.perf_counter() - t0) / iters * 1e9
        assert torch.equal(out_k, k) and torch.equal(out_v, v)
        cache.close()
        cpu = None
        if not args.no_cpu:
            kc = np.zeros((nb, h, 16, d), np.float32)
            vc = np.zeros_like(kc)
            kh, vh = k.cpu().numpy()[0], v.cpu().numpy()[0]
            reps, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < 3.0:
                oracle.write_kv(kc, vc, 0, 0, kh, vh)
                oracle.read_kv(kc, vc, [0], 1)
                reps += 1
            cpu_ns = (time.perf_counter() - t0) / reps * 1e9
            cpu = {"value": round(cpu_ns, 1), "unit": "ns/iter", "cores": 1, "kind": "port",
                   "sample": f"{reps} iterations of the oracle's write_kv + read_kv (3 s)"}
        print(json.dumps({
            "metric": "paged_kv_cache/read_write ns/iter (reference microbenchmark)",
            "value": round(ns, 1), "unit": "ns/iter", "n_gpus": 1, "steps": iters,
            "warmup": max(args.warmup, 20), "ms_per_step": round(ns / 1e6, 6),
            "higher_is_better": False,
            "vs_baseline": round(ns / ref_ns[nb], 5), "baseline_ns": ref_ns[nb],
            "baseline_source": "docs/perf/v27-after.md:61-63 (unnamed CUDA GPU, candle)",
            "speedup_vs_reference": round(ref_ns[nb] / ns, 1),
            "dtype": "f32", "data": "synthetic (N(0,1) token K/V)",
            "config": {"workload": f"paged_kv_cache read_write blocks{nb}_h2_d64: 1 layer, "
                                   "write_kv (block 0, offset 0) + read_kv (1 token)",
                       "global_batch": 1, "seq_len": 1, "parallelism": "none (1 GPU)"},
            "roofline": None, "cpu_baseline": cpu}), flush=True)


def run_e2e(pa, args):
    """Qwen2.5-0.5B-shaped engine, 24 layers, random bf16
    weights N(0, 0.02) (seed 4), 32 requests with prompts U[64, 512] of random
    ids, 256 greedy tokens each.  value = generated tokens / wall time of the
    whole generation (prefill + decode)."""
    from vllm_lite_amd import e2e

    cfg = e2e.qwen25_05b()
    w = e2e.Weights(cfg, seed=4, device=DEV)
    w.pack()  # load-time layout step of pa_linear's weights
    n_req, max_new = 32, 256
    g = torch.Generator().manual_seed(5)
    lens = torch.randint(64, 513, (n_req,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab, (n,), generator=g).tolist() for n in lens]
    blocks = sum((n + max_new + 15) // 16 for n in lens) + 64
    eng = e2e.Engine(cfg, w, blocks, device=DEV)
    eng.generate(prompts, min(8, max_new))  # warm-up: kernels, GEMM plans, workspace
    gen, t = eng.generate(prompts, max_new)
    total = t["prefill_s"] + t["decode_s"]
    decode_step = t["decode_s"] / (max_new - 1)
    # bytes a decode step must read: every weight once, plus the K/V of the
    # batch's contexts at the mid-generation point (bf16, Hkv heads)
    kv_mid = 2 * sum(n + max_new // 2 for n in lens) * cfg.kv_heads * cfg.head_dim * 2 * cfg.layers
    step_bytes = w.nbytes() + kv_mid
    achieved = step_bytes / decode_step / 1e9
    line = {
        "metric": "end-to-end greedy generation output tokens/s (Qwen2.5-0.5B shape)",
        "value": round(n_req * max_new / total, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": max_new, "warmup": 1, "ms_per_step": round(total / max_new * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random bf16 weights N(0, 0.02), random prompt ids)",
        "config": {"workload": "config 5: Qwen2.5-0.5B-shaped engine, 24 layers, 32 requests, "
                               "prompts U[64, 512], 256 greedy tokens",
                   "global_batch": n_req, "seq_len": max(lens) + max_new,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "one decode step (weights + KV)", "bytes_per_step": step_bytes,
                     "decode_step_ms": round(decode_step * 1e3, 3),
                     "prefill_ms": round(t["prefill_s"] * 1e3, 2)},
        "cpu_baseline": None if args.no_cpu else cpu_baseline_e2e(cfg, w, lens, max_new),
    }
    print(json.dumps(line), flush=True)


def cpu_baseline_e2e(cfg, w, lens, max_new, budget_s=12.0):
    """Config 5's decode step on the host: the reference's CPU forward
    restated (crates/model/src/causal_lm/model/mod.rs:143-164, decoder block
    crates/model/src/components/decoder_block/mod.rs:157-198) in f32 over the
    same weights, batched over the 32 requests (one matmul per projection
    instead of the reference's per-sequence loop, which only makes the CPU
    figure stronger): RMSNorm, QKV projection + bias, RoPE, the new token's
    K / V into a paged f32 cache, attention through the C oracle (gather,
    expand_kv, dense softmax, OpenMP), O projection, RMSNorm, SwiGLU MLP,
    final norm and the tied LM head, greedy argmax.  Contexts are the
    mid-generation ones (prompt + max_new / 2); every layer attends the same
    seeded K / V pool (the timing does not depend on the values).  Reported
    as output tokens/s of decode steps."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    threads = cpu_threads()
    torch.set_num_threads(threads)
    f = lambda t: t.detach().float().cpu()
    L, hq, hkv, d, hid = cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.hidden
    W = {"embed": f(w.embed), "norm": f(w.norm),
         "ln1": [f(x) for x in w.ln1], "ln2": [f(x) for x in w.ln2],
         "wqkv": [f(x) for x in w.wqkv], "bqkv": [f(x) for x in w.bqkv],
         "wo": [f(x) for x in w.wo], "wgu": [f(x) for x in w.wgu], "wd": [f(x) for x in w.wd]}
    b = len(lens)
    ctx = np.array([n + max_new // 2 for n in lens], np.int32)
    nblk = (ctx + 16) // 16 + 1
    pool = int(nblk.sum())
    rng = np.random.default_rng(6)
    kc = rng.standard_normal((pool, hkv, 16, d), dtype=np.float32)
    vc = rng.standard_normal((pool, hkv, 16, d), dtype=np.float32)
    bt = np.zeros((b, int(nblk.max())), np.int32)
    o = 0
    for i in range(b):
        bt[i, :nblk[i]] = np.arange(o, o + nblk[i])
        o += nblk[i]
    inv_freq = oracle.rope_inv_freq(d, cfg.rope_theta)
    silu = torch.nn.functional.silu

    def rms(x, g):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.eps) * g

    def rope(x):  # [b, h, d] at each sequence's position (the oracle's RoPE)
        return oracle.rope(x.contiguous().numpy(), ctx, inv_freq)

    slot_blk = bt[np.arange(b), ctx // 16]
    slot_off = ctx % 16

    def step(tok):
        x = W["embed"][tok]
        for l in range(L):
            h = rms(x, W["ln1"][l])
            qkv = h @ W["wqkv"][l].T + W["bqkv"][l]
            q = rope(qkv[:, :hq * d].view(b, hq, d))
            k = rope(qkv[:, hq * d:(hq + hkv) * d].view(b, hkv, d))
            v = qkv[:, (hq + hkv) * d:].view(b, hkv, d)
            kc[slot_blk, :, slot_off, :] = k
            vc[slot_blk, :, slot_off, :] = v.numpy()
            a = oracle.paged_attention(q, kc, vc, bt, np.arange(b + 1), ctx, threads=threads)
            x = x + torch.from_numpy(a).view(b, hq * d) @ W["wo"][l].T
            h = rms(x, W["ln2"][l])
            gu = h @ W["wgu"][l].T
            act = silu(gu[:, :cfg.inter]) * gu[:, cfg.inter:]
            x = x + act @ W["wd"][l].T
        return (rms(x, W["norm"]) @ W["embed"].T).argmax(-1)

    tok = torch.zeros(b, dtype=torch.int64)
    tok = step(tok)  # warm
    t0 = time.perf_counter()
    reps = 0
    while True:
        tok = step(tok)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 20:
            break
    return {"value": round(b * reps / el, 2), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"{reps} decode steps of the 32 requests at mid-generation contexts "
                      f"({el:.1f} s): f32 batched forward over the same weights, attention "
                      "through the oracle (gather + expand_kv + dense softmax, OpenMP)"}


def copy_calibration(args):
    """Plain 1 GiB device-to-device copy: the known-size reference for
    scaling rocprof FETCH_SIZE / WRITE_SIZE, and the achievable-HBM check."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=DEV).random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        dst.copy_(src)
    stop.record()
    torch.cuda.synchronize()
    t = start.elapsed_time(stop) / args.steps / 1e3
    print(json.dumps({"config": "copy", "bytes_read": n, "bytes_written": n,
                      "avg_launch_us": round(t * 1e6, 2),
                      "gbs_read_plus_write": round(2 * n / t / 1e9, 1)}), flush=True)


def run_write(pa, args):
    """The KV-cache write of BASELINE config 3's chunk: pa_reshape_and_cache
    of 4 x 2048 new tokens (pasts 0 / 512 / 1024 / 2048, 8 kv heads x 128,
    bf16) through seeded random block tables; the slot runs are
    block-aligned, so every block goes whole.  HBM-bound: algorithmic bytes
    = K and V read + written + the slots."""
    g = torch.Generator().manual_seed(2)
    hkv, d = 8, 128
    pasts, chunk = [0, 512, 1024, 2048], 2048
    nblks = [(p + chunk + 15) // 16 for p in pasts]
    pool = sum(nblks) + 16
    perm = torch.randperm(pool, generator=g)
    slots, o = [], 0
    for p, n in zip(pasts, nblks):
        pos = torch.arange(p, p + chunk)
        slots.append(perm[o:o + n][pos // 16] * 16 + pos % 16)
        o += n
    slots = torch.cat(slots).to(torch.int64).to(DEV)
    t = slots.numel()
    dg = torch.Generator(device=DEV).manual_seed(1234)
    k = torch.randn(t, hkv, d, generator=dg, device=DEV).to(torch.bfloat16)
    v = torch.randn(t, hkv, d, generator=dg, device=DEV).to(torch.bfloat16)
    kc, vc = pa.ops.new_cache(pool, hkv, d, torch.bfloat16, DEV)

    class W:
        def attend(self):
            pa.reshape_and_cache(k, v, kc, vc, slots)
    w = W()
    for _ in range(args.warmup):
        w.attend()
    tm = time_attend(w, max(args.steps, 20))
    alg = 2 * 2 * t * hkv * d * 2 + t * 8
    achieved = alg / tm / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "pa_reshape_and_cache (cache_write_kernel, whole blocks)",
            "alg_bytes_per_launch": alg, "avg_launch_us": round(tm * 1e6, 2)}
    flushed_legs(roof, w, max(args.steps, 20), lambda x: alg / x / 1e9 / HBM_PEAK_GBS,
                 args.no_flush)
    print(json.dumps({
        "metric": "paged KV-cache write tokens/s (config 3 chunk)",
        "value": round(t / tm, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(tm * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V, random block tables)",
        "config": {"workload": "config 3 write: 4 x 2048 tokens, 8 kv heads x 128, bf16",
                   "global_batch": 4, "seq_len": chunk, "parallelism": "none (1 GPU)"},
        "roofline": roof, "cpu_baseline": None}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="decode",
                    choices=["decode", "decode-fp8", "prefill", "prefill-fp8", "splitk", "qwen",
                             "e2e", "copy", "write", "kv-rw"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-flush", action="store_true",
                    help="skip the cache-flushed timing leg (keeps a kernel trace to warm launches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the "
              "multi-GPU sharding plan is design-only.", file=sys.stderr)
        sys.exit(2)

    pa = _package()
    torch.cuda.set_device(0)
    if args.config == "copy":
        return copy_calibration(args)
    if args.config == "e2e":
        return run_e2e(pa, args)
    if args.config == "write":
        return run_write(pa, args)
    if args.config == "kv-rw":
        return run_kv_rw(pa, args)
    w = Workload(pa, args.config)
    for _ in range(args.warmup):
        w.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        w.step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_per_step = el / args.steps * 1e3

    t_attn = time_attend(w, max(args.steps, 20))
    if w.kind == "decode":
        value = w.B * args.steps / el
        unit = "tokens/s"
        achieved = w.alg_bytes / t_attn / 1e9
        traffic, traffic_src = measured_traffic(args.config)
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": traffic, "traffic_source": traffic_src,
                "alg_bytes_per_launch": w.alg_bytes,
                "avg_launch_us": round(t_attn * 1e6, 2)}
        flushed_legs(roof, w, max(args.steps, 20),
                     lambda x: w.alg_bytes / x / 1e9 / HBM_PEAK_GBS, args.no_flush)
        if args.config == "decode-fp8":
            # the same launch through pa_decode_fp8_flagged (the bench's
            # finite values leave every block flag 0)
            flags = torch.zeros(w.kc.shape[0], dtype=torch.uint8, device=DEV)

            class WF:
                def attend(self):
                    w.pa.decode(w.q, w.kc, w.vc, w.bt, w.ctx_dev, w.max_ctx, scale=w.scale,
                                out=w.out, workspace=w.ws, block_flags=flags)
            WF().attend()
            tf = time_attend(WF(), max(args.steps, 20))
            roof["flagged_launch_us"] = round(tf * 1e6, 2)
            roof["flagged_frac"] = round(w.alg_bytes / tf / 1e9 / HBM_PEAK_GBS, 4)
        if args.config == "splitk":
            roof["unique_block_gbs"] = round((w.unique_kv_bytes) / t_attn / 1e9, 1)
            # batch-order independence of the shared-prefix grouping
            bt0 = w.bt
            order = {}
            for key, inter in (("two_prefixes_ordered_us", False),
                               ("two_prefixes_interleaved_us", True)):
                w.bt = w.two_prefix_tables(inter)
                w.attend()
                order[key] = round(time_attend(w, max(args.steps, 20)) * 1e6, 2)
            w.bt = bt0
            roof["batch_order"] = order
            # the profiled HBM bytes (FETCH + WRITE) over this run's launch time
            if traffic:
                roof["physical_frac"] = round(traffic / t_attn / 1e9 / HBM_PEAK_GBS, 4)
        # configs 2 (bf16, FP8): two 2048-token partitions per (kv head,
        # sequence), merged in the workgroup; config 4: the work cut evenly over
        # the GPU, a sequence group's shared block-table prefix attended once
        # (groups and prefixes found by decode_group_kernel), partial results merged by the
        # reduce kernel; config 1 (f32): the group kernel and the reduce kernel
        roof["kernel"] = {
            "decode": "pa_decode (decode_mfma_kernel, partitions merged in the workgroup)",
            "decode-fp8": "pa_decode (decode_fp8_kernel, partitions merged in the workgroup)",
            "splitk": "pa_decode (decode_group_kernel + decode_balanced_kernel + decode_reduce_kernel)",
            "qwen": "pa_decode (decode_f32_group_kernel + decode_reduce_kernel)",
        }[args.config]
    else:
        value = w.flops / t_attn / 1e12
        unit = "TFLOP/s"
        traffic, traffic_src = measured_traffic(args.config)
        roof = {"bound": "mfma", "achieved": round(value, 2), "peak": BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(value / BF16_PEAK_TFLOPS, 4),
                "traffic": traffic, "traffic_source": traffic_src,
                "kernel": ("pa_prefill (prefill_tiled_kernel, FP8 tiles)" if w.fp8 else
                           "pa_prefill (prefill_tiled_kernel)"), "flops_per_launch": w.flops,
                "avg_launch_us": round(t_attn * 1e6, 2)}
        flushed_legs(roof, w, max(args.steps, 20),
                     lambda x: w.flops / x / 1e12 / BF16_PEAK_TFLOPS, args.no_flush)
        if not args.no_flush:
            ceil = gemm_ceiling()
            roof["gemm_ceiling_tflops"] = round(ceil, 1)
            roof["frac_of_gemm_ceiling"] = round(value / ceil, 4)
    cpu = None if args.no_cpu else cpu_baseline(w)
    line = {
        "metric": METRIC if w.kind == "decode" else "paged-attn chunked prefill TFLOP/s",
        "value": round(value, 2), "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": ("fp8-e4m3 KV, bf16 q/out" if w.fp8 else
                  "bf16" if w.dtype == torch.bfloat16 else "f32"),
        "data": "synthetic (seeded N(0,1) Q/K/V, random block tables)",
        "config": {"workload": w.workload, "global_batch": w.B,
                   "seq_len": int(w.ctx.max()) if w.kind == "decode" else 2048,
                   "parallelism": "none (1 GPU)"},
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
