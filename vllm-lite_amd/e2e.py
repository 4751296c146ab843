"""End-to-end decoder around the paged-attention path.

A Qwen2.5-0.5B-shaped causal LM (24 layers, hidden 896, 14 / 2 heads x 64,
SwiGLU 4864, RoPE theta 1e6, vocab 151,936, tied embeddings) with random bf16
weights, run the way the reference's CausalLm runs it
(crates/model/src/causal_lm/model/mod.rs:143-164, decoder block
crates/model/src/components/decoder_block/mod.rs:157-198), but batched: one
StepBatch per engine step, and per layer
    residual add + norm         pa_rms_norm | pa_layer_norm
    QKV projection (+ bias)     hipBLASLt GEMM (torch.nn.functional.linear)
    RoPE + KV write + attention StepBatch.attention (pa_batch_attention)
    O projection                hipBLASLt GEMM
    residual add + norm         pa_rms_norm | pa_layer_norm
    gate|up projection          hipBLASLt GEMM
    SwiGLU                      pa_silu_mul
    down projection             hipBLASLt GEMM
The norm is chosen explicitly by ModelConfig.norm: "rms" (RMSNorm, what the
benchmark configuration states) or "layer" (the zero-bias LayerNorm the
reference's CausalLm constructs for these models,
crates/model/src/qwen3/model.rs:19,
crates/model/src/components/decoder_block/factory.rs:42-46).  Norm weights
start at 1, every other weight is N(0, 0.02).
"""
import dataclasses
import math
import time

import torch
import torch.nn.functional as F

from . import ops
from .kv_cache import PagedKvCache, StepBatch


@dataclasses.dataclass
class ModelConfig:
    layers: int = 24
    hidden: int = 896
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    inter: int = 4864
    vocab: int = 151936
    rope_theta: float = 1e6
    eps: float = 1e-6
    norm: str = "rms"  # "rms" | "layer" (zero-bias LayerNorm)


def qwen25_05b():
    return ModelConfig()


class Weights:
    """Random weights of the configuration (bf16 on the device)."""

    def __init__(self, cfg, seed=4, device="cuda", dtype=torch.bfloat16):
        g = torch.Generator(device=device).manual_seed(seed)

        def w(*shape):
            return (torch.randn(*shape, generator=g, device=device) * 0.02).to(dtype)

        h, d = cfg.hidden, cfg.head_dim
        qkv = (cfg.heads + 2 * cfg.kv_heads) * d
        self.embed = w(cfg.vocab, h)
        self.ln1 = [torch.ones(h, dtype=dtype, device=device) for _ in range(cfg.layers)]
        self.ln2 = [torch.ones(h, dtype=dtype, device=device) for _ in range(cfg.layers)]
        self.wqkv = [w(qkv, h) for _ in range(cfg.layers)]
        self.bqkv = [w(qkv) for _ in range(cfg.layers)]
        self.wo = [w(h, cfg.heads * d) for _ in range(cfg.layers)]
        self.wgu = [w(2 * cfg.inter, h) for _ in range(cfg.layers)]
        self.wd = [w(h, cfg.inter) for _ in range(cfg.layers)]
        self.norm = torch.ones(h, dtype=dtype, device=device)

    def nbytes(self):
        ts = [self.embed, self.norm]
        for lst in (self.ln1, self.ln2, self.wqkv, self.bqkv, self.wo, self.wgu, self.wd):
            ts += lst
        return sum(t.numel() * t.element_size() for t in ts)


class Engine:
    """Batched greedy generation over one paged KV cache."""

    def __init__(self, cfg, weights, num_blocks, device="cuda", graph=True):
        """graph: capture one decode step's forward in a HIP graph and replay
        it for the following steps (the batch is re-prepared on the host
        before every replay; see StepBatch.set_capacity)."""
        self.cfg, self.w, self.device = cfg, weights, torch.device(device)
        self.graph = graph
        self.cache = PagedKvCache(cfg.layers, cfg.kv_heads, cfg.head_dim, num_blocks,
                                  torch.bfloat16, device)
        self.batch = StepBatch()
        self.inv_freq = torch.from_numpy(ops.rope_inv_freq(cfg.head_dim, cfg.rope_theta)).to(
            self.device)
        self.free = list(range(num_blocks))
        self.scale = 1.0 / math.sqrt(cfg.head_dim)
        if cfg.norm not in ("rms", "layer"):
            raise ValueError(f"unknown norm {cfg.norm!r}")
        self._norm = ops.rms_norm if cfg.norm == "rms" else ops.layer_norm

    def forward(self, tokens, logit_rows):
        """One step over the prepared batch: tokens [T] (int64, device) ->
        logits of the rows logit_rows [R, vocab] (f32)."""
        c, w = self.cfg, self.w
        t = tokens.shape[0]
        hq, hkv, d = c.heads, c.kv_heads, c.head_dim
        x = F.embedding(tokens, w.embed)          # residual stream [T, hidden]
        h = torch.empty_like(x)
        add = None
        for layer in range(c.layers):
            self._norm(x, w.ln1[layer], c.eps, add=add, out=h)
            qkv = F.linear(h, w.wqkv[layer], w.bqkv[layer])
            q = qkv[:, :hq * d].contiguous().view(t, hq, d)  # the kernels take dense q rows
            k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
            v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
            attn = self.batch.attention(self.cache, layer, q, k, v, self.inv_freq, self.scale)
            o = F.linear(attn.view(t, hq * d), w.wo[layer])
            self._norm(x, w.ln2[layer], c.eps, add=o, out=h)
            act = ops.silu_mul(F.linear(h, w.wgu[layer]))
            add = F.linear(act, w.wd[layer])
        self._norm(x, w.norm, c.eps, add=add, out=h)
        return F.linear(h[logit_rows], w.embed).float()

    def generate(self, prompts, max_new):
        """Greedy generation for every prompt (lists of token ids).  Returns
        (generated ids [B, max_new] on the host, {"prefill_s", "decode_s"})."""
        b = len(prompts)
        lens = [len(p) for p in prompts]
        blocks = []
        for n in lens:
            need = (n + max_new + 15) // 16
            if need > len(self.free):
                raise RuntimeError("KV pool exhausted")
            blocks.append([self.free.pop() for _ in range(need)])
        try:
            torch.cuda.synchronize(self.device)
            t0 = time.perf_counter()
            self.batch.prepare(self.cache, lens, [0] * b, blocks)
            tokens = torch.tensor([x for p in prompts for x in p], dtype=torch.int64,
                                  device=self.device)
            last = torch.tensor([sum(lens[:i + 1]) - 1 for i in range(b)], device=self.device)
            nxt = self.forward(tokens, last).argmax(-1)
            out = [nxt]
            torch.cuda.synchronize(self.device)
            t1 = time.perf_counter()
            rows = torch.arange(b, device=self.device)
            self.batch.set_capacity(max(lens) + max_new if self.graph else 0)
            graph = static_tok = static_out = None
            for step in range(1, max_new):
                self.batch.prepare(self.cache, [1] * b, [n + step - 1 for n in lens], blocks)
                if not self.graph or step == 1:
                    # eager (also the warm-up of every launch the graph records)
                    nxt = self.forward(nxt, rows).argmax(-1)
                else:
                    if graph is None:
                        static_tok = nxt.clone()
                        graph = torch.cuda.CUDAGraph()
                        with torch.cuda.graph(graph):
                            static_out = self.forward(static_tok, rows).argmax(-1)
                    else:
                        static_tok.copy_(nxt)
                    graph.replay()
                    nxt = static_out.clone()
                out.append(nxt)
            gen = torch.stack(out, 1).cpu()
            t2 = time.perf_counter()
        finally:
            self.batch.set_capacity(0)
            for blk in blocks:
                self.free.extend(blk)
        return gen, {"prefill_s": t1 - t0, "decode_s": t2 - t1}
