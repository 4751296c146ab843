"""PagedKvCache: Python face of the C++ cache mirror (pa_kv_cache_*).

Method names and argument meanings follow the reference's PagedKvCache
(crates/model/src/paged_tensor/tensor_store/{mod.rs,buffer.rs}) and the
paged_gqa free functions (crates/model/src/components/attention/
paged_gqa.rs:29-112); failures the reference reports as Err raise PaError.
Index arguments are host-side lists; K/V payloads are device tensors in the
cache dtype, laid out [T, H, D] (one token: [H, D] or [1, H, D]).
"""
import ctypes as C

import torch

from . import _lib
from .ops import BLOCK_SIZE, PaError, _DTYPES, _check

_DT_BACK = {v: k for k, v in _DTYPES.items()}


def _i64_array(xs):
    xs = [int(x) for x in xs]
    return (C.c_int64 * max(len(xs), 1))(*xs), len(xs)


class PagedKvCache:
    """quantized=True mirrors PagedKvCache::new(..., quantized = true): an f32
    cache of int8 values with one scale per block (re-quantised per write)."""

    def __init__(self, num_layers, num_heads, head_dim, num_blocks, dtype=torch.float32,
                 device="cuda", quantized=False):
        self._lib = _lib.load()
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.dtype = dtype
        self.num_heads = num_heads
        self.head_dim = head_dim
        h = C.c_void_p()
        if quantized and dtype != torch.float32:
            raise ValueError("quantised caches are f32")
        self.quantized = quantized
        with torch.cuda.device(self.device):
            if quantized:
                _check("pa_kv_cache_create_quantized", self._lib.pa_kv_cache_create_quantized(
                    num_layers, num_heads, head_dim, num_blocks, C.byref(h)))
            else:
                _check("pa_kv_cache_create", self._lib.pa_kv_cache_create(
                    num_layers, num_heads, head_dim, num_blocks, _DTYPES[dtype], C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            self._lib.pa_kv_cache_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # accessors -----------------------------------------------------------
    def num_layers(self):
        return self._lib.pa_kv_cache_num_layers(self._h)

    def num_blocks(self):
        return self._lib.pa_kv_cache_num_blocks(self._h)

    def block_size(self):
        return self._lib.pa_kv_cache_block_size(self._h)

    def key_cache(self, layer):
        """Device tensor view of one layer's K cache [NB, H, 16, D]."""
        return self._layer_tensor(self._lib.pa_kv_cache_key_ptr(self._h, layer),
                                  (self.num_blocks(), self.num_heads, BLOCK_SIZE, self.head_dim))

    def value_cache(self, layer):
        """Device tensor view of one layer's V cache [NB, H, D, 16]."""
        return self._layer_tensor(self._lib.pa_kv_cache_value_ptr(self._h, layer),
                                  (self.num_blocks(), self.num_heads, self.head_dim, BLOCK_SIZE))

    def scales(self, layer):
        """Device tensor view of one layer's block scales [NB] (quantised only)."""
        if not self.quantized:
            raise ValueError("cache is not quantised")
        ptr = self._lib.pa_kv_cache_scales_ptr(self._h, layer)
        if not ptr:
            raise PaError("pa_kv_cache_scales_ptr", -2, "layer out of bounds")
        n = self.num_blocks()
        iface = {"shape": (n * 4,), "typestr": "|u1", "data": (ptr, False), "strides": None,
                 "version": 3}

        class _Buf:
            __cuda_array_interface__ = iface

        return torch.as_tensor(_Buf(), device=self.device).view(torch.float32)

    def _layer_tensor(self, ptr, shape):
        if not ptr:
            raise PaError("pa_kv_cache layer", -2, "layer out of bounds")
        es = torch.empty(0, dtype=self.dtype).element_size()
        n = 1
        for s in shape:
            n *= s
        # Wrap the library-owned buffer without copying; the view must not
        # outlive this cache.
        iface = {"shape": (n * es,), "typestr": "|u1", "data": (ptr, False), "strides": None,
                 "version": 3}

        class _Buf:
            __cuda_array_interface__ = iface

        raw = torch.as_tensor(_Buf(), device=self.device)
        return raw.view(self.dtype).view(shape)

    # reference operations ------------------------------------------------
    def _stream(self):
        return C.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)

    def _payload(self, k, v, tokens=None):
        """Checks a K/V pair the way write_kv / write_kv_batch do
        (buffer.rs:139-165, :42-67): same shape, trailing dims [H, D], and
        the expected token count; returns contiguous tensors and T."""
        for x in (k, v):
            if x.device != self.device or x.dtype != self.dtype:
                raise ValueError("payload must be a device tensor in the cache dtype")
        if tuple(k.shape) != tuple(v.shape):
            raise ValueError(f"k and v must have same dimensions, got {tuple(k.shape)} vs "
                             f"{tuple(v.shape)}")
        if k.dim() < 2 or tuple(k.shape[-2:]) != (self.num_heads, self.head_dim):
            raise ValueError(f"expected k shape [.., {self.num_heads}, {self.head_dim}], got "
                             f"{tuple(k.shape)}")
        t = k.numel() // (self.num_heads * self.head_dim)
        if tokens is not None and t != tokens:
            raise ValueError(f"expected {tokens} token(s), got {t}")
        return k.contiguous(), v.contiguous(), t

    def write_kv(self, layer_idx, block_id, token_offset, k, v):
        """PagedKvCache::write_kv (buffer.rs:103-267)."""
        k, v, _ = self._payload(k, v, 1)
        _check("write_kv", self._lib.pa_kv_cache_write_kv(
            self._h, layer_idx, block_id, token_offset, C.c_void_p(k.data_ptr()),
            C.c_void_p(v.data_ptr()), self._stream()))

    def write_kv_batch(self, layer_idx, block_id, token_offset, k_batch, v_batch):
        """PagedKvCache::write_kv_batch (buffer.rs:27-95); k/v [T, H, D]."""
        k, v, t = self._payload(k_batch, v_batch)
        _check("write_kv_batch", self._lib.pa_kv_cache_write_kv_batch(
            self._h, layer_idx, block_id, token_offset, C.c_void_p(k.data_ptr()),
            C.c_void_p(v.data_ptr()), t, self._stream()))

    def write_prefill_kv(self, layer_idx, block_ids, positions, seq_len, k, v):
        """write_prefill_kv (paged_gqa.rs:29-63); k/v [seq_len, H, D]."""
        k, v, _ = self._payload(k, v, seq_len)
        ids, n_ids = _i64_array(block_ids)
        pos, n_pos = _i64_array(positions)
        _check("write_prefill_kv", self._lib.pa_kv_cache_write_prefill_kv(
            self._h, layer_idx, ids, n_ids, pos, n_pos, seq_len, C.c_void_p(k.data_ptr()),
            C.c_void_p(v.data_ptr()), self._stream()))

    def read_kv(self, layer_idx, block_ids, seq_len):
        """PagedKvCache::read_kv (buffer.rs:273-339) -> (k, v) [n, H, D]."""
        ids, n_ids = _i64_array(block_ids)
        cover = min(seq_len, n_ids * BLOCK_SIZE) if n_ids and seq_len > 0 else 0
        out_k = torch.empty(cover, self.num_heads, self.head_dim, dtype=self.dtype,
                            device=self.device)
        out_v = torch.empty_like(out_k)
        n = C.c_int32(0)
        _check("read_kv", self._lib.pa_kv_cache_read_kv(
            self._h, layer_idx, ids, n_ids, seq_len,
            C.c_void_p(out_k.data_ptr()) if cover else None,
            C.c_void_p(out_v.data_ptr()) if cover else None, C.byref(n), self._stream()))
        return out_k[: n.value], out_v[: n.value]

    def block_hashes(self, layer_idx):
        """The layer's block-hash map (PagedKvCache::block_hashes,
        tensor_store/mod.rs:42): {hash: block_id}, filled by every write
        (buffer.rs:263-264)."""
        cnt = C.c_int64(0)
        _check("block_hash_count", self._lib.pa_kv_cache_block_hash_count(
            self._h, layer_idx, C.byref(cnt)))
        n = max(cnt.value, 1)
        hs, ids = (C.c_uint64 * n)(), (C.c_int64 * n)()
        got = C.c_int64(0)
        _check("block_hashes", self._lib.pa_kv_cache_block_hashes(
            self._h, layer_idx, hs, ids, cnt.value, C.byref(got)))
        return {int(hs[i]): int(ids[i]) for i in range(got.value)}

    def lookup_block_hash(self, layer_idx, h):
        """The block id recorded for hash h in the layer's map, or None."""
        bid = C.c_int64(0)
        _check("lookup_block_hash", self._lib.pa_kv_cache_lookup_block_hash(
            self._h, layer_idx, C.c_uint64(h), C.byref(bid)))
        return None if bid.value < 0 else bid.value


class StepBatch:
    """One engine step's batch for every layer (pa_batch_*).

    Built from the scheduler's per-sequence view of a step (the Batch of
    crates/traits/src/types.rs:84-117): tokens fed this step, tokens already
    cached, and each sequence's block ids.  attention() then runs one
    layer's KV write (with RoPE when inv_freq is given) and attention for
    all sequences, in place of the reference's per-sequence loop
    (crates/model/src/causal_lm/model/mod.rs:143-164)."""

    def __init__(self):
        self._lib = _lib.load()
        h = C.c_void_p()
        _check("pa_batch_create", self._lib.pa_batch_create(C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            self._lib.pa_batch_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prepare(self, cache, num_tokens, num_computed, block_ids):
        """num_tokens / num_computed: per-sequence ints; block_ids: list of
        per-sequence lists.  The uploads are queued on the current stream
        (not waited for); the batch's launches must use the same stream."""
        n = len(num_tokens)
        if len(num_computed) != n or len(block_ids) != n:
            raise ValueError("per-sequence lists must have equal length")
        nt = (C.c_int32 * max(n, 1))(*[int(x) for x in num_tokens])
        nc = (C.c_int32 * max(n, 1))(*[int(x) for x in num_computed])
        cnt = (C.c_int32 * max(n, 1))(*[len(b) for b in block_ids])
        flat = [int(x) for b in block_ids for x in b]
        ids = (C.c_int64 * max(len(flat), 1))(*flat)
        _check("pa_batch_prepare", self._lib.pa_batch_prepare(
            self._h, n, nt, nc, ids, cnt, cache.num_blocks(), cache._stream()))

    def num_tokens(self):
        return self._lib.pa_batch_num_tokens(self._h)

    def advance(self, cache):
        """pa_batch_advance: the prepared decode step moved one token on,
        on the device (no upload), on the cache's stream; capturable, so a
        captured decode step can advance itself on every replay."""
        _check("pa_batch_advance", self._lib.pa_batch_advance(self._h, cache._stream()))

    def set_capacity(self, max_context_len):
        """pa_batch_set_capacity: shape decode launches for a fixed maximum
        context so a captured step can be replayed (0 = per step)."""
        _check("pa_batch_set_capacity", self._lib.pa_batch_set_capacity(self._h,
                                                                          int(max_context_len)))

    def is_decode(self):
        return bool(self._lib.pa_batch_is_decode(self._h))

    def qkv_rope_cache(self, cache, layer, x, weight, bias, inv_freq, rms_eps=None):
        """pa_batch_qkv_rope_cache: the step's fused QKV projection of x
        [T, K] with RoPE and the KV-cache write in its epilogue; weight a
        PackedWeight with rope_heads.  Returns [T, (Hq + 2 Hkv) D]; pass its
        q view to attention() with key = value = None."""
        if weight.rope_heads is None:
            raise ValueError("qkv_rope_cache takes a PackedWeight with rope_heads")
        hq, hkv, d = weight.rope_heads
        t, k = x.shape
        if t != self.num_tokens() or hkv != cache.num_heads or d != cache.head_dim:
            raise ValueError("x / weight do not match the batch and cache")
        if x.dtype != cache.dtype or not x.is_contiguous() or x.device != cache.device:
            raise ValueError("x must be contiguous, on the cache's device and dtype")
        if inv_freq.dtype != torch.float32 or inv_freq.shape != (d // 2,):
            raise ValueError("inv_freq must be float32 [D/2]")
        out = torch.empty(t, weight.shape[0], dtype=x.dtype, device=x.device)
        _check("pa_batch_qkv_rope_cache", self._lib.pa_batch_qkv_rope_cache(
            self._h, cache._h, layer, hq, C.c_void_p(out.data_ptr()), C.c_void_p(x.data_ptr()),
            C.c_void_p(weight.data.data_ptr()),
            C.c_void_p(bias.data_ptr()) if bias is not None else None, k,
            1 if rms_eps is not None else 0, float(rms_eps) if rms_eps is not None else 0.0,
            C.c_void_p(inv_freq.data_ptr()), cache._stream()))
        return out

    def attention(self, cache, layer, q, key, value, inv_freq=None, scale=None):
        """q [T, Hq, D] (rotated in place with inv_freq), key / value
        [T, Hkv, D] (rows of all three may be strided views of a fused
        projection) -> out [T, Hq, D].  key = value = None: the step's K / V
        are already in the cache and q is final (qkv_rope_cache)."""
        t, hq, d = q.shape
        if t != self.num_tokens():
            raise ValueError(f"batch has {self.num_tokens()} tokens, q has {t}")
        if (key is None) != (value is None) or (key is None and inv_freq is not None):
            raise ValueError("key and value both or neither; no inv_freq without them")
        if key is not None and (key.shape != (t, cache.num_heads, d) or
                                value.shape != key.shape):
            raise ValueError("key / value must be [T, Hkv, D]")
        for x in (q, key, value):
            if x is None:
                continue
            if x.dtype != cache.dtype or x.device != cache.device or x.stride(2) != 1 or \
                    x.stride(1) != d or (t > 1 and x.stride(0) < x.shape[1] * d):
                raise ValueError("q / key / value rows must be [H, D] in the cache dtype, "
                                 "token rows not overlapping")
        if inv_freq is not None and (inv_freq.dtype != torch.float32 or
                                     inv_freq.shape != (d // 2,)):
            raise ValueError("inv_freq must be float32 [D/2]")
        if scale is None:
            scale = 1.0 / d ** 0.5
        out = torch.empty_like(q)
        _check("pa_batch_attention", self._lib.pa_batch_attention(
            self._h, cache._h, layer, hq, C.c_void_p(q.data_ptr()), q.stride(0),
            C.c_void_p(key.data_ptr()) if key is not None else None,
            key.stride(0) if key is not None else 0,
            C.c_void_p(value.data_ptr()) if value is not None else None,
            value.stride(0) if value is not None else 0, C.c_void_p(inv_freq.data_ptr()) if inv_freq is not None else None,
            float(scale), C.c_void_p(out.data_ptr()), cache._stream()))
        return out
