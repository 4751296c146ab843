"""torch-tensor wrappers of the stateless C entry points of libpa.so.

Tensors are passed by device pointer; work goes on the current HIP stream of
the tensors' device.  Each wrapper checks dtype, device, contiguity and
shape before calling, and raises PaError with the library's message when a
call returns a non-zero status.
"""
import ctypes as C
import math

import torch

from . import _lib

BLOCK_SIZE = 16
_DTYPES = {torch.float32: 0, torch.bfloat16: 1}
# FP8-E4M3 caches (the reference's codes) are uint8 tensors; q / out are bf16.
FP8 = 2


class PaError(RuntimeError):
    """A libpa entry point returned a negative pa_status."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def _check(fn, rc):
    if rc != 0:
        raise PaError(fn, rc, _lib.load().pa_last_error().decode())


def _stream(t):
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _dev(*ts):
    for t in ts:
        if not (t.is_cuda and t.is_contiguous()):
            raise ValueError("expected contiguous device tensors")


def _dtype_code(t):
    if t.dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype {t.dtype}")
    return _DTYPES[t.dtype]


def new_cache(num_blocks, num_kv_heads, head_dim, dtype, device="cuda"):
    """Zeroed (k_cache [NB, H, 16, D], v_cache [NB, H, D, 16]) for one layer;
    dtype torch.uint8 makes FP8-E4M3 caches."""
    k = torch.zeros(num_blocks, num_kv_heads, BLOCK_SIZE, head_dim, dtype=dtype, device=device)
    v = torch.zeros(num_blocks, num_kv_heads, head_dim, BLOCK_SIZE, dtype=dtype, device=device)
    return k, v


def _cache_dims(k_cache, v_cache):
    nb, h, bs, d = k_cache.shape
    if bs != BLOCK_SIZE or tuple(v_cache.shape) != (nb, h, d, BLOCK_SIZE):
        raise ValueError("caches must be K [NB, H, 16, D] and V [NB, H, D, 16]")
    if k_cache.dtype != v_cache.dtype:
        raise ValueError("K and V caches differ in dtype")
    return nb, h, d


def _rows_ok(x, h, d):
    """Token rows [H, D] of x [T, H, D]: contiguous within a row, and rows
    that do not overlap (a token stride of at least H * D; the C ABI reads a
    stride of 0 as "contiguous")."""
    return (x.stride(2) == 1 and x.stride(1) == d and
            (x.shape[0] <= 1 or x.stride(0) >= h * d))


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping):
    """Scatter key/value [T, H, D] into the caches at slot_mapping [T] (int64)."""
    _dev(k_cache, v_cache, slot_mapping)
    nb, h, d = _cache_dims(k_cache, v_cache)
    t = key.shape[0]
    if key.shape[1:] != (h, d) or value.shape != key.shape or slot_mapping.shape != (t,):
        raise ValueError("key/value must be [T, H, D] matching the cache; slot_mapping [T]")
    if slot_mapping.dtype != torch.int64 or key.dtype != k_cache.dtype or value.dtype != k_cache.dtype:
        raise ValueError("dtype mismatch")
    if not (_rows_ok(key, h, d) and _rows_ok(value, h, d)):
        raise ValueError("key/value rows must be contiguous [H, D], not overlapping")
    lib = _lib.load()
    _check("pa_reshape_and_cache", lib.pa_reshape_and_cache(
        _ptr(key), _ptr(value), _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping), t, h, d, nb,
        key.stride(0), value.stride(0), _dtype_code(k_cache), _stream(k_cache)))


def _cache_code(k_cache, q=None):
    """dtype code of a (q, cache) pair: uint8 caches are FP8 with bf16 q."""
    if k_cache.dtype == torch.uint8:
        if q is not None and q.dtype != torch.bfloat16:
            raise ValueError("FP8 caches take bf16 q")
        return FP8
    if q is not None and q.dtype != k_cache.dtype:
        raise ValueError("q must be in the cache dtype")
    return _dtype_code(k_cache)


def reshape_and_cache_fp8(key, value, k_cache, v_cache, slot_mapping, block_flags=None):
    """Quantise key/value [T, H, D] (f32 or bf16) into uint8 FP8 caches at
    slot_mapping [T] (int64), with the reference's E4M3 encoder.
    block_flags (uint8 [NB]): pa_reshape_and_cache_fp8_flagged, which also
    sets the flag of every block that receives a NaN / inf code."""
    _dev(k_cache, v_cache, slot_mapping)
    nb, h, d = _cache_dims(k_cache, v_cache)
    if k_cache.dtype != torch.uint8:
        raise ValueError("FP8 caches are uint8")
    t = key.shape[0]
    if key.shape[1:] != (h, d) or value.shape != key.shape or slot_mapping.shape != (t,):
        raise ValueError("key/value must be [T, H, D] matching the cache; slot_mapping [T]")
    if slot_mapping.dtype != torch.int64 or value.dtype != key.dtype:
        raise ValueError("dtype mismatch")
    if not (_rows_ok(key, h, d) and _rows_ok(value, h, d)):
        raise ValueError("key/value rows must be contiguous [H, D], not overlapping")
    lib = _lib.load()
    if block_flags is not None:
        _flags(block_flags, nb)
        _check("pa_reshape_and_cache_fp8_flagged", lib.pa_reshape_and_cache_fp8_flagged(
            _ptr(key), _ptr(value), _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping), t, h, d,
            nb, key.stride(0), value.stride(0), _dtype_code(key), _ptr(block_flags),
            _stream(k_cache)))
        return
    _check("pa_reshape_and_cache_fp8", lib.pa_reshape_and_cache_fp8(
        _ptr(key), _ptr(value), _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping), t, h, d, nb,
        key.stride(0), value.stride(0), _dtype_code(key), _stream(k_cache)))


def _flags(block_flags, nb):
    _dev(block_flags)
    if block_flags.dtype != torch.uint8 or block_flags.shape != (nb,):
        raise ValueError("block_flags must be uint8 [num_blocks]")


def slot_mapping(block_tables, positions, cu_seq_tokens):
    """Device slot mapping from block tables [B, MBS] (int32), positions [T]
    (int64) and cumulative token counts [B + 1] (int32)."""
    _dev(block_tables, positions, cu_seq_tokens)
    b, mbs = block_tables.shape
    out = torch.empty(positions.shape[0], dtype=torch.int64, device=positions.device)
    lib = _lib.load()
    _check("pa_slot_mapping", lib.pa_slot_mapping(
        _ptr(block_tables), mbs, _ptr(positions), _ptr(cu_seq_tokens), b, positions.shape[0],
        _ptr(out), _stream(positions)))
    return out


def read_kv(k_cache, v_cache, block_ids, seq_len):
    """Gather one sequence's first seq_len tokens -> (k, v) [seq_len, H, D]
    (f32 dequantised values for FP8 caches)."""
    _dev(k_cache, v_cache, block_ids)
    nb, h, d = _cache_dims(k_cache, v_cache)
    odt = torch.float32 if k_cache.dtype == torch.uint8 else k_cache.dtype
    out_k = torch.empty(seq_len, h, d, dtype=odt, device=k_cache.device)
    out_v = torch.empty_like(out_k)
    lib = _lib.load()
    _check("pa_read_kv", lib.pa_read_kv(
        _ptr(k_cache), _ptr(v_cache), _ptr(block_ids), block_ids.shape[0], seq_len, h, d, nb,
        _ptr(out_k), _ptr(out_v), _cache_code(k_cache), _stream(k_cache)))
    return out_k, out_v


def block_hash(k_cache, block_ids):
    """Reference block-content hash of each listed block (f32 cache);
    returns int64 holding the u64 bit patterns."""
    _dev(k_cache, block_ids)
    if k_cache.dtype != torch.float32:
        raise ValueError("block_hash is defined on f32 caches")
    nb, h, _, d = k_cache.shape
    out = torch.empty(block_ids.shape[0], dtype=torch.int64, device=k_cache.device)
    lib = _lib.load()
    _check("pa_block_hash", lib.pa_block_hash(
        _ptr(k_cache), _ptr(block_ids), block_ids.shape[0], h, d, nb, _ptr(out),
        _stream(k_cache)))
    return out


def decode_workspace_size(num_seqs, num_heads, head_dim, max_context_len):
    return int(_lib.load().pa_decode_workspace_size(num_seqs, num_heads, head_dim,
                                                     max_context_len))


def decode(q, k_cache, v_cache, block_tables, context_lens, max_context_len, scale=None,
           out=None, workspace=None, block_scales=None, block_flags=None):
    """Decode attention: q [B, Hq, D] -> out [B, Hq, D].  block_scales
    (f32 [NB]) marks the f32 caches as quantised (pa_decode_quantized);
    block_flags (uint8 [NB]) FP8 caches written with flags
    (pa_decode_fp8_flagged)."""
    _dev(q, k_cache, v_cache, block_tables, context_lens)
    nb, hkv, d = _cache_dims(k_cache, v_cache)
    b, hq, dq = q.shape
    if dq != d:
        raise ValueError("q must be [B, Hq, D]")
    code = _cache_code(k_cache, q)
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise ValueError("block_tables / context_lens must be int32")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    need = decode_workspace_size(b, hq, d, max_context_len)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    lib = _lib.load()
    if block_scales is not None:
        _quant_scales(block_scales, k_cache, nb)
        _check("pa_decode_quantized", lib.pa_decode_quantized(
            _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_scales),
            _ptr(block_tables), block_tables.shape[1], _ptr(context_lens), max_context_len, b, hq,
            hkv, d, nb, float(scale), _ptr(workspace), ws_bytes, _stream(q)))
        return out
    if block_flags is not None:
        if k_cache.dtype != torch.uint8:
            raise ValueError("block_flags are for FP8 caches")
        _flags(block_flags, nb)
        _check("pa_decode_fp8_flagged", lib.pa_decode_fp8_flagged(
            _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables),
            block_tables.shape[1], _ptr(context_lens), max_context_len, b, hq, hkv, d, nb,
            float(scale), _ptr(workspace), ws_bytes, _ptr(block_flags), _stream(q)))
        return out
    _check("pa_decode", lib.pa_decode(
        _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables),
        block_tables.shape[1], _ptr(context_lens), max_context_len, b, hq, hkv, d, nb,
        float(scale), _ptr(workspace), ws_bytes, code, _stream(q)))
    return out


def _quant_scales(block_scales, k_cache, nb):
    _dev(block_scales)
    if block_scales.dtype != torch.float32 or block_scales.shape != (nb,):
        raise ValueError("block_scales must be f32 [num_blocks]")
    if k_cache.dtype != torch.float32:
        raise ValueError("quantised caches are f32")


def prefill(q, k_cache, v_cache, block_tables, cu_q_lens, past_lens, max_q_len, scale=None,
            out=None, block_scales=None):
    """Chunked causal prefill: q [total_q, Hq, D] -> out [total_q, Hq, D].
    block_scales (f32 [NB]) marks the f32 caches as quantised."""
    _dev(q, k_cache, v_cache, block_tables, cu_q_lens, past_lens)
    nb, hkv, d = _cache_dims(k_cache, v_cache)
    tq, hq, dq = q.shape
    if dq != d:
        raise ValueError("q must be [total_q, Hq, D]")
    code = _cache_code(k_cache, q)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        out = torch.empty_like(q)
    lib = _lib.load()
    if block_scales is not None:
        _quant_scales(block_scales, k_cache, nb)
        _check("pa_prefill_quantized", lib.pa_prefill_quantized(
            _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_scales),
            _ptr(block_tables), block_tables.shape[1], _ptr(cu_q_lens), _ptr(past_lens),
            block_tables.shape[0], tq, max_q_len, hq, hkv, d, nb, float(scale), _stream(q)))
        return out
    _check("pa_prefill", lib.pa_prefill(
        _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(block_tables),
        block_tables.shape[1], _ptr(cu_q_lens), _ptr(past_lens), block_tables.shape[0], tq,
        max_q_len, hq, hkv, d, nb, float(scale), code, _stream(q)))
    return out


ROPE_TYPES = {"default": 0, "linear": 1, "yarn": 2, "dynamic": 3, "su": 4}


def rope_inv_freq(head_dim, theta, rope_type="default", factor=1.0, original_max_position=0,
                  cur_seq_len=0, short_factor=None, long_factor=None):
    """Host RoPE inverse-frequency table (numpy float32 [head_dim // 2])."""
    import numpy as np

    out = np.zeros(head_dim // 2, dtype=np.float32)

    def arr(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=np.float32)
        return a.ctypes.data_as(C.c_void_p)

    sf = None if short_factor is None else np.ascontiguousarray(short_factor, dtype=np.float32)
    lf = None if long_factor is None else np.ascontiguousarray(long_factor, dtype=np.float32)
    lib = _lib.load()
    _check("pa_rope_inv_freq", lib.pa_rope_inv_freq(
        head_dim, float(theta), ROPE_TYPES[rope_type], float(factor), int(original_max_position),
        int(cur_seq_len), arr(sf), arr(lf), out.ctypes.data_as(C.c_void_p)))
    return out


def rope_reshape_and_cache(q, key, value, k_cache, v_cache, slot_mapping, positions, inv_freq):
    """Rotate q [T, Hq, D] in place; rotate key [T, Hkv, D] into the K cache
    and copy value into the V cache at slot_mapping (int64); positions int64,
    inv_freq float32 [D/2] on the device."""
    _dev(k_cache, v_cache, slot_mapping, positions, inv_freq)
    nb, h, d = _cache_dims(k_cache, v_cache)
    t, hq, dq = q.shape
    if dq != d or key.shape[1:] != (h, d) or value.shape != key.shape or key.shape[0] != t:
        raise ValueError("q [T, Hq, D], key/value [T, Hkv, D] must match the cache")
    if positions.shape != (t,) or slot_mapping.shape != (t,) or inv_freq.shape != (d // 2,):
        raise ValueError("positions / slot_mapping [T], inv_freq [D/2]")
    if positions.dtype != torch.int64 or slot_mapping.dtype != torch.int64 or \
            inv_freq.dtype != torch.float32:
        raise ValueError("positions / slot_mapping int64, inv_freq float32")
    for x in (q, key, value):
        if x.dtype != k_cache.dtype or not x.is_cuda or not _rows_ok(x, x.shape[1], d):
            raise ValueError("q/key/value rows must be contiguous [H, D] in the cache dtype, "
                             "not overlapping")
    lib = _lib.load()
    _check("pa_rope_reshape_and_cache", lib.pa_rope_reshape_and_cache(
        _ptr(q), q.stride(0), _ptr(key), key.stride(0), _ptr(value), value.stride(0),
        _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping), _ptr(positions), _ptr(inv_freq), t, hq,
        h, d, nb, _dtype_code(k_cache), _stream(q)))


def _norm_args(residual, weight, add, out, bias=None):
    _dev(residual, weight)
    rows, hidden = residual.shape
    for name, t in (("weight", weight), ("bias", bias)):
        if t is not None and (t.shape != (hidden,) or t.dtype != residual.dtype):
            raise ValueError(f"{name} must be [hidden] in the residual dtype")
    if bias is not None:
        _dev(bias)
    if add is not None:
        _dev(add)
        if add.shape != residual.shape or add.dtype != residual.dtype:
            raise ValueError("add must match residual")
    if out is None:
        out = torch.empty_like(residual)
    return rows, hidden, out


def rms_norm(residual, weight, eps, add=None, out=None):
    """pa_rms_norm: residual += add (in place, when given), then
    out = residual / sqrt(mean(residual^2) + eps) * weight; [rows, hidden]."""
    rows, hidden, out = _norm_args(residual, weight, add, out)
    lib = _lib.load()
    _check("pa_rms_norm", lib.pa_rms_norm(
        _ptr(out), _ptr(residual), _ptr(add), _ptr(weight), rows, hidden, float(eps),
        _dtype_code(residual), _stream(residual)))
    return out


def layer_norm(residual, weight, eps, bias=None, add=None, out=None):
    """pa_layer_norm (LnLayerNorm, crates/model/src/components/norm/layer_norm.rs:26-39):
    residual += add (in place, when given), then
    out = (residual - mean) / sqrt(var + eps) * weight + bias; [rows, hidden]."""
    rows, hidden, out = _norm_args(residual, weight, add, out, bias)
    lib = _lib.load()
    _check("pa_layer_norm", lib.pa_layer_norm(
        _ptr(out), _ptr(residual), _ptr(add), _ptr(weight), _ptr(bias), rows, hidden,
        float(eps), _dtype_code(residual), _stream(residual)))
    return out


def silu_mul(gate_up, out=None):
    """pa_silu_mul: gate_up [rows, 2 * inter] -> silu(gate) * up [rows, inter]."""
    _dev(gate_up)
    rows, two = gate_up.shape
    inter = two // 2
    if out is None:
        out = torch.empty(rows, inter, dtype=gate_up.dtype, device=gate_up.device)
    lib = _lib.load()
    _check("pa_silu_mul", lib.pa_silu_mul(_ptr(out), _ptr(gate_up), rows, inter,
                                          _dtype_code(gate_up), _stream(gate_up)))
    return out


def argmax(logits, out=None):
    """pa_argmax: greedy token ids of logit rows [rows, vocab] (bf16 or f32,
    unit stride along the vocab) -> int64 [rows]; the first index of the
    largest value, NaN never chosen, 0 for a row with nothing above -inf
    (argmax_logits, crates/traits/src/sampling.rs:439-453)."""
    if not logits.is_cuda:
        raise ValueError("argmax: expected a device tensor")
    if logits.dim() != 2 or (logits.shape[1] > 1 and logits.stride(1) != 1):
        raise ValueError("argmax: logits must be [rows, vocab] with unit column stride")
    rows, cols = logits.shape
    if rows > 1 and logits.stride(0) < cols:
        logits = logits.contiguous()  # rows that overlap (e.g. an expanded view)
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    lib = _lib.load()
    _check("pa_argmax", lib.pa_argmax(_ptr(out), _ptr(logits), rows, cols,
                                      logits.stride(0) if rows > 1 else cols,
                                      _dtype_code(logits), _stream(logits)))
    return out


ACT_NONE, ACT_SILU_MUL = 0, 1
LINEAR_RMS_IN, LINEAR_ADD_OUT = 1, 2


class PackedWeight:
    """A bf16 weight [N, K] repacked by pa_linear_pack (see pa_dense.h); pass
    it to linear() in place of the row-major tensor.  col_scale [K] (bf16):
    folded into the columns (a norm weight in front of the projection).
    rope_heads=(num_heads, num_kv_heads, head_dim): the fused QKV weight
    packed by pa_linear_pack_qkv for linear_rope_cache (rotation pairs in
    one wavefront); linear() does not take it."""

    def __init__(self, weight, col_scale=None, rope_heads=None):
        _dev(weight)
        if not weight.is_contiguous():
            raise ValueError("pa_linear_pack takes a contiguous weight")
        if col_scale is not None and (col_scale.shape != (weight.shape[1],) or
                                      col_scale.dtype != weight.dtype):
            raise ValueError("col_scale must be [K] in the weight's dtype")
        self.shape = tuple(weight.shape)
        self.dtype = weight.dtype
        self.data = torch.empty_like(weight)
        self.rope_heads = tuple(rope_heads) if rope_heads is not None else None
        lib = _lib.load()
        if rope_heads is None:
            _check("pa_linear_pack", lib.pa_linear_pack(
                _ptr(self.data), _ptr(weight), _ptr(col_scale), weight.shape[0],
                weight.shape[1], _dtype_code(weight), _stream(weight)))
        else:
            hq, hkv, d = rope_heads
            if weight.shape[0] != (hq + 2 * hkv) * d:
                raise ValueError(f"weight {self.shape} is not a fused QKV weight of "
                                 f"{hq} + 2 x {hkv} heads of {d}")
            _check("pa_linear_pack_qkv", lib.pa_linear_pack_qkv(
                _ptr(self.data), _ptr(weight), _ptr(col_scale), hq, hkv, d, weight.shape[1],
                _dtype_code(weight), _stream(weight)))


def linear_rope_cache(x, weight, bias, positions, slot_mapping, inv_freq, k_cache, v_cache,
                      rms_eps=None, out=None):
    """pa_linear_rope_cache: the fused QKV projection of x [rows, K] with q and
    k rotated (positions [rows] int64, inv_freq [D/2] f32) and each token's
    k / v written to its slot (slot_mapping [rows] int64) of the caches
    (k_cache [NB, Hkv, 16, D], token-minor v_cache [NB, Hkv, D, 16], bf16).
    weight: PackedWeight(w_qkv, rope_heads=(Hq, Hkv, D)).  Returns out
    [rows, (Hq + 2 Hkv) D] (rotated q and k, v)."""
    if not isinstance(weight, PackedWeight) or weight.rope_heads is None:
        raise ValueError("linear_rope_cache takes a PackedWeight with rope_heads")
    hq, hkv, d = weight.rope_heads
    _dev(x, weight.data, positions, slot_mapping, inv_freq, k_cache, v_cache)
    rows, k = x.shape
    if weight.shape[1] != k:
        raise ValueError(f"weight {weight.shape} does not match x {tuple(x.shape)}")
    if positions.shape != (rows,) or slot_mapping.shape != (rows,) or \
            positions.dtype != torch.int64 or slot_mapping.dtype != torch.int64:
        raise ValueError("positions / slot_mapping must be int64 [rows]")
    if k_cache.shape[1:] != (hkv, BLOCK_SIZE, d) or v_cache.shape != (k_cache.shape[0], hkv, d,
                                                                       BLOCK_SIZE):
        raise ValueError("caches must be [NB, Hkv, 16, D] and [NB, Hkv, D, 16]")
    if bias is not None:
        _dev(bias)
        if bias.shape != (weight.shape[0],):
            raise ValueError("bias must be [(Hq + 2 Hkv) D]")
    if out is None:
        out = torch.empty(rows, weight.shape[0], dtype=x.dtype, device=x.device)
    _check("pa_linear_rope_cache", _lib.load().pa_linear_rope_cache(
        _ptr(out), _ptr(x), _ptr(weight.data), _ptr(bias), rows, hq, hkv, d, k,
        LINEAR_RMS_IN if rms_eps is not None else 0,
        float(rms_eps) if rms_eps is not None else 0.0, _ptr(positions), _ptr(slot_mapping),
        _ptr(inv_freq), _ptr(k_cache), _ptr(v_cache), k_cache.shape[0], _dtype_code(x),
        _stream(x)))
    return out


def linear_workspace_size(rows, n, k, act=ACT_NONE):
    """pa_linear_workspace_size: bytes of pa_linear's K-split workspace for
    this shape (0: the shape does not split)."""
    return _lib.load().pa_linear_workspace_size(rows, n, k, act)


def linear_workspace(rows, n, k, act=ACT_NONE, device="cuda"):
    """A zeroed workspace for pa_linear's K split at this shape (uint8 device
    tensor), or None when the shape does not split.  One workspace serves
    any number of calls that run one after another (each leaves its
    counters zero), e.g. every layer of a model, if it is sized for the
    largest of them."""
    nbytes = linear_workspace_size(rows, n, k, act)
    return torch.zeros(nbytes, dtype=torch.uint8, device=device) if nbytes else None


def linear(x, weight, bias=None, act=ACT_NONE, out=None, rms_eps=None, add_to_out=False,
           workspace=None):
    """pa_linear: x [rows, K] bf16, weight [N, K] (or the fused gate|up
    [2 N, K] with act=ACT_SILU_MUL), row-major or a PackedWeight -> out
    [rows, N] bf16.  rms_eps: RMS-normalise the rows of x on the fly (the
    norm weight folded into a PackedWeight's col_scale); add_to_out: out is
    the residual stream, updated in place with the result; workspace: from
    linear_workspace (K split over several workgroups per tile) or None."""
    packed = isinstance(weight, PackedWeight)
    if packed and weight.rope_heads is not None:
        raise ValueError("a weight packed with rope_heads is for linear_rope_cache")
    wt = weight.data if packed else weight
    _dev(x, wt)
    rows, k = x.shape
    n = weight.shape[0] // (2 if act == ACT_SILU_MUL else 1)
    if weight.shape[1] != k:
        raise ValueError(f"weight {tuple(weight.shape)} does not match x {tuple(x.shape)}")
    if not (x.is_contiguous() and wt.is_contiguous()):
        raise ValueError("pa_linear takes contiguous x and weight")
    if bias is not None and (bias.shape != (n,) or not bias.is_contiguous()):
        raise ValueError(f"bias {tuple(bias.shape)} does not match {n} outputs")
    if out is None:
        if add_to_out:
            raise ValueError("add_to_out needs out")
        out = torch.empty(rows, n, dtype=x.dtype, device=x.device)
    if workspace is not None:
        _dev(workspace)
        if workspace.dtype != torch.uint8:
            raise ValueError("workspace: expected a uint8 tensor from linear_workspace")
    flags = (LINEAR_RMS_IN if rms_eps is not None else 0) | (LINEAR_ADD_OUT if add_to_out else 0)
    lib = _lib.load()
    _check("pa_linear", lib.pa_linear(_ptr(out), _ptr(x), _ptr(wt),
                                      _ptr(bias) if bias is not None else None, rows, n, k, act,
                                      1 if packed else 0, flags,
                                      float(rms_eps) if rms_eps is not None else 0.0,
                                      _ptr(workspace) if workspace is not None else None,
                                      workspace.numel() if workspace is not None else 0,
                                      _dtype_code(x), _stream(x)))
    return out
