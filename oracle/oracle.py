"""numpy face of the C oracle (liboracle.so, built from pa_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the CPU
baseline bench.py times.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this module.

Arrays are numpy; bf16 data is carried as uint16 bit patterns.  Cache
layout here is the reference's [NB, H, 16, D] for both K and V (the GPU
library stores V token-minor; tests convert with v_to_ref / v_from_ref).
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        lib = C.CDLL(LIB_PATH)
        p, i32, i64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float
        lib.oracle_write_kv.argtypes = [p, p, i32, i32, i32, i64, i64, p, p, i32]
        lib.oracle_write_kv_batch.argtypes = [p, p, i32, i32, i32, i64, i64, p, p, i32, i32]
        lib.oracle_read_kv.argtypes = [p, p, i32, i32, i32, p, i32, i32, p, p, i32]
        lib.oracle_slot_mapping.argtypes = [p, i32, p, i32, i32, p]
        lib.oracle_slot_mapping.restype = None
        lib.oracle_write_prefill_kv.argtypes = [p, p, i32, i32, i32, p, i32, p, i32, i32, p, p,
                                                i32]
        lib.oracle_reshape_and_cache.argtypes = [p, p, p, p, p, i32, i32, i32, i32, i32]
        lib.oracle_expand_kv.argtypes = [p, i32, i32, i32, i32, p]
        lib.oracle_expand_kv.restype = None
        lib.oracle_block_hash.argtypes = [p, i64]
        lib.oracle_block_hash.restype = C.c_uint64
        lib.oracle_argmax_logits.argtypes = [p, i64]
        lib.oracle_argmax_logits.restype = i64
        lib.oracle_attention.argtypes = [p, p, p, i32, i32, i32, i32, i32, i32, f32, i32, p]
        lib.oracle_paged_attention.argtypes = [p, p, p, p, i32, p, p, i32, i32, i32, i32, i32,
                                               f32, i32, i32, i32, p]
        lib.oracle_quant_write_kv.argtypes = [p, p, p, i32, i32, i32, i64, i64, p, p]
        lib.oracle_quant_read_kv.argtypes = [p, p, p, i32, i32, i32, p, i32, i32, p, p]
        lib.oracle_rope_inv_freq.argtypes = [i32, f32, i32, f32, i32, i32, p, p, p]
        lib.oracle_rope_inv_freq.restype = None
        lib.oracle_rope.argtypes = [p, i32, i32, i32, p, p, i32]
        lib.oracle_rope.restype = None
        lib.oracle_fp8_encode.argtypes = [f32]
        lib.oracle_fp8_encode.restype = C.c_uint8
        lib.oracle_fp8_decode.argtypes = [C.c_uint8]
        lib.oracle_fp8_decode.restype = f32
        lib.oracle_fp8_encode_n.argtypes = [p, p, i64]
        lib.oracle_fp8_encode_n.restype = None
        lib.oracle_fp8_decode_n.argtypes = [p, p, i64]
        lib.oracle_fp8_decode_n.restype = None
        lib.oracle_f32_to_bf16.argtypes = [f32]
        lib.oracle_f32_to_bf16.restype = C.c_uint16
        _lib = lib
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _code(a):
    if a.dtype == np.float32:
        return 0
    if a.dtype == np.uint16:
        return 1
    raise ValueError(a.dtype)


# ---- dtype helpers ---------------------------------------------------------
def f32_to_bf16(x):
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h):
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def as_f32(a):
    return bf16_to_f32(a) if a.dtype == np.uint16 else np.asarray(a, dtype=np.float32)


def v_to_ref(v_cache_tm):
    """Token-minor V cache [NB, H, D, 16] -> reference layout [NB, H, 16, D]."""
    return np.ascontiguousarray(np.swapaxes(v_cache_tm, 2, 3))


def v_from_ref(v_cache_ref):
    return np.ascontiguousarray(np.swapaxes(v_cache_ref, 2, 3))


# ---- KV store --------------------------------------------------------------
def write_kv(k_cache, v_cache, block_id, token_offset, k, v):
    nb, h, _, d = k_cache.shape
    k = np.ascontiguousarray(k, dtype=k_cache.dtype)
    v = np.ascontiguousarray(v, dtype=k_cache.dtype)
    return load().oracle_write_kv(_p(k_cache), _p(v_cache), nb, h, d, block_id, token_offset,
                                  _p(k), _p(v), _code(k_cache))


def write_kv_batch(k_cache, v_cache, block_id, token_offset, k, v):
    nb, h, _, d = k_cache.shape
    k = np.ascontiguousarray(k, dtype=k_cache.dtype)
    v = np.ascontiguousarray(v, dtype=k_cache.dtype)
    t = k.size // (h * d)
    return load().oracle_write_kv_batch(_p(k_cache), _p(v_cache), nb, h, d, block_id,
                                        token_offset, _p(k), _p(v), t, _code(k_cache))


def read_kv(k_cache, v_cache, block_ids, seq_len):
    """-> (rc_or_count, k [n, H, D], v [n, H, D])."""
    nb, h, _, d = k_cache.shape
    ids = np.ascontiguousarray(block_ids, dtype=np.int64)
    cap = max(0, min(seq_len, len(ids) * 16))
    ok = np.zeros((cap, h, d), dtype=k_cache.dtype)
    ov = np.zeros_like(ok)
    n = load().oracle_read_kv(_p(k_cache), _p(v_cache), nb, h, d, _p(ids), len(ids), seq_len,
                              _p(ok), _p(ov), _code(k_cache))
    if n < 0:
        return n, None, None
    return n, ok[:n], ov[:n]


def slot_mapping(block_ids, positions, num_tokens):
    ids = np.ascontiguousarray(block_ids, dtype=np.int64)
    pos = np.ascontiguousarray(positions, dtype=np.int64) if positions is not None else None
    out = np.zeros(num_tokens, dtype=np.int64)
    load().oracle_slot_mapping(_p(ids), len(ids), _p(pos), -1 if pos is None else len(pos),
                               num_tokens, _p(out))
    return out


def write_prefill_kv(k_cache, v_cache, block_ids, positions, seq_len, k, v):
    nb, h, _, d = k_cache.shape
    ids = np.ascontiguousarray(block_ids, dtype=np.int64)
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    k = np.ascontiguousarray(k, dtype=k_cache.dtype)
    v = np.ascontiguousarray(v, dtype=k_cache.dtype)
    return load().oracle_write_prefill_kv(_p(k_cache), _p(v_cache), nb, h, d, _p(ids), len(ids),
                                          _p(pos), len(pos), seq_len, _p(k), _p(v),
                                          _code(k_cache))


def reshape_and_cache(k, v, k_cache, v_cache, slots):
    nb, h, _, d = k_cache.shape
    k = np.ascontiguousarray(k, dtype=k_cache.dtype)
    v = np.ascontiguousarray(v, dtype=k_cache.dtype)
    s = np.ascontiguousarray(slots, dtype=np.int64)
    return load().oracle_reshape_and_cache(_p(k), _p(v), _p(k_cache), _p(v_cache), _p(s),
                                           len(s), h, d, nb, _code(k_cache))


def expand_kv(x, num_q_heads):
    """[S, Hkv, D] f32 -> [S, Hq, D]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    s, hkv, d = x.shape
    out = np.zeros((s, num_q_heads, d), dtype=np.float32)
    load().oracle_expand_kv(_p(x), s, hkv, num_q_heads, d, _p(out))
    return out


def block_hash(data):
    data = np.ascontiguousarray(data, dtype=np.float32).ravel()
    return int(load().oracle_block_hash(_p(data), data.size))


def argmax_logits(logits):
    """Greedy token of each row of logits [rows, vocab] (last axis), int64."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    rows = x.reshape(-1, x.shape[-1]) if x.ndim > 1 else x.reshape(1, -1)
    lib = load()
    out = np.array([lib.oracle_argmax_logits(_p(r), r.size) for r in rows], np.int64)
    return out.reshape(x.shape[:-1]) if x.ndim > 1 else out[0]


# ---- attention -------------------------------------------------------------
def attention(q, k, v, past, scale=None, f64=False):
    """Dense masked GQA attention. q [Tq, Hq, D], k/v [Tk, Hkv, D] f32."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    tq, hq, d = q.shape
    tk, hkv, _ = k.shape
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(d))
    out = np.zeros_like(q)
    rc = load().oracle_attention(_p(q), _p(k), _p(v), tq, tk, past, hq, hkv, d, float(scale),
                                 int(f64), _p(out))
    if rc:
        raise ValueError(f"oracle_attention rc={rc}")
    return out


def paged_attention(q, k_cache, v_cache_ref, block_tables, q_start, past, scale=None,
                    f64=False, threads=0):
    """Batched paged attention on reference-layout caches.

    q [sum Tq, Hq, D] (f32 or bf16 bits), caches [NB, Hkv, 16, D],
    block_tables [B, MBS] int32, q_start [B+1], past [B]."""
    q = np.ascontiguousarray(q)
    tq, hq, d = q.shape
    nb, hkv, _, _ = k_cache.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    qs = np.ascontiguousarray(q_start, dtype=np.int32)
    pa = np.ascontiguousarray(past, dtype=np.int32)
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(d))
    out = np.zeros_like(q)
    rc = load().oracle_paged_attention(_p(q), _p(k_cache), _p(v_cache_ref), _p(bt), bt.shape[1],
                                       _p(qs), _p(pa), bt.shape[0], hq, hkv, d, nb,
                                       float(scale), _code(q), int(f64), int(threads), _p(out))
    if rc:
        raise ValueError(f"oracle_paged_attention rc={rc}")
    return out


def quant_write_kv(k_cache, v_cache, scales, block_id, token_offset, k, v):
    nb, h, _, d = k_cache.shape
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    return load().oracle_quant_write_kv(_p(k_cache), _p(v_cache), _p(scales), nb, h, d,
                                        block_id, token_offset, _p(k), _p(v))


def quant_read_kv(k_cache, v_cache, scales, block_ids, seq_len):
    nb, h, _, d = k_cache.shape
    ids = np.ascontiguousarray(block_ids, dtype=np.int64)
    cap = max(0, min(seq_len, len(ids) * 16))
    ok = np.zeros((cap, h, d), dtype=np.float32)
    ov = np.zeros_like(ok)
    n = load().oracle_quant_read_kv(_p(k_cache), _p(v_cache), _p(scales), nb, h, d, _p(ids),
                                    len(ids), seq_len, _p(ok), _p(ov))
    return n, ok[: max(n, 0)], ov[: max(n, 0)]


# ---- rotary embedding ------------------------------------------------------
ROPE_TYPES = {"default": 0, "linear": 1, "yarn": 2, "dynamic": 3, "su": 4}


def rope_inv_freq(head_dim, theta, rope_type="default", factor=1.0, original_max_position=0,
                  cur_seq_len=0, short_factor=None, long_factor=None):
    out = np.zeros(head_dim // 2, dtype=np.float32)
    sf = None if short_factor is None else np.ascontiguousarray(short_factor, dtype=np.float32)
    lf = None if long_factor is None else np.ascontiguousarray(long_factor, dtype=np.float32)
    load().oracle_rope_inv_freq(head_dim, float(theta), ROPE_TYPES[rope_type], float(factor),
                                int(original_max_position), int(cur_seq_len), _p(sf), _p(lf),
                                _p(out))
    return out


def rope(x, positions, inv_freq):
    """Rotate-half RoPE of x [T, H, D] (f32 or bf16 bits); returns a copy."""
    x = np.array(x, copy=True)
    t, h, d = x.shape
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    inv = np.ascontiguousarray(inv_freq, dtype=np.float32)
    load().oracle_rope(_p(x), t, h, d, _p(pos), _p(inv), _code(x))
    return x


def fp8_encode(x):
    """Reference FP8-E4M3 codes (uint8) of f32 values (any shape)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    load().oracle_fp8_encode_n(_p(x), _p(out), x.size)
    return out


def fp8_decode(b):
    """f32 values of reference FP8-E4M3 codes (any shape)."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.shape, np.float32)
    load().oracle_fp8_decode_n(_p(b), _p(out), b.size)
    return out
