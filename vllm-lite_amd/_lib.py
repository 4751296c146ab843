"""ctypes bindings of libpa.so (declarations mirror include/pa.h and
include/pa_kv_cache.h)."""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpa.so")

# Every symbol the headers declare, with (restype, argtypes).
_i32, _i64, _f32, _sz, _p = C.c_int32, C.c_int64, C.c_float, C.c_size_t, C.c_void_p
SIGNATURES = {
    "pa_last_error": (C.c_char_p, []),
    "pa_version": (C.c_char_p, []),
    "pa_reshape_and_cache": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i64,
                                    _i32, _p]),
    "pa_reshape_and_cache_fp8": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i64,
                                         _i32, _p]),
    "pa_slot_mapping": (_i32, [_p, _i32, _p, _p, _i32, _i32, _p, _p]),
    "pa_read_kv": (_i32, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _i32, _p]),
    "pa_block_hash": (_i32, [_p, _p, _i32, _i32, _i32, _i32, _p, _p]),
    "pa_decode_workspace_size": (_sz, [_i32, _i32, _i32, _i32]),
    "pa_reshape_and_cache_fp8_flagged": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32,
                                                 _i64, _i64, _i32, _p, _p]),
    "pa_decode_fp8_flagged": (_i32, [_p, _p, _p, _p, _p, _i32, _p, _i32, _i32, _i32, _i32, _i32,
                                      _i32, _f32, _p, _sz, _p, _p]),
    "pa_decode": (_i32, [_p, _p, _p, _p, _p, _i32, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                         _p, _sz, _i32, _p]),
    "pa_decode_noalloc": (_i32, [_p, _p, _p, _p, _p, _i32, _p, _i32, _i32, _i32, _i32, _i32,
                                 _i32, _f32, _i32, _p]),
    "pa_decode_noalloc_scratch_bytes": (_sz, []),
    "pa_prefill": (_i32, [_p, _p, _p, _p, _p, _i32, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32,
                          _i32, _f32, _i32, _p]),
    "pa_rms_norm": (_i32, [_p, _p, _p, _p, _i32, _i32, _f32, _i32, _p]),
    "pa_layer_norm": (_i32, [_p, _p, _p, _p, _p, _i32, _i32, _f32, _i32, _p]),
    "pa_silu_mul": (_i32, [_p, _p, _i32, _i32, _i32, _p]),
    "pa_linear": (_i32, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p, _sz,
                         _i32, _p]),
    "pa_linear_workspace_size": (_sz, [_i32, _i32, _i32, _i32]),
    "pa_linear_pack": (_i32, [_p, _p, _p, _i32, _i32, _i32, _p]),
    "pa_argmax": (_i32, [_p, _p, _i32, _i32, _i64, _i32, _p]),
    "pa_linear_rope_cache": (_i32, [_p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                                    _p, _p, _p, _p, _p, _i32, _i32, _p]),
    "pa_linear_pack_qkv": (_i32, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _p]),
    "pa_decode_quantized": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _p, _i32, _i32, _i32, _i32,
                                   _i32, _i32, _f32, _p, _sz, _p]),
    "pa_prefill_quantized": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _p, _p, _i32, _i32, _i32, _i32,
                                    _i32, _i32, _i32, _f32, _p]),
    "pa_kv_cache_create_quantized": (_i32, [_i32, _i32, _i32, _i32, C.POINTER(_p)]),
    "pa_kv_cache_is_quantized": (_i32, [_p]),
    "pa_kv_cache_scales_ptr": (_p, [_p, _i32]),
    "pa_rope_reshape_and_cache": (_i32, [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _p, _p, _i32,
                                         _i32, _i32, _i32, _i32, _i32, _p]),
    "pa_rope_inv_freq": (_i32, [_i32, _f32, _i32, _f32, _i32, _i32, _p, _p, _p]),
    "pa_kv_cache_create": (_i32, [_i32, _i32, _i32, _i32, _i32, C.POINTER(_p)]),
    "pa_kv_cache_destroy": (None, [_p]),
    "pa_kv_cache_num_layers": (_i32, [_p]),
    "pa_kv_cache_num_blocks": (_i32, [_p]),
    "pa_kv_cache_block_size": (_i32, [_p]),
    "pa_kv_cache_num_heads": (_i32, [_p]),
    "pa_kv_cache_head_dim": (_i32, [_p]),
    "pa_kv_cache_dtype": (_i32, [_p]),
    "pa_kv_cache_key_ptr": (_p, [_p, _i32]),
    "pa_kv_cache_value_ptr": (_p, [_p, _i32]),
    "pa_kv_cache_write_kv": (_i32, [_p, _i32, _i64, _i64, _p, _p, _p]),
    "pa_kv_cache_write_kv_batch": (_i32, [_p, _i32, _i64, _i64, _p, _p, _i32, _p]),
    "pa_kv_cache_write_prefill_kv": (_i32, [_p, _i32, _p, _i32, _p, _i32, _i32, _p, _p, _p]),
    "pa_kv_cache_read_kv": (_i32, [_p, _i32, _p, _i32, _i32, _p, _p, C.POINTER(_i32), _p]),
    "pa_kv_cache_block_hash_count": (_i32, [_p, _i32, C.POINTER(_i64)]),
    "pa_kv_cache_block_hashes": (_i32, [_p, _i32, _p, _p, _i64, C.POINTER(_i64)]),
    "pa_kv_cache_lookup_block_hash": (_i32, [_p, _i32, C.c_uint64, C.POINTER(_i64)]),
    "pa_batch_create": (_i32, [C.POINTER(_p)]),
    "pa_batch_destroy": (None, [_p]),
    "pa_batch_prepare": (_i32, [_p, _i32, _p, _p, _p, _p, _i32, _p]),
    "pa_batch_num_tokens": (_i32, [_p]),
    "pa_batch_set_capacity": (_i32, [_p, _i32]),
    "pa_batch_is_decode": (_i32, [_p]),
    "pa_batch_advance": (_i32, [_p, _p]),
    "pa_batch_qkv_rope_cache": (_i32, [_p, _p, _i32, _i32, _p, _p, _p, _p, _i32, _i32, _f32,
                                       _p, _p]),
    "pa_batch_attention": (_i32, [_p, _p, _i32, _i32, _p, _i64, _p, _i64, _p, _i64, _p, _f32,
                                  _p, _p]),
}

_lib = None


def load():
    """Loads libpa.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
