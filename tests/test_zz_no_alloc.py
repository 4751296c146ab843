"""pa_decode_noalloc (the allocation-free decode entry point) against
pa_decode, through the C ABI: two calls in a row on the shared scratch, the
second smaller, each bit-identical to pa_decode with its own workspace."""
import math

import numpy as np
import pytest
import torch

from helpers import make_decode_case
from test_gpu_cache_ops import DEV, to_dev

pytestmark = pytest.mark.gpu


def noalloc(pa, q, kc, vc, bt, ctx, max_ctx):
    lib = pa._lib.load()
    out = torch.empty_like(q)
    b, hq, d = q.shape
    rc = lib.pa_decode_noalloc(out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                               bt.data_ptr(), bt.shape[1], ctx.data_ptr(), max_ctx, b, hq,
                               kc.shape[1], d, kc.shape[0], 1 / math.sqrt(d),
                               pa.ops._dtype_code(q), torch.cuda.current_stream().cuda_stream)
    return rc, out


def test_decode_noalloc_matches_decode_two_calls(pa, oracle):
    # both sizes split into more partitions than one workgroup merges, so
    # the scratch carries partial results into decode_reduce_kernel; the
    # second call is smaller and follows the first on the same scratch
    for seed, ctx in ((21, [20000, 9000, 17, 15000]), (22, [9000, 300])):
        rng = np.random.default_rng(seed)
        case = make_decode_case(rng, len(ctx), 32, 8, 128, ctx, dtype="bf16")
        q, kc = to_dev(case["q"]), to_dev(case["k_cache"])
        vc = to_dev(oracle.v_from_ref(case["v_cache_ref"]))
        bt, cl = to_dev(case["block_tables"]), to_dev(case["ctx"])
        assert pa.decode_workspace_size(len(ctx), 32, 128, max(ctx)) > 0
        rc, got = noalloc(pa, q, kc, vc, bt, cl, max(ctx))
        assert rc == 0, pa._lib.load().pa_last_error()
        ref = pa.decode(q, kc, vc, bt, cl, max(ctx))
        torch.cuda.synchronize()
        assert torch.equal(got, ref), seed


def test_decode_noalloc_rejects_oversized_split(pa):
    # B 64 at context 32768: 64 x 32 x 64 partitions x 130 floats > 64 MiB
    lib = pa._lib.load()
    assert lib.pa_decode_noalloc_scratch_bytes() == 64 << 20
    q = torch.zeros(64, 32, 128, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(4, 8, 16, 128, dtype=torch.bfloat16, device=DEV)
    bt = torch.zeros(64, 2048, dtype=torch.int32, device=DEV)
    cl = torch.full((64,), 32768, dtype=torch.int32, device=DEV)
    rc, _ = noalloc(pa, q, kc, kc, bt, cl, 32768)
    assert rc == -4 and b"scratch" in lib.pa_last_error()
