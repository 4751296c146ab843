"""GPU parity of pa_linear (the skinny-M projections of a decode step) against
an fp32 torch matmul of the same bf16 operands: plain, with bias, and with the
fused SwiGLU epilogue; ragged row counts around the 32-row tile, K split over
one and many wavefronts; argument errors."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def operands(m, n, k, seed, wscale=0.02):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=DEV) * wscale).to(torch.bfloat16)
    b = (torch.randn(n, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    return x, w, b


def close(out, ref):
    # bf16 output of an f32-accumulated product: half an ulp of bf16 plus the
    # f32 summation-order difference
    torch.testing.assert_close(out.float(), ref, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("m,n,k", [(1, 32, 32), (5, 64, 896), (32, 1152, 896), (33, 896, 4864),
                                   (64, 896, 896), (17, 256, 4864), (31, 4096, 96),
                                   (9, 48, 64), (40, 1008, 128)])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("packed", [False, True])
def test_linear_matches_fp32(pa, m, n, k, with_bias, packed):
    x, w, b = operands(m, n, k, m * 7 + n + k)
    out = pa.linear(x, pa.ops.PackedWeight(w) if packed else w, bias=b if with_bias else None)
    ref = x.float() @ w.float().T
    if with_bias:
        ref = ref + b.float()
    assert out.shape == (m, n) and out.dtype == torch.bfloat16
    close(out, ref)


@pytest.mark.parametrize("m,inter,k", [(32, 4864, 896), (3, 16, 64), (40, 48, 4864)])
def test_linear_swiglu_matches_unfused(pa, m, inter, k):
    x, w, _ = operands(m, 2 * inter, k, m + inter + k, wscale=0.05)
    out = pa.linear(x, w, act=pa.ops.ACT_SILU_MUL)
    gu = (x.float() @ w.float().T).to(torch.bfloat16).float()  # the unfused projection's output
    ref = F.silu(gu[:, :inter]) * gu[:, inter:]
    assert out.shape == (m, inter)
    close(out, ref)
    # and the same as the unfused path through pa_silu_mul, and from packed weights
    unfused = pa.silu_mul(pa.linear(x, w))
    close(out, unfused.float())
    assert torch.equal(pa.linear(x, pa.ops.PackedWeight(w), act=pa.ops.ACT_SILU_MUL), out)


@pytest.mark.parametrize("n,k", [(16, 32), (48, 96), (896, 4864)])
def test_pack_layout(pa, n, k):
    # fragment (tile, step) is 1 KB; lane 16 j + c holds row 16 tile + c,
    # columns 32 step + 8 j .. +7 -- an independent torch restatement
    _, w, _ = operands(1, n, k, n + k)
    packed = pa.ops.PackedWeight(w).data
    ref = w.view(n // 16, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(n, k)
    assert torch.equal(packed, ref)


def test_lm_head_shape(pa):
    # the tied LM head of the Qwen2.5-0.5B shape: 151936 outputs, K = 896
    x, w, _ = operands(32, 151936, 896, 5)
    out = pa.linear(x, w)
    close(out, x.float() @ w.float().T)


@pytest.mark.parametrize("m,n,k", [(32, 151936, 896), (1, 65648, 896), (17, 65536, 128),
                                   (32, 70000 // 16 * 16, 160), (9, 65600, 192),
                                   (7, 66048, 992)])
@pytest.mark.parametrize("rms", [False, True])
def test_wide_projection_from_lds(pa, m, n, k, rms):
    # packed weights of >= 4096 tiles with one batch tile: linear_wide_kernel
    # (X in LDS, tiles dealt over a persistent grid; odd tile ranges, units of
    # 7 / 4 / 1 K steps, the largest K it takes)
    x, w, _ = operands(m, n, k, m + n + k)
    gamma = None
    if rms:
        x = (x.float() * 3 + 0.5).to(torch.bfloat16)
        g = torch.Generator(device=DEV).manual_seed(k + 1)
        gamma = (1 + 0.2 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    out = pa.linear(x, pa.ops.PackedWeight(w, col_scale=gamma), rms_eps=1e-6 if rms else None)
    xr = rms_ref(x, gamma, 1e-6) if rms else x.float()
    close(out, xr @ w.float().T)


def test_linear_rejects_unsupported(pa):
    x, w, b = operands(4, 64, 96, 1)
    with pytest.raises(pa.PaError):
        pa.linear(x[:, :80].contiguous(), w[:, :80].contiguous())  # K not a multiple of 32
    # N not a multiple of 16: the tiled GEMM takes it (K a multiple of 64)
    x2, w2, _ = operands(4, 40, 128, 2)
    close(pa.linear(x2, w2), x2.float() @ w2.float().T)
    with pytest.raises(pa.PaError):
        pa.linear(x.float(), w.float())  # f32
    with pytest.raises(pa.PaError):
        pa.linear(x, w, bias=b[:32].contiguous(), act=pa.ops.ACT_SILU_MUL)
    empty = pa.linear(x[:0], w)
    assert empty.shape == (0, 64)


def rms_ref(x, gamma, eps):
    xf = x.float()
    return xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * gamma.float()


@pytest.mark.parametrize("m,n,k", [(32, 896, 896), (5, 256, 896), (40, 64, 4864)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_rms_in_matches_norm_then_matmul(pa, m, n, k, with_bias):
    # PA_LINEAR_RMS_IN with the norm weight folded into the packed columns ==
    # RMSNorm then the projection (fp32 reference)
    x, w, b = operands(m, n, k, m + 3 * n + k)
    x = (x.float() * 3 + 0.5).to(torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(k)
    gamma = (1 + 0.2 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16)
    out = pa.linear(x, pa.ops.PackedWeight(w, col_scale=gamma), bias=b if with_bias else None,
                    rms_eps=1e-6)
    ref = rms_ref(x, gamma, 1e-6) @ w.float().T
    if with_bias:
        ref = ref + b.float()
    close(out, ref)


def test_linear_rms_in_swiglu(pa):
    m, inter, k = 32, 4864, 896
    x, w, _ = operands(m, 2 * inter, k, 11, wscale=0.05)
    gamma = torch.full((k,), 0.75, dtype=torch.bfloat16, device=DEV)
    out = pa.linear(x, pa.ops.PackedWeight(w, col_scale=gamma), act=pa.ops.ACT_SILU_MUL,
                    rms_eps=1e-6)
    gu = (rms_ref(x, gamma, 1e-6) @ w.float().T).to(torch.bfloat16).float()
    # g and u are rounded to bf16 on both sides (as the unfused path does), from
    # different accumulation orders and a norm-scaled weight: either may land one
    # bf16 ulp (2^-8 relative) apart, which silu(g) * u carries twice
    torch.testing.assert_close(out.float(), F.silu(gu[:, :inter]) * gu[:, inter:], atol=2e-2,
                               rtol=3e-2)


@pytest.mark.parametrize("packed", [False, True])
def test_linear_adds_into_residual(pa, packed):
    m, n, k = 33, 896, 896
    x, w, _ = operands(m, n, k, 13)
    res = (torch.randn(m, n, device=DEV) * 2).to(torch.bfloat16)
    expect = (res.float() + (x.float() @ w.float().T).to(torch.bfloat16).float())
    out = res.clone()
    got = pa.linear(x, pa.ops.PackedWeight(w) if packed else w, out=out, add_to_out=True)
    assert got.data_ptr() == out.data_ptr()
    close(out, expect)


@pytest.mark.parametrize("m,n,k,act,rms,add", [
    (32, 896, 4864, 0, False, True),     # the decode step's down projection
    (1, 896, 4864, 0, False, False),
    (64, 896, 4864, 0, False, True),     # two row tiles
    (20, 256, 2048, 0, True, False),     # RMS-in: partial sums of squares too
    (8, 256, 4096, 1, True, False),      # SwiGLU epilogue after the split
    (5, 48, 3072, 0, False, False),      # bias-free, 3 tiles
])
def test_linear_split_k(pa, m, n, k, act, rms, add):
    # K split over workgroups (pa_linear's workspace): against fp32, twice in
    # a row on one workspace, then again on fewer rows (a counter left
    # non-zero would leave a tile's output unwritten or summed early); the
    # split is independent of arrival order, so repeated calls agree bit for
    # bit
    ws = pa.ops.linear_workspace(64, n, k, act, DEV)
    assert ws is not None and ws.numel() >= pa.ops.linear_workspace_size(m, n, k, act)
    g = torch.Generator(device=DEV).manual_seed(m + n + k)
    w = (torch.randn((2 if act else 1) * n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wp = pa.ops.PackedWeight(w)
    for rows in (m, max(1, m // 3)):
        x = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
        xf = x.float()
        if rms:
            xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
        y = xf @ w.float().T
        if act:
            gg = y[:, :n].to(torch.bfloat16).float()
            uu = y[:, n:].to(torch.bfloat16).float()
            y = F.silu(gg) * uu
        res = torch.randn(rows, n, generator=g, device=DEV).to(torch.bfloat16) if add else None
        outs = []
        for _ in range(2):
            o = res.clone() if add else None
            outs.append(pa.linear(x, wp, act=act, out=o, add_to_out=add,
                                  rms_eps=1e-6 if rms else None, workspace=ws))
        assert torch.equal(outs[0], outs[1])
        ref = y + res.float() if add else y
        # rms: the 1 / rms factor and the bf16 rounding of g, u add a few ulp
        torch.testing.assert_close(outs[0].float(), ref, atol=3e-2 if (rms or add) else 2e-2,
                                   rtol=3e-2 if rms else 1e-2)
        nsplit = pa.ops.linear(x, wp, act=act, rms_eps=1e-6 if rms else None)
        if not add:
            torch.testing.assert_close(outs[0].float(), nsplit.float(), atol=2e-2, rtol=1e-2)


# k = 4096: more than 64 K steps per workgroup, the stage-4 instance
@pytest.mark.parametrize("rows,hq,hkv,d,k", [(32, 14, 2, 64, 896), (5, 32, 8, 128, 256),
                                             (40, 4, 4, 64, 64), (1, 8, 2, 32, 128),
                                             (3, 8, 2, 128, 4096)])
@pytest.mark.parametrize("rms,with_bias", [(True, True), (False, False)])
def test_linear_rope_cache_matches_unfused(pa, rows, hq, hkv, d, k, rms, with_bias):
    # pa_linear_rope_cache == pa_linear on the row-major-packed weight, then
    # pa_rope_reshape_and_cache on the q / k / v views of its output: the
    # same bf16 projection values, the same rotation, the same cache writes
    # (bit for bit), one slot outside the pool skipped, untouched slots zero
    n = (hq + 2 * hkv) * d
    g = torch.Generator(device=DEV).manual_seed(rows * 3 + hq + d + k)
    x = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    bias = (torch.randn(n, generator=g, device=DEV) * 0.1).to(torch.bfloat16) if with_bias \
        else None
    gamma = (1 + 0.1 * torch.randn(k, generator=g, device=DEV)).to(torch.bfloat16) if rms \
        else None
    nb = 8
    positions = torch.randint(0, 4000, (rows,), generator=g, device=DEV)
    slots = torch.randperm(nb * 16, generator=g, device=DEV)[:rows].clone()
    slots[rows // 2] = -1 if rows > 1 else slots[0]
    inv_freq = torch.from_numpy(pa.rope_inv_freq(d, 1e6)).to(DEV)
    eps = 1e-6 if rms else None

    kc0 = torch.zeros(nb, hkv, 16, d, dtype=torch.bfloat16, device=DEV)
    vc0 = torch.zeros(nb, hkv, d, 16, dtype=torch.bfloat16, device=DEV)
    ref = pa.linear(x, pa.ops.PackedWeight(w, col_scale=gamma), bias, rms_eps=eps)
    q = ref[:, :hq * d].view(rows, hq, d)
    kk = ref[:, hq * d:(hq + hkv) * d].view(rows, hkv, d)
    vv = ref[:, (hq + hkv) * d:].view(rows, hkv, d)
    pa.rope_reshape_and_cache(q, kk, vv, kc0, vc0, slots, positions, inv_freq)

    kc1 = torch.zeros_like(kc0)
    vc1 = torch.zeros_like(vc0)
    wq = pa.ops.PackedWeight(w, col_scale=gamma, rope_heads=(hq, hkv, d))
    got = pa.ops.linear_rope_cache(x, wq, bias, positions, slots, inv_freq, kc1, vc1,
                                   rms_eps=eps)
    # q rotated in place by the unfused path; k columns of ref are unrotated
    # there (rotated on their way into the cache), v as projected
    assert torch.equal(got[:, :hq * d], ref[:, :hq * d])
    assert torch.equal(got[:, (hq + hkv) * d:], ref[:, (hq + hkv) * d:])
    assert torch.equal(kc1, kc0) and torch.equal(vc1, vc0)
    # the rotated k columns of the output are what went into the cache
    kg = got[:, hq * d:(hq + hkv) * d].view(rows, hkv, d)
    for r in range(rows):
        s = int(slots[r])
        if s >= 0:
            assert torch.equal(kg[r], kc1[s // 16, :, s % 16, :])
            assert torch.equal(vv[r], vc1[s // 16, :, :, s % 16])
    with pytest.raises(ValueError):
        pa.linear(x, wq)   # a rope-packed weight is not a plain packed weight


def test_linear_split_k_graph_replays(pa):
    # the K split in a captured graph: three calls on one workspace per
    # replay; each replay (new inputs copied in between, eager work and a
    # synchronisation in between) equals the eager result bit for bit
    m, n, k = 32, 896, 4864
    g = torch.Generator(device=DEV).manual_seed(9)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wp = pa.ops.PackedWeight(w)
    ws = pa.ops.linear_workspace(m, n, k, device=DEV)
    x = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    res = torch.zeros(m, n, dtype=torch.bfloat16, device=DEV)

    def step():
        for _ in range(3):
            pa.linear(x, wp, out=res, add_to_out=True, workspace=ws)

    step()  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(3):
        x.copy_(torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16))
        start = torch.randn(m, n, generator=g, device=DEV).to(torch.bfloat16)
        res.copy_(start)
        graph.replay()
        torch.cuda.synchronize()
        got = res.clone()
        res.copy_(start)
        step()
        torch.cuda.synchronize()
        assert torch.equal(got, res), i


def test_linear_split_k_workspace_any_call_order(pa):
    # One workspace shared by calls whose split plans differ (the engine's
    # down projection at <= 32 rows: 56 tiles x 4 splits; at 33-64 rows:
    # 112 tiles x 2 splits), in both orders and interleaved.  The counter
    # region sits at a fixed place, so leftover partial sums of one plan
    # never read as counters of the next; each call is checked against fp32
    # and against the same call on a fresh workspace (bit for bit).
    n, k = 896, 4864
    g = torch.Generator(device=DEV).manual_seed(17)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wp = pa.ops.PackedWeight(w)
    ws = pa.ops.linear_workspace(64, n, k, device=DEV)
    assert ws.numel() >= max(pa.ops.linear_workspace_size(r, n, k) for r in range(1, 65))
    for rows in (7, 32, 33, 64, 20, 48, 1, 40, 40, 3):
        x = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
        got = pa.linear(x, wp, workspace=ws)
        fresh = pa.linear(x, wp, workspace=pa.ops.linear_workspace(rows, n, k, device=DEV))
        assert torch.equal(got, fresh), rows
        torch.testing.assert_close(got.float(), x.float() @ w.float().T, atol=2e-2, rtol=1e-2)


# Prefill-sized batches (rows > 64) take the tiled GEMM (gemm_tiled_kernel,
# 128 x 128 workgroup tiles, or 256 x 256 for outputs of 256 such tiles or
# more): the config-5 projections at prompt-chunk row counts, ragged row and
# column tails around both tiles, bias, SwiGLU and the residual add.
@pytest.mark.parametrize("m,n,k", [(65, 896, 896), (130, 256, 896), (1000, 896, 896),
                                   (777, 896, 4864), (128, 128, 64), (4100, 1152, 896),
                                   (2100, 8000, 128), (9000, 896, 896)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_tiled_gemm_matches_fp32(pa, m, n, k, with_bias):
    x, w, b = operands(m, n, k, m * 3 + n + k)
    out = pa.linear(x, w, bias=b if with_bias else None)
    ref = x.float() @ w.float().T
    if with_bias:
        ref = ref + b.float()
    assert out.shape == (m, n)
    close(out, ref)


@pytest.mark.parametrize("m,inter,k", [(300, 4864, 896), (65, 64, 128)])
def test_tiled_gemm_swiglu(pa, m, inter, k):
    x, w, _ = operands(m, 2 * inter, k, m + inter, wscale=0.05)
    out = pa.linear(x, w, act=pa.ops.ACT_SILU_MUL)
    gu = (x.float() @ w.float().T).to(torch.bfloat16).float()
    close(out, F.silu(gu[:, :inter]) * gu[:, inter:])


def test_tiled_gemm_add_out(pa):
    x, w, _ = operands(257, 896, 4864, 11)
    res = torch.randn(257, 896, device=DEV).to(torch.bfloat16)
    out = res.clone()
    pa.linear(x, w, out=out, add_to_out=True)
    y = (x.float() @ w.float().T).to(torch.bfloat16).float()
    close(out, res.float() + y)


def test_tiled_gemm_large_prefill_chunk(pa):
    # the config-5 gate|up projection over a whole prompt batch (9000 rows)
    x, w, _ = operands(9000, 2 * 4864, 896, 3, wscale=0.05)
    out = pa.linear(x, w, act=pa.ops.ACT_SILU_MUL)
    gu = (x.float() @ w.float().T).to(torch.bfloat16).float()
    close(out, F.silu(gu[:, :4864]) * gu[:, 4864:])
