"""Slot sizing of the balanced split-K decode, checked on the CPU.

decode_balanced_kernel cuts all (segment, unit) work of a launch evenly over
N wavefronts and writes one partial result per (row, wavefront that meets
the row's segment) into that row's slots; decode_reduce_kernel merges them.
pa_decode sizes the slots per row from max_context_len.  This file restates
the kernels' integer layout arithmetic (groups of sequences that begin with
the same block, their common prefix, wave_of / seg_slots in decode.hip) in
Python and checks, over seeded random ragged shared-prefix layouts, that no
row ever needs more slots than the plan gives it, and that
pa_decode_workspace_size covers the plan's workspace.  A layout that needs
ceil(n / 8) + 3 slots is included (it overflowed the former + 2 sizing).
"""
import numpy as np
import pytest

BLOCK = 16
MIN_UNITS = 8      # kBalanceMinUnits: units (32 tokens) per wavefront at least
WAVES = 1024       # kBalanceWaves
GROUP_MAX = 1024   # kGroupMaxSeqs


def plan_slots(max_ctx):
    max_units = (max_ctx + 2 * BLOCK - 1) // (2 * BLOCK)
    return (max_units + MIN_UNITS - 1) // MIN_UNITS + 3


def layout_slots(ctx, tables, hq, hkv):
    """Slots each (sequence, query head) row needs, by the kernels' arithmetic."""
    b, mbs = tables.shape
    cap = int(max(ctx.max(), 0))
    g_ = hq // hkv
    clamp = [min(min(int(c), mbs * BLOCK), cap) for c in ctx]
    units = [(c + 2 * BLOCK - 1) // (2 * BLOCK) if c > 0 else 0 for c in clamp]
    if g_ <= 8 and 2 <= b <= GROUP_MAX:
        sp = 16 // g_
        none = 0xFFFFFFFF
        keys = sorted((((int(tables[s, 0]) & 0xFFFFFFFF) if clamp[s] // 32 > 0 else none), s)
                      for s in range(b))
        groups, cur, prev = [], [], None
        for hi, s in keys:
            if cur and (hi == none or hi != prev or len(cur) == sp):
                groups.append(cur)
                cur = []
            cur.append(s)
            prev = hi
        groups.append(cur)
        lcp = []
        for grp in groups:
            if len(grp) < 2:
                lcp.append(0)
                continue
            L = max(min(clamp[s] // 32 for s in grp), 0)
            diff = next((i for i in range(mbs)
                         if any(tables[m, i] != tables[grp[0], i] for m in grp[1:])), None)
            lcp.append(min(L, diff // 2) if diff is not None and diff < 2 * L else L)
    else:
        groups = [[s] for s in range(b)]
        lcp = [0] * b
    gunits = [(L + sum(units[m] - L for m in grp)) * hkv for grp, L in zip(groups, lcp)]
    total = sum(gunits)
    if total == 0:
        return np.zeros((b, hq), np.int64)
    nw = max(1, min(WAVES, total // MIN_UNITS))

    def wave_of(u):
        return ((u + 1) * nw - 1) // total

    def seg_slots(start, n):
        return wave_of(start + n - 1) - wave_of(start) + 1 if n > 0 else 0

    slots = np.zeros((b, hq), np.int64)
    cg = 0
    for grp, L, gu in zip(groups, lcp, gunits):
        off = cg + hkv * L
        for m in grp:
            n = units[m] - L
            for h in range(hq):
                kvh = h // g_
                slots[m, h] = seg_slots(cg + kvh * L, L) + seg_slots(off + kvh * n, n)
            off += hkv * n
        cg += gu
    return slots


def shared_tables(rng, ctx, runs):
    """Block tables: `runs` = list of (members, shared blocks); the rest private."""
    b = len(ctx)
    mbs = int(((ctx + BLOCK - 1) // BLOCK).max())
    nxt = sum(nsh for _, nsh in runs)   # shared prefixes take the lowest ids
    tables = np.full((b, mbs), -1, np.int64)
    for s in range(b):
        n = (int(ctx[s]) + BLOCK - 1) // BLOCK
        tables[s, :n] = np.arange(nxt, nxt + n)
        nxt += n
    nxt = 0
    for members, nsh in runs:
        pre = np.arange(nxt, nxt + nsh)
        nxt += nsh
        for m in members:
            k = min(nsh, (int(ctx[m]) + BLOCK - 1) // BLOCK)
            tables[m, :k] = pre[:k]
    return tables


def test_shared_layout_needs_plus_three():
    # B 3, 32 / 8 heads (groups of 2 sequences), sequences 0 and 1 sharing
    # 182 blocks: a row needs 19 slots, one more than ceil(n / 8) + 2 = 18.
    ctx = np.array([4007, 4096, 1087])
    tables = shared_tables(None, ctx, [([0, 1], 182)])
    need = layout_slots(ctx, tables, 32, 8).max()
    assert need == 19
    assert need > plan_slots(4096) - 1          # the former sizing overflowed
    assert need <= plan_slots(4096)


def test_unshared_rows_reach_one_segment_bound():
    # Without shared prefixes a row has one segment: at most ceil(n / 8) + 1
    # slots, which ragged layouts of B 6, G 1, contexts up to 16384 reach.
    rng = np.random.default_rng(5)
    found = False
    for _ in range(400):
        ctx = rng.integers(1, 16385, 6)
        ctx[0] = 16384
        tables = shared_tables(rng, ctx, [])
        need = layout_slots(ctx, tables, 4, 4).max()
        assert need <= plan_slots(16384)
        found |= need == plan_slots(16384) - 2
    assert found, "no layout reached the bound (the sweep lost its teeth)"


@pytest.mark.parametrize("seed", range(40))
def test_random_shared_prefix_layouts_fit(seed):
    rng = np.random.default_rng(1000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    g_ = int(rng.choice([1, 2, 4, 7, 8, 16]))
    b = int(rng.integers(2, 40))
    ctx = rng.integers(1, int(rng.choice([3000, 9000, 33000])), b)
    ctx[rng.integers(0, b)] = int(ctx.max()) + int(rng.integers(0, 500))
    runs = []
    perm = rng.permutation(b)
    i = 0
    while i < b:   # random runs of sharers in random batch positions
        n = int(rng.integers(1, 7))
        runs.append((list(perm[i:i + n]), int(rng.integers(0, 300))))
        i += n
    tables = shared_tables(rng, ctx, runs)
    need = layout_slots(ctx, tables, hkv * g_, hkv).max()
    assert need <= plan_slots(int(ctx.max()))


def test_workspace_size_covers_the_plan(pa):
    lib = pa._lib.load()
    for b, hq, d in ((3, 32, 128), (16, 32, 128), (64, 14, 64), (1024, 8, 256)):
        for ctx in (600, 1000, 4096, 8191, 32768, 131072):
            np_ = plan_slots(ctx)
            need = b * hq * np_ * (d + 2) * 4 + (6 * b + 2) * 4
            assert lib.pa_decode_workspace_size(b, hq, d, ctx) >= need, (b, hq, d, ctx)
