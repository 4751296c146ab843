"""GPU parity of pa_argmax (greedy sampling over logit rows) with the
oracle's restatement of argmax_logits (crates/traits/src/sampling.rs:439-453):
bit-exact indices for bf16 and f32 rows, vocabulary sizes that take the
vector and the scalar load paths, ties, NaN, all -inf, signed zeros,
strided rows and the empty vocabulary."""
import numpy as np
import pytest
import torch


pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def special_rows(x):
    """Overwrites the first rows of x [rows, vocab] (f32, host) with the
    edge cases of the reference's rule."""
    n = x.shape[1]
    cases = [
        lambda r: r.fill_(1.0),                                   # all equal: index 0
        lambda r: r.fill_(float("nan")),                          # all NaN: 0
        lambda r: r.fill_(float("-inf")),                         # nothing above -inf: 0
        lambda r: (r.fill_(0.0), r.__setitem__(0, -0.0)),         # -0 == +0: index 0
        lambda r: r.__setitem__(slice(0, None, 2), float("nan")),  # NaN interleaved
        lambda r: (r.__setitem__(n - 1, 1e4), r.__setitem__(n // 2, 1e4)),  # tie, first wins
        lambda r: r.__setitem__(n - 1, float("inf")),             # the last column
        lambda r: r.__setitem__(0, float("nan")),                 # NaN in front of the max
    ]
    for i, f in enumerate(cases[:x.shape[0]]):
        f(x[i])
    return x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,vocab", [(32, 151936), (3, 1001), (9, 8), (1, 7), (12, 4096),
                                        (64, 32000)])
def test_argmax_matches_oracle(pa, oracle, dtype, rows, vocab):
    g = torch.Generator().manual_seed(rows * 31 + vocab)
    host = special_rows(torch.randn(rows, vocab, generator=g) * 4)
    # bf16 rounding makes many ties: the first must win
    x = host.to(dtype)
    expect = oracle.argmax_logits(x.float().numpy())
    got = pa.argmax(x.to(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, expect)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_argmax_strided_rows(pa, oracle, dtype):
    g = torch.Generator().manual_seed(5)
    full = (torch.randn(16, 2048, generator=g) * 3).to(dtype)
    fd = full.to(DEV)
    # 16-byte aligned rows of stride 2048 (vector loads), then an unaligned
    # start (scalar loads)
    for lo, n in ((64, 1536), (3, 1500)):
        expect = oracle.argmax_logits(full[:, lo:lo + n].float().numpy())
        np.testing.assert_array_equal(pa.argmax(fd[:, lo:lo + n]).cpu().numpy(), expect)


def test_argmax_expanded_rows(pa, oracle):
    # a broadcast view (row stride 0) is read as the rows it shows
    row = (torch.randn(1, 3000, generator=torch.Generator().manual_seed(2)) * 3)
    x = row.to(DEV).expand(5, 3000)
    expect = oracle.argmax_logits(row.expand(5, 3000).numpy())
    np.testing.assert_array_equal(pa.argmax(x).cpu().numpy(), expect)


def test_argmax_empty_vocab_and_rows(pa):
    x = torch.empty(4, 0, dtype=torch.bfloat16, device=DEV)
    np.testing.assert_array_equal(pa.argmax(x).cpu().numpy(), np.zeros(4, np.int64))
    x = torch.empty(0, 100, dtype=torch.float32, device=DEV)
    assert pa.argmax(x).shape == (0,)


def test_argmax_rejects_bad_layout(pa):
    x = torch.zeros(8, 16, dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):
        pa.argmax(x.t())
