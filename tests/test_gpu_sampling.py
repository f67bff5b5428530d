"""Batched sampling on the GPU (tsa_sample_tokens) vs the oracle.

The kernel returns token indices, so the bar is equality with the oracle's
(the reference's sort/softmax/cumsum/searchsorted in fp32). The reference
sums fp32 probabilities in sort order; the kernel sums the same masses
exactly. A row may therefore differ only where one of its decisions lies
within fp32 cumsum rounding of its threshold: the oracle's fp64
decision_margin below MARGIN, which these tests check for every differing
row. Cases: the reference's known answers and allowed-set rule
(tests/model/test_batch_sampling.py); a Qwen3-vocab batch (151936 tokens)
with mixed temperatures, top-k, top-p and greedy rows in bf16, f16 and f32;
all-equal and few-valued rows (ties resolved in index order, buckets split
again); rows half masked to -inf; strided logits; repeat calls; a row alone
vs inside a batch. Top-k and greedy rows of 16-bit logits take the candidate
pass (the row read once into registers, a sample bounding its k-th largest
value, the few elements above it ranked and decided on); it is checked
against the oracle in the cases above and against the histogram paths
(TSA_SAMPLE_CANDIDATES=0) on the same rows token for token, and its edge rows
(too many candidates, -0 beside +0, the largest top_k it takes and the next,
flat rows with many candidates, short and odd-sized rows) against the
oracle. A batch of at most 256 rows of >= 16384 16-bit logits (most cases
here) spreads each histogram row's statistics and histogram passes over
several workgroups (sample_tokens' workspace); those rows are checked
against the oracle above and, token for token, against the one-workgroup
launch, including the server's default request.
"""

import os

import pytest
import torch

from oracle import sampling as osm
from tinyserver_amd import _lib
from tinyserver_amd.kernels import sample_tokens

pytestmark = pytest.mark.gpu
DEV = "cuda"
MARGIN = 2e-4  # fp32 cumsum rounding over a 151936-token row, with room


def _gpu(rows, temperature, top_k, top_p, uniforms, dtype=torch.float32):
    t = lambda v, dt: torch.tensor(v, dtype=dt, device=DEV)
    logits = rows.to(DEV, dtype) if torch.is_tensor(rows) else t(rows, dtype)
    out = sample_tokens(logits, t(temperature, torch.float32), t(top_k, torch.int64), t(top_p, torch.float32),
                        t(uniforms, torch.float32))
    torch.cuda.synchronize()
    return out.cpu()


def _oracle(rows, temperature, top_k, top_p, uniforms, dtype=torch.float32):
    t = lambda v, dt: torch.tensor(v, dtype=dt)
    logits = (rows if torch.is_tensor(rows) else t(rows, torch.float32)).to(dtype)
    return osm.sample_tokens(logits, t(temperature, torch.float32), t(top_k, torch.int64), t(top_p, torch.float32),
                             t(uniforms, torch.float32))


def _compare(rows, temperature, top_k, top_p, uniforms, dtype=torch.float32, what=""):
    got = _gpu(rows, temperature, top_k, top_p, uniforms, dtype)
    ref = _oracle(rows, temperature, top_k, top_p, uniforms, dtype)
    logits = (rows if torch.is_tensor(rows) else torch.tensor(rows)).to(dtype).float()
    diff = (got != ref).nonzero().flatten().tolist()
    for i in diff:
        m = osm.decision_margin(logits[i], temperature[i], top_k[i], top_p[i], uniforms[i])
        assert m < MARGIN, f"{what} row {i}: kernel {got[i].item()} vs oracle {ref[i].item()}, margin {m:.3e}"
    print(f"{what}: {len(diff)} of {len(got)} rows differ, all within fp32 rounding of a threshold", flush=True)
    return got, diff


def test_reference_known_answers():
    assert _gpu([[0.0] * 4] * 4, [1.0] * 4, [0] * 4, [1.0] * 4, [0.1, 0.4, 0.6, 0.9]).tolist() == [0, 1, 2, 3]
    assert _gpu([[0.0, 5.0, 5.0, 1.0]], [0.0], [0], [1.0], [0.99]).tolist() == [1]
    assert _gpu([[1.0, 9.0, 3.0, 7.0]], [1.0], [0], [1.0], [0.0]).tolist() == [1]
    row = [5.0, 4.0, 3.0, 2.0, 1.0, 0.0]
    assert _gpu([row] * 3, [1.0] * 3, [1, 2, 3], [1.0] * 3, [0.999] * 3).tolist() == [0, 1, 2]
    rows = [[-10.0] * 10 for _ in range(3)]
    rows[0][2], rows[1][7], rows[2][0] = 10.0, 10.0, 10.0
    assert _gpu(rows, [1.0] * 3, [0] * 3, [1e-6] * 3, [0.9] * 3).tolist() == [2, 7, 0]
    out = _gpu(torch.randn(3, 10), [1.0] * 3, [0] * 3, [1.0] * 3, [0.5] * 3)
    assert out.shape == (3,) and out.dtype == torch.int64


@pytest.mark.parametrize("top_k,top_p", [(0, 1.0), (5, 1.0), (0, 0.6), (5, 0.6), (1, 1.0), (1000, 1.0), (3, 0.3)])
def test_picks_inside_allowed_set(top_k, top_p):
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(4, 60, generator=g)
    allowed = [osm.allowed_set(logits[i], 0.9, top_k, top_p) for i in range(4)]
    for step in range(40):
        u = [(step * 4 + i) / 160.0 for i in range(4)]
        got = _gpu(logits, [0.9] * 4, [top_k] * 4, [top_p] * 4, u)
        assert all(t in allowed[i] for i, t in enumerate(got.tolist())), (step, got.tolist())


def _qwen3_batch(seed, b=64, v=151936):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(b, v, generator=g) * 2.5
    hot = torch.randint(0, v, (b, 8), generator=g)
    logits.scatter_add_(1, hot, torch.rand(b, 8, generator=g) * 12)  # a few likely tokens per row
    temperature = [[0.0, 0.6, 1.0, 1.3][i % 4] for i in range(b)]
    top_k = [[0, 1, 20, 50, 1000, 0, 200][i % 7] for i in range(b)]
    top_p = [[1.0, 0.9, 0.5, 0.95, 0.8][i % 5] for i in range(b)]
    uniforms = torch.rand(b, generator=g).tolist()
    return logits, temperature, top_k, top_p, uniforms


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_qwen3_vocab_batch(dtype):
    logits, temperature, top_k, top_p, uniforms = _qwen3_batch(11)
    _, diff = _compare(logits, temperature, top_k, top_p, uniforms, dtype, what=f"qwen3 vocab {dtype}")
    assert len(diff) <= 2


def test_ties_and_few_values():
    v = 151936
    g = torch.Generator().manual_seed(12)
    equal = torch.zeros(4, v)
    levels = (torch.randint(0, 6, (4, v), generator=g).float() - 3.0) * 0.5  # six values: buckets far past LDS
    rows = torch.cat([equal, levels])
    temperature = [1.0] * 8
    top_k = [0, 1000, 7, 0, 0, 5000, 100000, 0]
    top_p = [1.0, 1.0, 1.0, 0.3, 1.0, 0.9, 0.5, 0.99]
    uniforms = [0.37, 0.999, 0.0, 0.71, 0.5, 0.25, 0.62, 0.9]
    got, _ = _compare(rows, temperature, top_k, top_p, uniforms, what="ties")
    assert got[0].item() == int(0.37 * v)  # all equal: rank = index, uniform over the vocab
    # Thousands of equal probabilities: the fp32 cumsum drifts by more than one
    # of them, so hold the kernel to the same steps in fp64 instead.
    t = lambda vals, dt: torch.tensor(vals, dtype=dt)
    exact = osm.sample_tokens(rows, t(temperature, torch.float32), t(top_k, torch.int64), t(top_p, torch.float32),
                              t(uniforms, torch.float32), dtype=torch.float64)
    assert got.tolist() == exact.tolist()


def test_masked_rows():
    v = 151936
    g = torch.Generator().manual_seed(13)
    logits = torch.randn(6, v, generator=g) * 2
    logits[:, ::2] = float("-inf")
    temperature = [1.0, 0.7, 1.0, 1.0, 0.0, 1.2]
    top_k = [0, 100000, 50, 0, 0, 80000]
    top_p = [1.0, 1.0, 0.9, 0.5, 1.0, 0.99]
    uniforms = [0.5, 0.999, 0.1, 0.3, 0.7, 0.0]
    got, _ = _compare(logits, temperature, top_k, top_p, uniforms, what="masked")
    assert all(t % 2 == 1 for t in got.tolist())


def test_strided_logits_and_repeat_calls():
    logits, temperature, top_k, top_p, uniforms = _qwen3_batch(14, b=16)
    wide = torch.zeros(16, 2, logits.shape[1] + 64)
    wide[:, 1, :-64] = logits
    view = wide.to(DEV, torch.bfloat16)[:, 1, :-64]  # row stride 2 * (V + 64), like out.logits[0, :B, :]
    t = lambda v, dt: torch.tensor(v, dtype=dt, device=DEV)
    args = (t(temperature, torch.float32), t(top_k, torch.int64), t(top_p, torch.float32), t(uniforms, torch.float32))
    first = sample_tokens(view, *args)
    for _ in range(20):
        assert torch.equal(sample_tokens(view, *args), first)
    assert torch.equal(first.cpu(), _gpu(logits, temperature, top_k, top_p, uniforms, torch.bfloat16))


def test_row_alone_matches_row_in_batch():
    logits, temperature, top_k, top_p, uniforms = _qwen3_batch(15, b=16, v=4096)
    batched = _gpu(logits, temperature, top_k, top_p, uniforms)
    for i in range(16):
        assert _gpu(logits[i : i + 1], temperature[i : i + 1], top_k[i : i + 1], top_p[i : i + 1],
                    uniforms[i : i + 1]).item() == batched[i].item()


def test_rejects_bad_shapes():
    with pytest.raises(ValueError, match="Expected logits shape"):
        sample_tokens(torch.randn(10, device=DEV), torch.ones(1, device=DEV),
                      torch.zeros(1, dtype=torch.int64, device=DEV), torch.ones(1, device=DEV),
                      torch.ones(1, device=DEV) * 0.5)
    with pytest.raises(ValueError, match="Expected top_k shape"):
        sample_tokens(torch.randn(2, 10, device=DEV), torch.ones(2, device=DEV),
                      torch.zeros(3, dtype=torch.int64, device=DEV), torch.ones(2, device=DEV),
                      torch.ones(2, device=DEV) * 0.5)


DEGENERATE = (0, 1, 2, 3, 5, 6, 7)  # rows of _nonfinite_rows whose softmax is NaN


def _nonfinite_rows(v, dtype):
    g = torch.Generator().manual_seed(16)
    rows = torch.randn(10, v, generator=g) * 2.5
    rows[0, 7] = float("nan")              # one NaN among finite logits
    rows[1, ::3] = float("nan")            # many NaNs
    rows[2, 100] = float("inf")            # a +inf maximum
    rows[3, :] = float("nan")              # every logit NaN
    rows[4, 5] = float("-inf")             # one -inf: an ordinary row
    rows[5, 9] = float("inf")              # +inf and NaN
    rows[5, 10] = float("nan")
    rows[6, :] = float("-inf")             # every logit -inf
    rows[7, 50] = float("inf")             # two +inf, ties in index order
    rows[7, 20] = float("inf")
    rows[8, : v // 2] = float("-inf")      # half masked, finite rest: ordinary
    rows[9, :] = float("-inf")             # one finite logit among -inf
    rows[9, v - 3] = 1.0
    return rows.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_nonfinite_rows_match_reference(dtype):
    """Rows with NaN, +inf or only -inf logits at the Qwen3 vocabulary size.
    The reference's formulation fixes the answer: a greedy row takes rank 0
    of the stable descending sort (NaN first, so the first NaN; else the
    first maximum; index 0 when every logit is -inf); any other row whose
    softmax is NaN gets searchsorted's past-the-end rank clamped to the last
    rank (the last index of the minimum, vocab-1 when all are NaN). Every
    index lies in [0, vocab) and equals the oracle's, for greedy and sampled
    rows, with and without top-k/top-p."""
    v = 151936
    rows = _nonfinite_rows(v, dtype)
    n = rows.shape[0]
    for temp, k, p, u in ((0.0, 0, 1.0, 0.5), (1.0, 0, 1.0, 0.3), (0.7, 50, 0.9, 0.6), (1.0, 0, 0.5, 0.9),
                          (0.9, 10, 0.8, 0.0)):
        args = ([temp] * n, [k] * n, [p] * n, [u] * n)
        got, _ = _compare(rows, *args, dtype=dtype, what=f"non-finite T={temp} k={k} p={p} u={u}")
        ref = _oracle(rows, *args, dtype=dtype)
        assert ((got >= 0) & (got < v)).all(), (temp, k, p, u, got.tolist())
        for i in DEGENERATE:  # fixed by the NaN/inf rules, not by rounding
            assert got[i].item() == ref[i].item(), (i, temp, k, p, u, got.tolist(), ref.tolist())
    # the hand-derived answers, for the greedy and one sampled setting
    greedy = _gpu(rows, [0.0] * n, [0] * n, [1.0] * n, [0.5] * n, dtype=dtype).tolist()
    assert greedy[0] == 7 and greedy[1] == 0 and greedy[2] == 100 and greedy[3] == 0
    assert greedy[5] == 10 and greedy[6] == 0 and greedy[7] == 20 and greedy[9] == v - 3
    sampled = _gpu(rows, [1.0] * n, [0] * n, [1.0] * n, [0.3] * n, dtype=dtype).tolist()
    assert sampled[3] == v - 1 and sampled[6] == v - 1


def _single_kernel(logits, temperature, top_k, top_p, uniforms):
    """sample_tokens with the candidate pass switched off: every row on the
    histogram paths."""
    os.environ["TSA_SAMPLE_CANDIDATES"] = "0"
    try:
        out = sample_tokens(logits, temperature, top_k, top_p, uniforms)
        torch.cuda.synchronize()
    finally:
        del os.environ["TSA_SAMPLE_CANDIDATES"]
    return out.cpu()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_candidate_path_matches_single_kernel(dtype):
    """The same 64 Qwen3-vocab rows through both paths: the same tokens,
    except where the oracle's decision margin puts a row within fp32
    rounding of a threshold."""
    logits, temperature, top_k, top_p, uniforms = _qwen3_batch(17)
    t = lambda v, dt: torch.tensor(v, dtype=dt, device=DEV)
    args = (logits.to(DEV, dtype), t(temperature, torch.float32), t(top_k, torch.int64), t(top_p, torch.float32),
            t(uniforms, torch.float32))
    fast = sample_tokens(*args).cpu()
    full = _single_kernel(*args)
    lf = logits.to(dtype).float()
    diff = (fast != full).nonzero().flatten().tolist()
    for i in diff:
        m = osm.decision_margin(lf[i], temperature[i], top_k[i], top_p[i], uniforms[i])
        assert m < MARGIN, f"row {i}: candidate path {fast[i].item()} vs single kernel {full[i].item()}, margin {m:.3e}"
    print(f"candidate vs single-kernel path, {dtype}: {len(diff)} of 64 rows differ", flush=True)
    assert len(diff) <= 2


def test_candidate_path_edge_rows():
    """bf16 rows at the edges of the candidate path, against the oracle:
    all-equal and two-valued rows (too many candidates: the histogram paths
    take them); -0 and +0 ties; top_k 512 (the largest the pass takes) and
    513; greedy rows with the tied maximum at both ends of the row."""
    v = 151936
    g = torch.Generator().manual_seed(18)
    base = torch.randn(4, v, generator=g) * 2.5
    equal = torch.zeros(2, v)
    two = (torch.rand(2, v, generator=g) < 0.5).float()
    zeros = torch.randn(2, v, generator=g)
    zeros[:, ::5] = 0.0
    zeros[:, 1::5] = -0.0
    zeros[:, 2::7] = -3.0
    tied = torch.randn(2, v, generator=g)
    tied[:, [v - 1, 40000, 7]] = 9.0  # the same maximum at three places
    rows = torch.cat([base, equal, two, zeros, tied])
    temperature = [0.8, 1.0, 0.7, 1.2, 1.0, 1.0, 1.0, 0.9, 1.0, 0.5, 0.0, 1.0]
    top_k = [512, 513, 1, 50, 10, 1, 20, 500, 3, 5, 0, 2]
    top_p = [0.9, 0.9, 1.0, 0.5, 1.0, 1.0, 0.7, 1.0, 1.0, 0.6, 1.0, 1.0]
    uniforms = [0.5, 0.2, 0.9, 0.99, 0.3, 0.0, 0.45, 0.8, 0.1, 0.7, 0.5, 0.75]
    got, _ = _compare(rows, temperature, top_k, top_p, uniforms, dtype=torch.bfloat16, what="candidate edges")
    assert got[10].item() == 7  # greedy: the first index of the tied maximum
    ref_exact = osm.sample_tokens(rows.to(torch.bfloat16), torch.tensor(temperature), torch.tensor(top_k),
                                  torch.tensor(top_p), torch.tensor(uniforms), dtype=torch.float64)
    assert got[4:6].tolist() == ref_exact[4:6].tolist()  # all-equal rows: exact in fp64


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_candidate_path_large_k(dtype):
    """top_k from 127 up to the pass's largest, 512, on Qwen3-vocab rows with
    a few hot tokens and on flat rows (many near-ties, so far more than k
    candidates): the oracle, and the histogram paths token for token."""
    v = 151936
    g = torch.Generator().manual_seed(23)
    hot, _, _, _, _ = _qwen3_batch(24, b=8)
    flat = torch.randn(8, v, generator=g) * 0.05
    rows = torch.cat([hot, flat])
    ks = [127, 128, 129, 200, 300, 400, 511, 512] * 2
    temperature = [1.0, 0.8, 1.2, 0.7, 1.0, 0.9, 1.1, 1.0] * 2
    top_p = [1.0, 0.95, 0.9, 1.0, 0.8, 1.0, 0.99, 0.5] * 2
    uniforms = torch.rand(16, generator=g).tolist()
    got, _ = _compare(rows, temperature, ks, top_p, uniforms, dtype=dtype, what=f"large k {dtype}")
    t = lambda x, dt: torch.tensor(x, dtype=dt, device=DEV)
    full = _single_kernel(rows.to(DEV, dtype), t(temperature, torch.float32), t(ks, torch.int64),
                          t(top_p, torch.float32), t(uniforms, torch.float32))
    assert torch.equal(got, full), (got.tolist(), full.tolist())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_candidate_path_negative_rows(dtype):
    """Rows with no non-negative logit (shifted logits, log-probabilities,
    shifted rows a third -inf), whose signed raw maxima are each set's
    smallest element: the candidate pass takes its samples from the keys
    instead. The oracle, and the histogram paths token for token."""
    base, _, _, _, _ = _qwen3_batch(28, b=4)
    shifted = base - 40.0
    logp = torch.log_softmax(base / 0.8, dim=-1)
    masked = shifted.clone()
    masked[:, ::3] = -float("inf")
    rows = torch.cat([shifted, logp, masked])
    temperature = [0.8, 1.0, 0.0, 1.2] * 3
    ks = [50, 1, 0, 400, 20, 128, 0, 50, 50, 3, 0, 300]
    top_p = [0.9, 1.0, 1.0, 0.95, 0.5, 1.0, 1.0, 0.9, 0.9, 1.0, 1.0, 0.8]
    g = torch.Generator().manual_seed(29)
    uniforms = torch.rand(12, generator=g).tolist()
    got, _ = _compare(rows, temperature, ks, top_p, uniforms, dtype=dtype, what=f"negative rows {dtype}")
    t = lambda x, dt: torch.tensor(x, dtype=dt, device=DEV)
    full = _single_kernel(rows.to(DEV, dtype), t(temperature, torch.float32), t(ks, torch.int64),
                          t(top_p, torch.float32), t(uniforms, torch.float32))
    assert torch.equal(got, full), (got.tolist(), full.tolist())


@pytest.mark.parametrize("v", [8, 200, 1001, 4096 + 8, 155648, 155656])
def test_candidate_path_short_and_odd_rows(v):
    """Short rows (most threads hold no chunk), a row whose length is not a
    multiple of 8, the longest row the pass holds in registers (155,648
    logits) and the next multiple of 8 (the histogram paths), against the
    oracle."""
    g = torch.Generator().manual_seed(19 + v)
    rows = torch.randn(6, v, generator=g) * 2
    k = min(5, v - 1)
    _compare(rows, [1.0, 0.0, 0.7, 1.0, 1.3, 0.9], [k, 0, 1, k, 3 if v > 3 else 1, 2], [0.9, 1.0, 1.0, 0.5, 1.0, 0.8],
             [0.1, 0.5, 0.6, 0.99, 0.3, 0.0], dtype=torch.bfloat16, what=f"v={v}")


def _one_workgroup(logits, temperature, top_k, top_p, uniforms):
    """tsa_sample_tokens without a workspace: every row on one workgroup."""
    out = torch.empty(logits.shape[0], dtype=torch.int64, device=DEV)
    views = [_lib.view(x) for x in (out, logits, temperature, top_k, top_p, uniforms)]
    _lib.check(_lib.load().tsa_sample_tokens(*map(_lib.ref, views), _lib.stream_of(logits.device)), "one workgroup")
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("b", [1, 3, 64, 85, 86, 256])
def test_split_rows_match_one_workgroup(dtype, b):
    """A batch of at most 256 rows of >= 16384 16-bit logits spreads its
    histogram rows' statistics and histogram passes over several workgroups
    per row (16 segments at b = 1 and 3, 8 at 64, 6 at 85, 5 at 86, 2 at
    256), and up to b = 85 (segments of at most 28,160 logits) the
    histogram pass also writes each segment's bucket lists, which the
    decision gathers from: token for token the one-workgroup path's, for
    rows of every kind (the server's default request, top-p only, full,
    top_k > 512 with top-p, top-k and greedy rows that take the candidate
    pass)."""
    g = torch.Generator().manual_seed(31 + b)
    v = 151936
    logits = torch.randn(b, v, generator=g) * 2.5
    logits.scatter_add_(1, torch.randint(0, v, (b, 8), generator=g), torch.rand(b, 8, generator=g) * 12)
    kinds = [(1.0, 0, 0.95), (0.8, 0, 0.9), (1.3, 0, 1.0), (0.7, 2000, 0.8), (1.0, 50, 0.9), (0.0, 0, 1.0)]
    temperature = [kinds[i % 6][0] for i in range(b)]
    top_k = [kinds[i % 6][1] for i in range(b)]
    top_p = [kinds[i % 6][2] for i in range(b)]
    uniforms = torch.rand(b, generator=g).tolist()
    t = lambda x, dt: torch.tensor(x, dtype=dt, device=DEV)
    args = (logits.to(DEV, dtype), t(temperature, torch.float32), t(top_k, torch.int64), t(top_p, torch.float32),
            t(uniforms, torch.float32))
    assert _lib.load().tsa_sample_tokens_workspace_bytes(b, v) > 0
    split = sample_tokens(*args).cpu()
    assert torch.equal(split, _one_workgroup(*args)), (split.tolist(), _one_workgroup(*args).tolist())


def test_server_default_request():
    """The reference server's default request (temperature 1.0, top_p 0.95,
    top_k 0: server/api/schema.py:11-15) over a 64-row Qwen3-vocab bf16
    batch, through the split rows: against the oracle and the one-workgroup
    path."""
    logits, _, _, _, uniforms = _qwen3_batch(27)
    b = logits.shape[0]
    _compare(logits, [1.0] * b, [0] * b, [0.95] * b, uniforms, torch.bfloat16, what="server default")
    t = lambda x, dt: torch.tensor(x, dtype=dt, device=DEV)
    args = (logits.to(DEV, torch.bfloat16), t([1.0] * b, torch.float32), t([0] * b, torch.int64),
            t([0.95] * b, torch.float32), t(uniforms, torch.float32))
    assert torch.equal(sample_tokens(*args).cpu(), _one_workgroup(*args))


def test_split_workspace_checks():
    """tsa_sample_tokens_ws: a workspace smaller than asked for is refused; a
    NULL one is the one-workgroup launch."""
    lib = _lib.load()
    logits, temperature, top_k, top_p, uniforms = _qwen3_batch(28, b=8)
    t = lambda x, dt: torch.tensor(x, dtype=dt, device=DEV)
    args = (logits.to(DEV, torch.bfloat16), t(temperature, torch.float32), t(top_k, torch.int64),
            t(top_p, torch.float32), t(uniforms, torch.float32))
    out = torch.empty(8, dtype=torch.int64, device=DEV)
    views = [_lib.view(x) for x in (out, *args)]
    need = lib.tsa_sample_tokens_workspace_bytes(8, logits.shape[1])
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError, match="workspace too small"):
        _lib.check(lib.tsa_sample_tokens_ws(*map(_lib.ref, views), ws.data_ptr(), need - 1, _lib.stream_of(ws.device)),
                   "ws")
    _lib.check(lib.tsa_sample_tokens_ws(*map(_lib.ref, views), None, 0, _lib.stream_of(ws.device)), "ws")
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), _one_workgroup(*args))


def test_graph_replays_match_eager():
    """sample_tokens captured in a HIP graph (a serving step's usual form):
    three replays, with eager work and a synchronisation between them, each
    equal to the eager call, for candidate-pass and histogram-path rows."""
    logits, temperature, top_k, top_p, uniforms = _qwen3_batch(26, b=16)
    t = lambda x, dt: torch.tensor(x, dtype=dt, device=DEV)
    args = (logits.to(DEV, torch.bfloat16), t(temperature, torch.float32), t(top_k, torch.int64),
            t(top_p, torch.float32), t(uniforms, torch.float32))
    eager = sample_tokens(*args).cpu()
    out = torch.full((16,), -1, dtype=torch.int64, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        sample_tokens(*args, out=out)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sample_tokens(*args, out=out)
    for rep in range(3):
        out.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), eager), (rep, out.tolist(), eager.tolist())
        sample_tokens(*args)  # eager work between replays
        torch.cuda.synchronize()
