"""The sampling oracle (oracle/sampling.py) pinned on the CPU.

* The reference's known answers (tests/model/test_batch_sampling.py:64-70,
  139-141, 179-213): hand-computed CDF, greedy ties to the lowest index,
  u = 0, per-row top-k, tiny top-p.
* The reference's independent rule (:27-52, an fp64 loop over the sorted
  order): every pick lies in the allowed set, for the reference's filter
  grid.
* Closed form: over a fine grid of uniforms, each kept token is picked for a
  share of the grid equal to its renormalised probability.
* Identities: top_k = 1 is argmax, top_k >= V is no filter, greedy rows are
  argmax, a row's token does not depend on the rest of the batch.
* A planted mistake (the top-p test on the mass *including* the rank) fails
  the allowed-set check, so that check can tell.
"""

import pytest
import torch

from oracle import sampling as osm


def _call(rows, temperature, top_k, top_p, uniforms, fn=osm.sample_tokens):
    return fn(torch.tensor(rows, dtype=torch.float32), torch.tensor(temperature, dtype=torch.float32),
              torch.tensor(top_k, dtype=torch.int64), torch.tensor(top_p, dtype=torch.float32),
              torch.tensor(uniforms, dtype=torch.float32))


def test_reference_known_answers():
    assert _call([[0.0] * 4] * 4, [1.0] * 4, [0] * 4, [1.0] * 4, [0.1, 0.4, 0.6, 0.9]).tolist() == [0, 1, 2, 3]
    assert _call([[0.0, 5.0, 5.0, 1.0]], [0.0], [0], [1.0], [0.99]).tolist() == [1]
    assert _call([[1.0, 9.0, 3.0, 7.0]], [1.0], [0], [1.0], [0.0]).tolist() == [1]
    row = [5.0, 4.0, 3.0, 2.0, 1.0, 0.0]
    assert _call([row] * 3, [1.0] * 3, [1, 2, 3], [1.0] * 3, [0.999] * 3).tolist() == [0, 1, 2]
    rows = [[-10.0] * 10 for _ in range(3)]
    rows[0][2], rows[1][7], rows[2][0] = 10.0, 10.0, 10.0
    assert _call(rows, [1.0] * 3, [0] * 3, [1e-6] * 3, [0.9] * 3).tolist() == [2, 7, 0]


def _planted_top_p(logits, temperature, top_k, top_p, uniforms):
    """The oracle with the top-p test moved onto the inclusive mass."""
    x = logits.float() / temperature.float().clamp(min=1e-5).unsqueeze(-1)
    sx, order = torch.sort(x, dim=-1, descending=True, stable=True)
    probs = torch.softmax(sx, dim=-1)
    cum = torch.cumsum(probs, dim=-1)
    remove = cum > top_p.unsqueeze(-1)
    remove[:, 0] = False
    probs = probs.masked_fill(remove, 0.0)
    cdf = torch.cumsum(probs, dim=-1)
    picked = torch.searchsorted(cdf, (uniforms.unsqueeze(-1) * cdf[:, -1:]).contiguous()).clamp(max=x.shape[1] - 1)
    return order.gather(-1, picked).squeeze(-1)


@pytest.mark.parametrize("top_k,top_p", [(0, 1.0), (5, 1.0), (0, 0.6), (5, 0.6), (1, 1.0), (1000, 1.0), (3, 0.3)])
def test_picks_inside_allowed_set(top_k, top_p):
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(4, 60, generator=g)
    allowed = [osm.allowed_set(logits[i], 0.9, top_k, top_p) for i in range(4)]
    for step in range(40):
        u = [(step * 4 + i) / 160.0 for i in range(4)]
        got = _call(logits.tolist(), [0.9] * 4, [top_k] * 4, [top_p] * 4, u)
        assert all(t in allowed[i] for i, t in enumerate(got.tolist()))


def test_planted_mistake_leaves_allowed_set():
    g = torch.Generator().manual_seed(4)
    logits = torch.randn(4, 60, generator=g)
    allowed = [osm.allowed_set(logits[i], 0.9, 0, 0.6) for i in range(4)]
    bad = False
    for step in range(40):
        u = [(step * 4 + i) / 160.0 for i in range(4)]
        got = _call(logits.tolist(), [0.9] * 4, [0] * 4, [0.6] * 4, u, fn=_planted_top_p)
        bad |= any(t not in allowed[i] for i, t in enumerate(got.tolist()))
    # the planted rule drops the rank that straddles top_p, which the rule keeps;
    # so it never picks outside the set -- but it never picks that rank either
    kept_ranks = set()
    for step in range(400):
        u = [step / 400.0] * 4
        kept_ranks |= set(_call(logits.tolist(), [0.9] * 4, [0] * 4, [0.6] * 4, u).tolist())
    planted = set()
    for step in range(400):
        u = [step / 400.0] * 4
        planted |= set(_call(logits.tolist(), [0.9] * 4, [0] * 4, [0.6] * 4, u, fn=_planted_top_p).tolist())
    assert bad or planted != kept_ranks


def test_pick_frequencies_match_closed_form():
    g = torch.Generator().manual_seed(7)
    row = torch.randn(12, generator=g) * 1.5
    temp, top_k, top_p = 0.8, 9, 0.85
    n = 20000
    got = _call([row.tolist()] * n, [temp] * n, [top_k] * n, [top_p] * n, [(i + 0.5) / n for i in range(n)])
    x = row.double() / temp
    xs, order = torch.sort(x, descending=True, stable=True)
    p = torch.softmax(xs[:top_k], dim=0)
    before = torch.cumsum(p, 0) - p
    keep = before <= top_p
    keep[0] = True
    q = p[keep] / p[keep].sum()
    for rank, tok in enumerate(order[: int(keep.sum())].tolist()):
        share = (got == tok).double().mean().item()
        assert abs(share - q[rank].item()) < 2.0 / n + 1e-4, (rank, share, q[rank].item())
    assert set(got.tolist()) <= set(order[: int(keep.sum())].tolist())


def test_identities():
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(4, 30, generator=g)
    assert _call(logits.tolist(), [1.0] * 4, [1] * 4, [1.0] * 4, [0.0, 0.4, 0.8, 0.99]).tolist() == \
        logits.argmax(-1).tolist()
    u = [0.15, 0.55, 0.85, 0.3]
    assert torch.equal(_call(logits.tolist(), [1.0] * 4, [0] * 4, [1.0] * 4, u),
                       _call(logits.tolist(), [1.0] * 4, [999] * 4, [1.0] * 4, u))
    assert _call(logits.tolist(), [0.0] * 4, [0] * 4, [0.9] * 4, u).tolist() == logits.argmax(-1).tolist()
    rows = torch.randn(8, 50, generator=g)
    us = [(i + 0.3) / 8 for i in range(8)]
    batched = _call(rows.tolist(), [1.0] * 8, [10] * 8, [0.95] * 8, us)
    for i in range(8):
        assert _call([rows[i].tolist()], [1.0], [10], [0.95], [us[i]]).item() == batched[i].item()


def test_decision_margin_flags_a_straddled_threshold():
    row = torch.tensor([1.0, 0.0, -1.0])
    p = torch.softmax(row.double(), 0)
    # u exactly on the first cdf step: margin 0
    assert osm.decision_margin(row, 1.0, 0, 1.0, float(p[0])) < 1e-12
    assert osm.decision_margin(row, 1.0, 0, 1.0, float(p[0]) / 2) > 0.05  # nearest: mass before rank 2 (0.91) vs 1.0
    # top_p exactly at the mass before rank 1
    assert osm.decision_margin(row, 1.0, 0, float(p[0]), 0.01) < 1e-12


def test_rejects_bad_shapes():
    with pytest.raises(ValueError, match="Expected logits shape"):
        osm.sample_tokens(torch.randn(10), torch.ones(1), torch.zeros(1, dtype=torch.int64), torch.ones(1),
                          torch.ones(1) * 0.5)
    with pytest.raises(ValueError, match="Expected top_k shape"):
        osm.sample_tokens(torch.randn(2, 10), torch.ones(2), torch.zeros(3, dtype=torch.int64), torch.ones(2),
                          torch.ones(2) * 0.5)


def test_nonfinite_rows_follow_sort_and_searchsorted_rules():
    """What the reference's formulation gives rows whose softmax is NaN,
    derived by hand from torch's semantics: the stable descending sort puts
    NaN first (ties by index); a greedy row takes rank 0; otherwise softmax
    and cumsum are NaN, searchsorted's lower bound of a NaN target runs past
    the end (its test, not (cdf >= target), is true for NaN), and the clamp
    to vocab-1 picks the last rank: the last index of the minimum."""
    v = 12
    nan, inf = float("nan"), float("inf")
    rows = torch.tensor([
        [0.5, 1.0, nan, 2.0, -1.0, 0.0, -1.0, 3.0, nan, 0.1, 0.2, 0.3],  # NaN at 2 and 8; min -1 last at 6
        [nan] * v,
        [-inf] * v,
        [0.0, inf, 1.0, inf, -2.0, -2.0, 5.0, 0.0, 0.0, 0.0, 0.0, 0.0],   # +inf at 1 and 3; min -2 last at 5
    ])
    n = rows.shape[0]
    for k, p, u in ((0, 1.0, 0.5), (3, 0.9, 0.1), (0, 0.2, 0.99)):
        greedy = osm.sample_tokens(rows, torch.zeros(n), torch.full((n,), k), torch.full((n,), p),
                                   torch.full((n,), u)).tolist()
        assert greedy == [2, 0, 0, 1]
        sampled = osm.sample_tokens(rows, torch.ones(n), torch.full((n,), k), torch.full((n,), p),
                                    torch.full((n,), u)).tolist()
        assert sampled == [6, v - 1, v - 1, 5]
