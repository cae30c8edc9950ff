"""Pins the routing oracle (CPU): the reference's own known answers, the
pure-Python brute force, closed forms and special cases."""
import math
import random

import pytest
import torch

from oracle import brute
from oracle import routing as R


def test_masked_softmax_known_answer():
    # reference tests/test_indexer.py:10-18
    scores = torch.tensor([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
    mask = torch.tensor([[True, True, False], [False, True, True]])
    p = R.masked_probs(scores, mask)
    assert p[0, 2].item() == 0.0 and p[1, 0].item() == 0.0
    assert abs(p[0, :2].sum().item() - 1.0) < 1e-5
    assert abs(p[1, 1:].sum().item() - 1.0) < 1e-5
    # closed form e^1/(e^1+e^2)
    assert abs(p[0, 0].item() - math.exp(1) / (math.exp(1) + math.exp(2))) < 1e-7


def test_masked_softmax_all_masked_row_and_dtype():
    s = torch.randn(3, 5).bfloat16()
    m = torch.ones(3, 5, dtype=torch.bool)
    m[1] = False
    p = R.masked_probs(s, m)
    assert p.dtype == torch.bfloat16
    assert torch.all(p[1] == 0)
    ref = torch.softmax(s.double(), -1)
    assert torch.allclose(p[0].double(), ref[0], atol=4e-3)


def test_select_blocks_causal_known_answer():
    # reference tests/test_indexer.py:20-40
    scores = torch.zeros(1, 4, 4)
    scores[0, 3, 0] = 10.0
    r = R.select_route(scores, causal=True, block_size=16, local_window_blocks=1, top_p=0.9,
                       min_remote_blocks=0, max_remote_blocks=2, remote_capacity=2)
    assert r["remote_counts"][0, 0].item() == 0
    assert r["remote_counts"][0, 3].item() == 1
    assert r["remote_indices"][0, 3, 0].item() == 0


def test_select_blocks_guardrails():
    # reference tests/test_indexer.py:42-61
    torch.manual_seed(1)
    scores = torch.randn(2, 8, 8)
    r = R.select_route(scores, causal=False, local_window_blocks=2, top_p=0.99, min_remote_blocks=1,
                       max_remote_blocks=3, remote_capacity=4)
    c = r["remote_counts"]
    assert int(c.min()) >= 1 and int(c.max()) <= 3


CASES = [
    # causal, local_window, top_p, kmin, kmax, cap, nb, qb, sharpness
    (False, 0, 0.9, 0, 4, 4, 16, 6, 6.0),
    (False, 2, 0.9, 1, 3, 5, 12, 5, 8.0),
    (False, 3, 0.5, 2, 6, 6, 20, 4, 3.0),
    (True, 0, 0.9, 0, 3, 4, 10, 10, 6.0),
    (True, 2, 0.8, 1, 2, 3, 10, 10, 7.0),
    (True, 1, 0.95, 0, 8, 8, 12, 12, 5.0),
    (False, 4, 0.3, 0, 5, 5, 10, 3, 9.0),  # base mass can exceed top_p
]


@pytest.mark.parametrize("case", CASES)
def test_select_route_matches_brute_force(case):
    causal, lw, top_p, kmin, kmax, cap, nb, qb, sharp = case
    rng = random.Random(hash(case) & 0xffff)
    B = 2
    # quantised sharp scores: distinct values on a coarse grid, so fp32 vs fp64 cannot flip ranks
    vals = [[[rng.randrange(-40, 40) * sharp / 40.0 + 1e-3 * j for j in range(nb)] for _ in range(qb)] for _ in range(B)]
    scores = torch.tensor(vals, dtype=torch.float32)
    r = R.select_route(scores, causal=causal, local_window_blocks=lw, top_p=top_p, min_remote_blocks=kmin,
                       max_remote_blocks=kmax, remote_capacity=cap)
    for b in range(B):
        for q in range(qb):
            c, l, m = brute.masks(q, nb, causal, lw)
            idx, cnt = brute.select_row(vals[b][q], c, l, m, top_p, kmin, kmax, cap)
            cum = r["cumulative"][b, q]
            tgt = float(r["target"][b, q])
            # a count is only comparable when no cumulative mass sits within fp32 noise of the target
            near = bool(((cum - tgt).abs() < 1e-5).any())
            if not near:
                assert int(r["remote_counts"][b, q]) == cnt, (b, q)
            got = r["remote_indices"][b, q, :cnt].tolist()
            assert got == idx[:cnt], (b, q, got, idx[:cnt])


def test_select_special_cases():
    # single spike -> one remote block
    s = torch.full((1, 1, 32), -20.0)
    s[0, 0, 7] = 20.0
    r = R.select_route(s, causal=False, top_p=0.9, max_remote_blocks=8, remote_capacity=8)
    assert int(r["remote_counts"][0, 0]) == 1 and int(r["remote_indices"][0, 0, 0]) == 7
    # flat scores -> K_max cap binds
    r = R.select_route(torch.zeros(1, 1, 64), causal=False, top_p=0.9, max_remote_blocks=5, remote_capacity=5)
    assert int(r["remote_counts"][0, 0]) == 5
    # no remote candidates -> 0 even with K_min
    r = R.select_route(torch.zeros(1, 2, 4), causal=True, local_window_blocks=4, top_p=0.9, min_remote_blocks=2,
                       max_remote_blocks=3, remote_capacity=3)
    assert r["remote_counts"].tolist() == [[0, 0]]
    # base mass >= top_p -> target 0 -> count = K_min
    s = torch.zeros(1, 1, 10)
    s[0, 0, :2] = 30.0
    r = R.select_route(s, causal=False, local_window_blocks=2, top_p=0.9, min_remote_blocks=2, max_remote_blocks=4,
                       remote_capacity=4)
    assert int(r["remote_counts"][0, 0]) == 2
    # capacity beyond total blocks zero-pads
    r = R.select_route(torch.randn(1, 1, 3), causal=False, top_p=0.9, max_remote_blocks=3, remote_capacity=6)
    assert r["remote_indices"][0, 0, 3:].tolist() == [0, 0, 0]


def test_cumsum_accumulates_in_fp64():
    # the property the GPU prefix sum relies on (fp64 running sum, rounded per element)
    torch.manual_seed(0)
    p = torch.softmax(torch.randn(8, 2048) * 0.3, -1)
    c = p.cumsum(-1)
    ref = torch.cumsum(p.double(), -1).float()
    assert torch.equal(c, ref)


def test_cosine_scores_closed_form():
    torch.manual_seed(0)
    q = torch.randn(2, 5, 16)
    k = torch.randn(2, 7, 16)
    s = R.cosine_scores_f32(q, k)
    ref = torch.einsum("bqd,bkd->bqk", q.double(), k.double()) / (
        q.double().norm(dim=-1)[..., None] * k.double().norm(dim=-1)[:, None, :]) / 4.0
    assert torch.allclose(s.double(), ref, atol=1e-6)


def test_mlp_pooled_route_against_fp64_and_brute_topk():
    torch.manual_seed(3)
    D, Nb, base, remote = 64, 24, 3, 5
    x = torch.randn(10, D)
    wq = torch.randn(16, D) * D ** -0.5
    keys = torch.randn(Nb, 16) * 0.25
    active = R.mlp_pooled_route(x, wq, keys, base, remote)
    q = x.double().mean(0) @ wq.double().t()
    q = q / torch.sqrt((q * q).mean() + 1.1920928955078125e-07)
    s = (q @ keys.double().t()).tolist()
    top = brute.topk_desc(s[base:], remote)
    assert active.tolist() == list(range(base)) + [t + base for t in top]
    assert active.dtype == torch.int32


def test_decode_route_brute_force():
    torch.manual_seed(5)
    B, P, d = 3, 40, 16
    kp = torch.nn.functional.normalize(torch.randn(B, P, d), dim=-1)
    qi = torch.randn(B, 1, d) * 3
    page, W, pos = 8, 64, 8 * 30 + 3
    r = R.decode_route(qi, kp, pos, page, W, completed_pages=30, top_p=0.6, min_remote=1, max_remote=5)
    flp = r["first_local_page"]
    assert flp == (pos + 1 - W) // page
    for b in range(B):
        qn = qi[b, 0].double() / qi[b, 0].double().norm()
        s = [(float(qn @ kp[b, j].double()) / 4.0) for j in range(flp)]
        m = max(s)
        e = [math.exp(v - m) for v in s]
        z = sum(e)
        p = [v / z for v in e]
        order = sorted(range(flp), key=lambda j: (-p[j], j))
        run, below = 0.0, 0
        for j in order:
            run += p[j]
            below += run < 0.6
        need = max(1, min(below + 1, min(5, flp)))
        assert r["pages"][b] == order[:need]
        assert all(pg < flp for pg in r["pages"][b])
