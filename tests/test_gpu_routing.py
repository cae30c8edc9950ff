"""GPU parity of the HIP routing kernels against the CPU oracle.

Routing is bit-exact up to the reference's own indeterminacy (equal or
ulp-close probabilities, cumulative mass on the target); see route_check.py.
Floating-point outputs: masked_softmax within 1e-6 relative (fp32: exp and the
row sum may each differ by a few ulp from ATen's CPU kernels) / 1 bf16 ulp of
the oracle; decode-route context within bf16 rel-L2 2e-3."""
import math

import pytest
import torch

from oracle import routing as R
from route_check import check_rows, tolerances

pytestmark = pytest.mark.gpu


def _scores(B, Qb, Nb, seed, scale=3.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, Qb, Nb, generator=g) * scale).to(dtype)


def _compare(fsi, dev, s, **kw):
    route = fsi.select_blocks(s.to(dev), **kw)
    ora = R.select_route(s, **kw)
    _, remote = R.route_masks(s.shape[1], s.shape[2], kw.get("causal", True), kw.get("local_window_blocks", 0))[1:]
    rtol, ctol = tolerances(s.dtype)
    bad = check_rows(route.remote_indices, route.remote_counts, ora, remote, rtol, ctol)
    assert not bad, bad
    return route, ora


CASES = [
    # (B, Qb, Nb, causal, local, top_p, kmin, kmax, cap, scale)
    (2, 16, 16, True, 0, 0.9, 0, 4, 4, 3.0),
    (1, 40, 40, True, 4, 0.95, 2, 8, 8, 2.0),
    (2, 8, 65, False, 0, 0.9, 4, 64, 64, 4.0),
    (1, 4, 300, False, 8, 0.7, 0, 16, 32, 1.0),
    (1, 3, 1024, False, 0, 0.99, 1, 200, 256, 0.5),
    (2, 6, 4096, False, 0, 0.9, 4, 64, 64, 6.0),
    (1, 5, 3, False, 0, 0.9, 0, 3, 6, 1.0),     # capacity beyond the number of blocks
    (1, 70, 70, True, 2, 0.5, 0, 16, 16, 8.0),  # sharp rows, causal + local
    (3, 1, 7, False, 2, 1.0, 0, 7, 7, 1.0),     # top_p = 1
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_select_blocks_parity(fsi, dev, case, dtype):
    B, Qb, Nb, causal, lw, p, kmin, kmax, cap, scale = case
    print(f"[case] select_blocks {case} {dtype}", flush=True)
    s = _scores(B, Qb, Nb, seed=Nb + Qb, scale=scale, dtype=dtype)
    route, ora = _compare(fsi, dev, s, causal=causal, local_window_blocks=lw, top_p=p, min_remote_blocks=kmin,
                          max_remote_blocks=kmax, remote_capacity=cap)
    if lw > 0:
        assert torch.equal(route.base_indices.cpu(), ora["base_indices"])
        assert torch.equal(route.base_counts.cpu(), ora["base_counts"])
    else:
        assert route.base_indices is None and route.base_counts is None


def test_select_blocks_reference_known_answer(fsi, dev):
    """tests/test_indexer.py:20-40 of the reference, on the GPU."""
    scores = torch.tensor([[[0.0, 0.0, 0.0, 0.0],
                            [10.0, 0.0, 0.0, 0.0],
                            [0.0, 10.0, 0.0, 0.0],
                            [0.0, 0.0, 10.0, 0.0]]])
    route = fsi.select_blocks(scores.to(dev), causal=True, local_window_blocks=0, top_p=0.9,
                              min_remote_blocks=0, max_remote_blocks=2, remote_capacity=2)
    assert route.remote_counts.cpu().tolist() == [[0, 1, 1, 1]]
    assert route.remote_indices.cpu()[0, 1, 0].item() == 0
    assert route.remote_indices.cpu()[0, 2, 0].item() == 1
    assert route.remote_indices.cpu()[0, 3, 0].item() == 2
    assert route.base_indices is None


def test_select_blocks_exact_ties_rank_by_index(fsi, dev):
    s = torch.zeros(1, 2, 10)
    route = fsi.select_blocks(s.to(dev), causal=False, top_p=0.35, max_remote_blocks=10, remote_capacity=10)
    assert route.remote_indices.cpu()[0, 0].tolist() == list(range(10))
    assert route.remote_counts.cpu().tolist() == [[4, 4]]  # cum 0.1,0.2,0.3 < 0.35 -> 3 + 1


def test_select_blocks_per_row_parameters(fsi, dev):
    print("[case] per-row top_p / K_min / K_max", flush=True)
    B, Qb, Nb = 2, 5, 50
    s = _scores(B, Qb, Nb, seed=9)
    g = torch.Generator().manual_seed(1)
    p = torch.rand(B, Qb, generator=g) * 0.8 + 0.1
    kmin = torch.randint(0, 3, (Qb,), generator=g)
    kmax = torch.randint(3, 12, (B, 1), generator=g)
    _compare(fsi, dev, s, causal=False, top_p=p, min_remote_blocks=kmin, max_remote_blocks=kmax, remote_capacity=12)


def test_select_blocks_stats_and_empty_rows(fsi, dev):
    s = _scores(2, 9, 9, seed=4)
    route, ora = _compare(fsi, dev, s, causal=True, local_window_blocks=0, top_p=0.9, min_remote_blocks=1,
                          max_remote_blocks=3, remote_capacity=3)
    assert route.remote_counts.cpu()[:, 0].tolist() == [0, 0]  # query block 0 has no complete block
    for key in ("cap_rate", "mean_remote_blocks", "base_only_rate"):
        assert abs(float(getattr(route, key)) - float(ora[key])) < 1e-6, key
    assert route.block_scores is not None


LARGE_CASES = [
    # rows longer than one wave holds (> 4096 blocks): one 16-wave workgroup per row
    # (B, Qb, Nb, causal, local, top_p, kmin, kmax, cap, scale)
    (1, 3, 8192, False, 0, 0.9, 4, 64, 64, 6.0),        # 8 slots per lane per wave
    (1, 2, 16384, False, 16, 0.95, 2, 200, 256, 4.0),   # 16 slots, local window, 256 ranked
    (1, 2, 40000, False, 0, 0.8, 0, 32, 32, 8.0),       # 64 slots, ragged last wave
    (1, 4200, 4200, True, 8, 0.9, 1, 16, 16, 6.0),      # causal: early rows have fewer candidates than capacity
]


@pytest.mark.parametrize("case", LARGE_CASES, ids=[f"L{i}" for i in range(len(LARGE_CASES))])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_select_blocks_large_rows(fsi, dev, case, dtype):
    B, Qb, Nb, causal, lw, p, kmin, kmax, cap, scale = case
    print(f"[case] select_blocks large {case} {dtype}", flush=True)
    s = _scores(B, Qb, Nb, seed=Nb + 7, scale=scale, dtype=dtype)
    route, ora = _compare(fsi, dev, s, causal=causal, local_window_blocks=lw, top_p=p, min_remote_blocks=kmin,
                          max_remote_blocks=kmax, remote_capacity=cap)
    same = route.remote_counts.cpu() == ora["remote_counts"]
    assert int(same.sum()) >= same.numel() - max(2, same.numel() // 500)


def test_select_blocks_capacity_limits(fsi, dev):
    s = torch.zeros(1, 1, 70000, device=dev)
    with pytest.raises(RuntimeError, match="blocks per row"):
        fsi.select_blocks(s, causal=False)
    s = torch.zeros(1, 1, 1000, device=dev)
    with pytest.raises(RuntimeError, match="ranked"):
        fsi.select_blocks(s, causal=False, max_remote_blocks=300, remote_capacity=300)


def test_masked_softmax_parity(fsi, dev):
    g = torch.Generator().manual_seed(2)
    s = torch.randn(3, 7, 300, generator=g) * 4
    mask = torch.rand(7, 300, generator=g) > 0.3
    mask[2] = False  # all-masked row -> zeros
    got = fsi.masked_softmax(s.to(dev), mask.to(dev)).cpu()
    ref = R.masked_probs(s, mask[None].expand(3, -1, -1))
    assert torch.all(got[:, 2] == 0)
    assert torch.allclose(got, ref, rtol=1e-6, atol=1e-12)
    sb = s.bfloat16()
    gotb = fsi.masked_softmax(sb.to(dev), mask.to(dev)).cpu()
    refb = R.masked_probs(sb, mask[None].expand(3, -1, -1))
    assert gotb.dtype == torch.bfloat16
    ulp = (gotb.float() - refb.float()).abs() / refb.float().abs().clamp_min(1e-30)
    assert float(ulp.max()) <= 2.0 ** -8 + 1e-9


def _c2_inputs(Q, N, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    keys = torch.nn.functional.normalize(torch.randn(N, 16, generator=g), dim=-1)
    j = torch.stack([torch.randperm(N, generator=g)[:4] for _ in range(Q)])
    w = torch.distributions.Dirichlet(torch.full((4,), 0.3)).sample((Q,))
    q = (w[..., None] * keys[j]).sum(1) + 0.1 * torch.randn(Q, 16, generator=g)
    return q.to(dtype), keys.to(dtype)


@pytest.mark.parametrize("Q,N,kmin,kmax,cap", [(64, 256, 4, 64, 64), (300, 4096, 4, 64, 64), (40, 1000, 0, 16, 32),
                                               (17, 4096, 2, 100, 128)])
def test_score_and_route_parity(fsi, dev, Q, N, kmin, kmax, cap):
    print(f"[case] score_and_route Q={Q} N={N}", flush=True)
    torch.manual_seed(0)
    q, k = _c2_inputs(Q, N, seed=Q + N)
    idx, cnt, mass = fsi.score_and_route(q.to(dev), k.to(dev), causal=False, top_p=0.9, min_remote_blocks=kmin,
                                         max_remote_blocks=kmax, remote_capacity=cap, return_mass=True)
    s = R.cosine_scores_f32(q[None], k[None])
    ora = R.select_route(s, causal=False, top_p=0.9, min_remote_blocks=kmin, max_remote_blocks=kmax,
                         remote_capacity=cap)
    remote = torch.ones(Q, N, dtype=torch.bool)
    bad = check_rows(idx, cnt, ora, remote, 1e-6, 1e-5)
    assert not bad, bad
    # mass = cumulative mass of the selected blocks
    oc = ora["remote_counts"][0].long()
    cm = ora["cumulative"][0]
    ref_mass = torch.where(oc > 0, cm.gather(1, (oc - 1).clamp_min(0)[:, None])[:, 0], torch.zeros(Q))
    same = cnt.cpu()[0].long() == oc
    assert torch.allclose(mass.cpu()[0][same], ref_mass[same], atol=2e-6)


def test_score_and_route_batched_and_causal(fsi, dev):
    g = torch.Generator().manual_seed(7)
    q = torch.randn(2, 50, 16, generator=g)
    k = torch.randn(2, 50, 16, generator=g)
    idx, cnt = fsi.score_and_route(q.to(dev), k.to(dev), causal=True, local_window_blocks=3, top_p=0.8,
                                   min_remote_blocks=1, max_remote_blocks=6, remote_capacity=8)
    s = R.cosine_scores_f32(q, k)
    ora = R.select_route(s, causal=True, local_window_blocks=3, top_p=0.8, min_remote_blocks=1, max_remote_blocks=6,
                         remote_capacity=8)
    _, _, remote = R.route_masks(50, 50, True, 3)
    bad = check_rows(idx, cnt, ora, remote, 1e-6, 1e-5)
    assert not bad, bad


@pytest.mark.parametrize("Q,N,kmin,kmax,cap", [(20, 8192, 4, 64, 64), (6, 16384, 2, 100, 128), (3, 65536, 0, 16, 16)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_score_and_route_large_rows(fsi, dev, Q, N, kmin, kmax, cap, dtype):
    print(f"[case] score_and_route large Q={Q} N={N} {dtype}", flush=True)
    q, k = _c2_inputs(Q, N, seed=N + Q, dtype=dtype)
    idx, cnt, mass = fsi.score_and_route(q.to(dev), k.to(dev), causal=False, top_p=0.9, min_remote_blocks=kmin,
                                         max_remote_blocks=kmax, remote_capacity=cap, return_mass=True)
    s = R.cosine_scores_f32(q[None], k[None])
    ora = R.select_route(s, causal=False, top_p=0.9, min_remote_blocks=kmin, max_remote_blocks=kmax,
                         remote_capacity=cap)
    bad = check_rows(idx, cnt, ora, torch.ones(Q, N, dtype=torch.bool), 1e-6, 1e-5)
    assert not bad, bad
    oc = ora["remote_counts"][0].long()
    cm = ora["cumulative"][0]
    ref_mass = torch.where(oc > 0, cm.gather(1, (oc - 1).clamp_min(0)[:, None])[:, 0], torch.zeros(Q))
    same = cnt.cpu()[0].long() == oc
    assert torch.allclose(mass.cpu()[0][same], ref_mass[same], atol=2e-6)


def _decode_inputs(B, P, seed):
    g = torch.Generator().manual_seed(seed)
    kp = torch.nn.functional.normalize(torch.randn(B, P, 16, generator=g), dim=-1)
    vp = torch.randn(B, P, 16, generator=g).bfloat16()
    qi = torch.nn.functional.rms_norm(torch.randn(B, 16, generator=g), (16,)).bfloat16()
    return qi, kp, vp


@pytest.mark.parametrize("B,P,page,W,pos,kmin,kmax,top_p", [
    (4, 40, 8, 64, 8 * 30 + 3, 1, 5, 0.6),
    (32, 2048, 64, 1024, 131071, 0, 32, 0.9),
    (3, 100, 16, 32, 16 * 100 - 1, 2, 64, 0.95),
    (2, 10, 64, 1024, 500, 0, 8, 0.9),         # no remote pages yet
    (3, 5000, 64, 1024, 64 * 5000 - 1, 0, 32, 0.9),     # more pages than one wave holds: 16-wave workgroup
    (2, 16384, 64, 2048, 64 * 16384 - 1, 4, 64, 0.95),  # 1 M tokens of context
    (2, 40000, 16, 256, 16 * 40000 - 7, 0, 256, 0.99),  # 64 slots per lane, 256 ranked
])
def test_decode_route_parity(fsi, dev, B, P, page, W, pos, kmin, kmax, top_p):
    print(f"[case] decode_route B={B} P={P} pos={pos}", flush=True)
    qi, kp, vp = _decode_inputs(B, P, seed=P)
    completed = min(P, (pos + 1) // page)
    pages, counts, ctx = fsi.decode_route(qi.to(dev), kp.to(dev), vp.to(dev), pos=pos, page_size=page,
                                          local_window=W, completed_pages=completed, top_p=top_p,
                                          min_remote_blocks=kmin, max_remote_blocks=kmax, return_context=True)
    ora = R.decode_route(qi.float()[:, None], kp, pos, page, W, completed, top_p, kmin, kmax)
    pages, counts = pages.cpu(), counts.cpu()
    for b in range(B):
        ref = ora["pages"][b]
        got = pages[b, :int(counts[b])].tolist()
        assert all(x == -1 for x in pages[b, int(counts[b]):].tolist())
        if got == ref:
            continue
        probs = ora["probs"][b]
        assert len(got) == len(ref) or abs(float(ora["cumulative"][b, min(len(got), len(ref)) - 1]) - top_p) < 1e-5
        n = min(len(got), len(ref))
        assert torch.allclose(probs[got[:n]], probs[ref[:n]], rtol=1e-6, atol=0), (b, got, ref)
    # additive-stream context: softmax over all completed pages, probabilities in bf16
    if completed > 0:
        qn = torch.nn.functional.normalize(qi.float(), dim=-1)
        sc = torch.einsum("bd,bpd->bp", qn, kp[:, :completed]) / 4.0
        pr = torch.softmax(sc, -1).bfloat16().float()
        ref_ctx = torch.einsum("bp,bpd->bd", pr, vp[:, :completed].float())
        err = (ctx.cpu().float() - ref_ctx).norm() / ref_ctx.norm()
        assert float(err) <= 2e-3
    else:
        assert torch.all(ctx.cpu() == 0)
