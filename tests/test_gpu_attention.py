"""GPU parity of the paged KV cache and foveal decode attention.

KV pool writes/reads are bit-exact.  Attention outputs: bf16 rel-L2 <= 2e-3
against fp64 textbook attention over the same support (probabilities are
rounded to bf16 before the PV product, as flash-style kernels do)."""
import copy
import math

import pytest
import torch

from oracle import attention as A
from oracle import pattention as Pt

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _cache(fsi, dev, B, Hkv, hd, max_seq, seed, n_phys=None):
    g = torch.Generator().manual_seed(seed)
    P = -(-max_seq // 64)
    n_phys = n_phys or B * P + 3
    table = torch.randperm(n_phys, generator=g)[:B * P].view(B, P).to(torch.int32)
    c = fsi.FovealKVCache(B, max_seq, Hkv, hd, 16, 64, dev, torch.bfloat16, n_phys_pages=n_phys, page_table=table)
    k = torch.randn(B, Hkv, max_seq, hd, generator=g).bfloat16()
    v = torch.randn(B, Hkv, max_seq, hd, generator=g).bfloat16()
    c.load_dense(k.to(dev), v.to(dev))
    return c, k, v


@pytest.mark.parametrize("hd", [64, 128])
def test_kv_pool_round_trip(fsi, dev, hd):
    print(f"[case] kv round trip hd={hd}", flush=True)
    c, k, v = _cache(fsi, dev, 3, 2, hd, 300, seed=hd)
    kk, vv = c.to_dense(300)
    assert torch.equal(kk.cpu(), k) and torch.equal(vv.cpu(), v)
    # a strided (non-contiguous) source and an offset start
    k2 = torch.randn(3, 2, 5, hd).bfloat16()
    v2 = torch.randn(3, 5, 2, hd).bfloat16().transpose(1, 2)
    c.load_dense(k2.to(dev), v2.to(dev), start=100)
    kk, vv = c.to_dense(300)
    assert torch.equal(kk.cpu()[:, :, 100:105], k2) and torch.equal(vv.cpu()[:, :, 100:105], v2)
    assert torch.equal(kk.cpu()[:, :, :100], k[:, :, :100])


CASES = [
    # B, Hq, Hkv, hd, max_seq, pos, window, pages per seq
    (2, 8, 2, 128, 1024, 700, 100, [[0, 5, 3], [2]]),
    (3, 4, 4, 64, 512, 511, 64, [[1], [0, 2, 4], []]),
    (1, 16, 1, 128, 640, 33, 1024, [[]]),
    (2, 32, 8, 128, 4096, 4000, 1024, [[0, 10, 20, 30, 40, 44], [7]]),
    (2, 8, 1, 64, 2048, 1500, 77, [[3, 1, 22], [0]]),
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_decode_attention_parity(fsi, dev, case):
    B, Hq, Hkv, hd, max_seq, pos, W, pages = case
    print(f"[case] decode_attention {case[:7]}", flush=True)
    c, k, v = _cache(fsi, dev, B, Hkv, hd, max_seq, seed=B * 100 + Hq)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, Hq, hd, generator=g).bfloat16()
    cap = max(1, max(len(p) for p in pages))
    rp = torch.full((B, cap), -1, dtype=torch.int32)
    for b, p in enumerate(pages):
        rp[b, :len(p)] = torch.tensor(p, dtype=torch.int32)
    cnt = torch.tensor([len(p) for p in pages], dtype=torch.int32)
    scale = 1.0 / math.sqrt(hd)
    out = fsi.decode_attention(q.to(dev), c, pos=pos, window=W, remote_pages=rp.to(dev), remote_counts=cnt.to(dev),
                               scale=scale).cpu()
    ref = A.decode_attention_f64(q.float(), k, v, pos, W, pages, 64, scale)
    assert Pt.rel_l2(out.float(), ref.float()) <= TOL


FUSED_CASES = [
    # B, Hq, Hkv, hd, max_seq, pos (int or per-sequence), window, K_min, K_max, top_p
    (2, 8, 2, 128, 1024, 900, 128, 0, 3, 0.8),
    (3, 16, 4, 64, 4096, [4000, 3000, 2500], 512, 1, 6, 0.9),
    (4, 32, 8, 128, 8192, 8191, 1024, 0, 32, 0.9),
    (1, 8, 8, 64, 2048, 2047, 64, 2, 70, 0.95),  # more than 64 candidates: 4 sort slots per lane
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=[f"f{i}" for i in range(len(FUSED_CASES))])
@pytest.mark.parametrize("batch0", [False, True])
def test_decode_step_attention_fused(fsi, dev, case, batch0):
    """fsi_decode_step_attn: routing workgroups beside the local-window partials,
    then the selected pages and the merge.  Pages, counts and context equal the
    separate decode_route call exactly (same routing code); the attention is
    checked against the fp64 oracle over the routed pages."""
    B, Hq, Hkv, hd, max_seq, pos, W, kmin, kmax, top_p = case
    print(f"[case] fused decode step {case} batch0={batch0}", flush=True)
    c, k, v = _cache(fsi, dev, B, Hkv, hd, max_seq, seed=B * 7 + hd)
    g = torch.Generator().manual_seed(9)
    q = torch.randn(B, Hq, hd, generator=g).bfloat16().to(dev)
    qi = torch.nn.functional.rms_norm(torch.randn(B, 16, generator=g), (16,)).bfloat16().to(dev)
    c.kp_cache.copy_(torch.nn.functional.normalize(torch.randn(B, c.max_pages, 16, generator=g), dim=-1).to(dev))
    c.vp_cache.copy_(torch.randn(B, c.max_pages, 16, generator=g).bfloat16().to(dev))
    pos_arg = torch.tensor(pos, dtype=torch.int32, device=dev) if isinstance(pos, list) else pos
    pos_max = max(pos) if isinstance(pos, list) else pos
    completed = (pos_max + 1) // 64
    scale = 1.0 / math.sqrt(hd)
    with torch.no_grad():
        out, pages, counts, ctx = fsi.decode_step_attention(
            q, qi, c, pos=pos_arg, window=W, completed_pages=completed, top_p=top_p, min_remote_blocks=kmin,
            max_remote_blocks=kmax, scale=scale, return_context=True, batch0=batch0)
        rp, rc, rctx = fsi.decode_route(qi, c.kp_cache, c.vp_cache, pos=pos_arg, page_size=64, local_window=W,
                                        completed_pages=completed, top_p=top_p, min_remote_blocks=kmin,
                                        max_remote_blocks=kmax, return_context=True)
    assert torch.equal(pages, rp) and torch.equal(counts, rc) and torch.equal(ctx, rctx)
    cnt = counts.cpu().tolist()
    sel = [pages[b, :cnt[b]].cpu().tolist() for b in range(B)]
    att = [sel[0]] * B if batch0 else sel
    ref = A.decode_attention_f64(q.cpu().float(), k, v, pos, W, att, 64, scale)
    assert Pt.rel_l2(out.cpu().float(), ref.float()) <= TOL


def test_decode_step_attention_wide_batch_long_window(fsi, dev):
    """Many (sequence, KV head) pairs and a window of 8192 tokens (257 chunks): the
    occupancy-sized local launch gets only a few waves per pair, and each of them
    may take at most 64 chunks, so the split must never fall below
    ceil(chunks / 64).  The fused step must equal the separate route + attention."""
    B, Hq, Hkv, hd, W, kmax = 128, 8, 8, 64, 8192, 8
    max_seq = W + 64
    pos = max_seq - 1
    print(f"[case] fused decode step wide batch B={B} Hkv={Hkv} W={W}", flush=True)
    c, k, v = _cache(fsi, dev, B, Hkv, hd, max_seq, seed=77)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, Hq, hd, generator=g).bfloat16().to(dev)
    qi = torch.nn.functional.rms_norm(torch.randn(B, 16, generator=g), (16,)).bfloat16().to(dev)
    c.kp_cache.copy_(torch.nn.functional.normalize(torch.randn(B, c.max_pages, 16, generator=g), dim=-1).to(dev))
    completed = (pos + 1) // 64
    scale = 1.0 / math.sqrt(hd)
    with torch.no_grad():
        out, pages, counts = fsi.decode_step_attention(q, qi, c, pos=pos, window=W, completed_pages=completed,
                                                       top_p=0.9, min_remote_blocks=0, max_remote_blocks=kmax,
                                                       scale=scale)
        split = fsi.decode_attention(q, c, pos=pos, window=W, remote_pages=pages, remote_counts=counts, scale=scale)
    assert Pt.rel_l2(out.float(), split.float()) <= TOL
    cnt = counts.cpu().tolist()
    sel = [pages[b, :cnt[b]].cpu().tolist() for b in range(0, B, 16)]
    ref = A.decode_attention_f64(q[::16].cpu().float(), k[::16], v[::16], pos, W, sel, 64, scale)
    assert Pt.rel_l2(out[::16].cpu().float(), ref.float()) <= TOL


@pytest.mark.parametrize("batch0", [False, True])
def test_decode_step_attention_many_pages(fsi, dev, batch0):
    """More complete pages (5000, 320 K tokens) than the fused launch's routing
    workgroups hold: the step runs the 16-wave routing kernel, then the window
    and the selected pages.  Pages equal the separate decode_route; attention
    against fp64 over the routed pages."""
    B, Hq, Hkv, hd, W, kmax = 2, 8, 2, 64, 1024, 32
    max_seq = 64 * 5000
    pos = max_seq - 1
    print(f"[case] fused decode step, 5000 pages, batch0={batch0}", flush=True)
    c, k, v = _cache(fsi, dev, B, Hkv, hd, max_seq, seed=91)
    g = torch.Generator().manual_seed(6)
    q = torch.randn(B, Hq, hd, generator=g).bfloat16().to(dev)
    qi = torch.nn.functional.rms_norm(torch.randn(B, 16, generator=g), (16,)).bfloat16().to(dev)
    c.kp_cache.copy_(torch.nn.functional.normalize(torch.randn(B, c.max_pages, 16, generator=g), dim=-1).to(dev))
    c.vp_cache.copy_(torch.randn(B, c.max_pages, 16, generator=g).bfloat16().to(dev))
    completed = (pos + 1) // 64
    scale = 1.0 / math.sqrt(hd)
    with torch.no_grad():
        out, pages, counts, ctx = fsi.decode_step_attention(
            q, qi, c, pos=pos, window=W, completed_pages=completed, top_p=0.9, min_remote_blocks=0,
            max_remote_blocks=kmax, scale=scale, return_context=True, batch0=batch0)
        rp, rc, rctx = fsi.decode_route(qi, c.kp_cache, c.vp_cache, pos=pos, page_size=64, local_window=W,
                                        completed_pages=completed, top_p=0.9, min_remote_blocks=0,
                                        max_remote_blocks=kmax, return_context=True)
    assert torch.equal(pages, rp) and torch.equal(counts, rc) and torch.equal(ctx, rctx)
    cnt = counts.cpu().tolist()
    assert min(cnt) > 0
    sel = [pages[b, :cnt[b]].cpu().tolist() for b in range(B)]
    att = [sel[0]] * B if batch0 else sel
    ref = A.decode_attention_f64(q.cpu().float(), k, v, pos, W, att, 64, scale)
    assert Pt.rel_l2(out.cpu().float(), ref.float()) <= TOL


def test_decode_step_attention_graph_replays(fsi, dev):
    """The fused step captured in a graph and replayed with eager work in between:
    every replay equals the eager result."""
    B, Hq, Hkv, hd, max_seq, pos, W, kmin, kmax, top_p = FUSED_CASES[2]
    c, k, v = _cache(fsi, dev, B, Hkv, hd, max_seq, seed=21)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B, Hq, hd, generator=g).bfloat16().to(dev)
    qi = torch.nn.functional.rms_norm(torch.randn(B, 16, generator=g), (16,)).bfloat16().to(dev)
    c.kp_cache.copy_(torch.nn.functional.normalize(torch.randn(B, c.max_pages, 16, generator=g), dim=-1).to(dev))

    def step():
        return fsi.decode_step_attention(q, qi, c, pos=pos, window=W, completed_pages=(pos + 1) // 64, top_p=top_p,
                                         min_remote_blocks=kmin, max_remote_blocks=kmax, scale=0.08)

    with torch.no_grad():
        eager = step()
        outs = {}
        graph = torch.cuda.CUDAGraph()
        st = torch.cuda.Stream(dev)
        st.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(st), torch.cuda.graph(graph, stream=st):
            outs["r"] = step()
        torch.cuda.synchronize(dev)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize(dev)
            for a, b in zip(outs["r"], eager):
                assert torch.equal(a, b)
            torch.randn(1024, 1024, device=dev).sum().item()  # eager work between replays


def test_decode_attention_per_sequence_positions(fsi, dev):
    B, Hq, Hkv, hd = 4, 8, 2, 128
    c, k, v = _cache(fsi, dev, B, Hkv, hd, 1024, seed=7)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(B, Hq, hd, generator=g).bfloat16()
    pos = [1023, 64, 500, 0]
    pages = [[1, 2], [], [0, 3], []]
    rp = torch.tensor([[1, 2], [-1, -1], [0, 3], [-1, -1]], dtype=torch.int32)
    cnt = torch.tensor([2, 0, 2, 0], dtype=torch.int32)
    out = fsi.decode_attention(q.to(dev), c, pos=torch.tensor(pos).to(dev), window=128, remote_pages=rp.to(dev),
                               remote_counts=cnt.to(dev), scale=0.1).cpu()
    ref = A.decode_attention_f64(q.float(), k, v, pos, 128, pages, 64, 0.1)
    assert Pt.rel_l2(out.float(), ref.float()) <= TOL


@pytest.mark.parametrize("layout", ["paged_bf16", "dense_f32", "dense_bf16_page16"])
def test_decode_attention_query_gradient(fsi, dev, layout):
    """dq of decode_attention on the device (fsi_decode_attn_bwd_q) against fp64
    autograd of softmax attention over the same support (window tokens then the
    selected pages), per-sequence positions, one sequence without pages: fp32
    rel-L2 2e-5, bf16 1e-2."""
    B, Hq, Hkv, hd, S = 3, 8, 2, 64, 512
    dtype = torch.float32 if layout == "dense_f32" else torch.bfloat16
    page = 16 if layout.endswith("page16") else 64
    g = torch.Generator().manual_seed(31)
    k = torch.randn(B, Hkv, S, hd, generator=g).to(dtype)
    v = torch.randn(B, Hkv, S, hd, generator=g).to(dtype)
    if layout == "paged_bf16":
        n_phys = B * (S // 64) + 2
        table = torch.randperm(n_phys, generator=g)[:B * (S // 64)].view(B, S // 64).to(torch.int32)
        c = fsi.FovealKVCache(B, S, Hkv, hd, 16, 64, dev, dtype, n_phys_pages=n_phys, page_table=table)
    else:
        c = fsi.FovealKVCache(B, S, Hkv, hd, 16, page, dev, dtype, paged=False)
    assert c.paged == (layout == "paged_bf16")
    c.load_dense(k.to(dev), v.to(dev))
    q = torch.randn(B, Hq, hd, generator=g).to(dtype)
    dout = torch.randn(B, Hq, hd, generator=g).to(dtype)
    pos = [S - 1, 300, 40]
    pages = [[0, 2], [1], []]
    cap = 2
    rp = torch.full((B, cap), -1, dtype=torch.int32)
    for b, p in enumerate(pages):
        rp[b, :len(p)] = torch.tensor(p, dtype=torch.int32)
    cnt = torch.tensor([len(p) for p in pages], dtype=torch.int32)
    W, scale = 100, hd ** -0.5
    qd = q.to(dev).requires_grad_()
    out = fsi.decode_attention(qd, c, pos=torch.tensor(pos).to(dev), window=W, remote_pages=rp.to(dev),
                               remote_counts=cnt.to(dev), scale=scale)
    out.backward(dout.to(dev))
    q64 = q.double().requires_grad_()
    ref = A.decode_attention_f64(q64, k, v, pos, W, pages, page, scale)
    ref.backward(dout.double())
    tol = 2e-5 if dtype == torch.float32 else 1e-2
    assert qd.grad.dtype == dtype
    assert Pt.rel_l2(qd.grad.cpu().float(), q64.grad.float()) <= tol


def test_decode_attention_invalid_page_reported(fsi, dev, monkeypatch):
    c, k, v = _cache(fsi, dev, 1, 1, 64, 256, seed=3)
    q = torch.randn(1, 1, 64).bfloat16().to(dev)
    rp = torch.tensor([[9]], dtype=torch.int32, device=dev)  # beyond the 4-page table
    cnt = torch.tensor([1], dtype=torch.int32, device=dev)
    monkeypatch.setenv("FSI_CHECK", "1")
    with pytest.raises(IndexError):
        fsi.decode_attention(q, c, pos=200, window=64, remote_pages=rp, remote_counts=cnt, scale=0.125)


def test_decode_step_module(fsi, dev):
    """FovealSparseAttention.decode_step over several pages against the CPU
    restatement with the same weights: selected pages (near-tie tolerant) and
    the output of every step, over the pages the module selected (the same as
    the restatement's except at a near-tie).  The module output also passes
    through four bf16 library GEMMs (q/k/v/out projections) on each side, so
    its bar is rel-L2 1e-2."""
    torch.manual_seed(0)
    m = fsi.FovealSparseAttention(hidden_size=256, num_heads=8, num_kv_heads=2, head_dim=64, page_size=64,
                                  local_window_blocks=2, top_p=0.8, min_remote_pages=1, max_remote_pages=3,
                                  remote_capacity=3).to(torch.bfloat16)
    ora = A.DecodeStepOracle(copy.deepcopy(m), batch=2, max_seq_len=640)
    md = m.to(dev)
    cache = md.init_kv_cache(2, 640, dev)
    g = torch.Generator().manual_seed(4)
    xs = torch.randn(400, 2, 1, 256, generator=g).bfloat16()
    worst, differing = 0.0, 0
    with torch.no_grad():
        for t in range(400):
            out, aux = md.decode_step(xs[t].to(dev), cache)
            sel = aux["selected_remote_pages"]
            ref, pages, r = ora.step(xs[t], attend=sel)
            if sel != pages:
                # only a near-tie may reorder or resize the selection
                differing += 1
                for b in range(2):
                    got, exp = sel[b], pages[b]
                    if got != exp:
                        pr = r["probs"][b]
                        n = min(len(got), len(exp))
                        assert torch.allclose(pr[got[:n]], pr[exp[:n]], rtol=1e-5), (t, b, got, exp)
            worst = max(worst, Pt.rel_l2(out.cpu().float(), ref.float()))
    assert cache.completed_pages == 6 and cache.seq_len == 400
    assert differing <= 4, differing
    assert worst <= 1e-2, worst
