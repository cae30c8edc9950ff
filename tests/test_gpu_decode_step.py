"""The one-launch decode step: fsi_decode_step_attn with at least one (sequence, KV
head) pair per compute unit (256 on MI355X) and at most 2048 complete pages runs
decode_step_fused_kernel, where four waves of each pair's workgroup route the
sequence while four stream the local window.  The pages, counts and context must
equal the separate decode_route call exactly (the same routing code); the
attention is checked against fp64 softmax attention over the routed pages
(rel-L2 <= 2e-3, the bf16 bar) for a few sequences, whose K / V are read back
from the pool."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle import pattention as Pt

pytestmark = pytest.mark.gpu

TOL = 2e-3

CASES = [
    # B, Hq, Hkv, hd, max_seq, pos ("per-seq" = one position per sequence), window, K_min, K_max, top_p, context
    (32, 32, 8, 64, 4096, 4000, 512, 0, 8, 0.9, True),          # head_dim 64, 64 pages (4 slots per lane)
    (32, 8, 8, 64, 9600, "per-seq", 128, 2, 70, 0.95, True),    # K_max > 64 (4 sort slots), per-sequence positions
    (32, 32, 8, 128, 2048, 2047, 1024, 0, 32, 0.9, False),     # window over half the context, no context output
    (64, 16, 4, 128, 3072, 3000, 256, 1, 16, 0.8, True),        # 64 sequences x 4 KV heads, GQA group 4
    (256, 4, 1, 64, 44800, 44799, 1024, 0, 12, 0.9, True),      # 700 pages (16 slots per lane), one KV head
    (32, 32, 8, 128, 4096, "mixed", 1024, 0, 16, 0.9, True),    # some sequences inside their window: no pages
]


def _device_cache(fsi, dev, B, Hkv, hd, max_seq, seed):
    P = -(-max_seq // 64)
    g = torch.Generator(device=dev).manual_seed(seed)
    n_phys = B * P + 5
    table = torch.randperm(n_phys, device=dev, generator=g)[:B * P].view(B, P).to(torch.int32)
    c = fsi.FovealKVCache(B, max_seq, Hkv, hd, 16, 64, dev, torch.bfloat16, n_phys_pages=n_phys, page_table=table)
    c.k_cache.normal_(generator=g)
    c.v_cache.normal_(generator=g)
    c.kp_cache.copy_(F.normalize(torch.randn(B, P, 16, device=dev, generator=g), dim=-1))
    c.vp_cache.normal_(generator=g)
    c.seq_len, c.completed_pages = max_seq, P
    return c, g


@pytest.mark.parametrize("case", CASES, ids=[f"s{i}" for i in range(len(CASES))])
def test_decode_step_one_launch(fsi, dev, case):
    B, Hq, Hkv, hd, max_seq, pos, W, kmin, kmax, top_p, want_ctx = case
    print(f"[case] one-launch decode step {case}", flush=True)
    assert B * Hkv >= torch.cuda.get_device_properties(dev).multi_processor_count, "case must take the one-launch path"
    c, g = _device_cache(fsi, dev, B, Hkv, hd, max_seq, seed=B + hd + Hkv)
    if pos in ("per-seq", "mixed"):
        if pos == "per-seq":
            pos_list = [max_seq - 1 - (37 * b) % 1500 for b in range(B)]
        else:  # positions 0 .. max_seq - 1: the first sequences have no page before their window
            pos_list = [(b * 131) % max_seq for b in range(B)]
        pos_arg = torch.tensor(pos_list, dtype=torch.int32, device=dev)
    else:
        pos_list = [pos] * B
        pos_arg = pos
    completed = (max(pos_list) + 1) // 64
    q = torch.randn(B, Hq, hd, device=dev, generator=g).bfloat16()
    qi = F.rms_norm(torch.randn(B, 16, device=dev, generator=g), (16,)).bfloat16()
    scale = 1.0 / math.sqrt(hd)
    kw = dict(pos=pos_arg, window=W, completed_pages=completed, top_p=top_p, min_remote_blocks=kmin,
              max_remote_blocks=kmax)
    with torch.no_grad():
        res = fsi.decode_step_attention(q, qi, c, scale=scale, return_context=want_ctx, **kw)
        out, pages, counts = res[:3]
        ref = fsi.decode_route(qi, c.kp_cache, c.vp_cache, page_size=64, local_window=W,
                               completed_pages=completed, top_p=top_p, min_remote_blocks=kmin,
                               max_remote_blocks=kmax, pos=pos_arg, return_context=want_ctx)
    assert torch.equal(pages, ref[0]) and torch.equal(counts, ref[1])
    if want_ctx:
        assert torch.equal(res[3], ref[2])
    cnt = counts.cpu().tolist()
    assert max(cnt) > 0
    if pos == "mixed":
        assert min(cnt) == 0  # the case covers sequences with nothing to route
    for b in sorted({0, 1, B // 2, B - 1}):
        kk, vv = c.to_dense(max_seq, batch=slice(b, b + 1))
        sel = [pages[b, :cnt[b]].cpu().tolist()]
        want = A.decode_attention_f64(q[b:b + 1].cpu().float(), kk.cpu(), vv.cpu(), [pos_list[b]], W, sel, 64, scale)
        err = Pt.rel_l2(out[b:b + 1].cpu().float(), want.float())
        assert err <= TOL, (b, err)


def test_decode_step_one_launch_graph_replays(fsi, dev):
    """The one-launch step captured in a graph, replayed three times with eager work
    in between: every replay equals the eager result bit for bit."""
    B, Hq, Hkv, hd, max_seq, W = 32, 32, 8, 128, 4096, 1024
    c, g = _device_cache(fsi, dev, B, Hkv, hd, max_seq, seed=5)
    q = torch.randn(B, Hq, hd, device=dev, generator=g).bfloat16()
    qi = F.rms_norm(torch.randn(B, 16, device=dev, generator=g), (16,)).bfloat16()

    def step():
        return fsi.decode_step_attention(q, qi, c, pos=max_seq - 1, window=W, completed_pages=max_seq // 64,
                                         top_p=0.9, min_remote_blocks=0, max_remote_blocks=32, scale=0.09,
                                         return_context=True)

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


def test_decode_step_one_launch_invalid_page_reported(fsi, dev, monkeypatch):
    """A selected page whose page-table entry is outside the pool is skipped and
    reported (IndexError under FSI_CHECK=1), as in the split path."""
    B, Hq, Hkv, hd, max_seq = 32, 8, 8, 64, 2048
    c, g = _device_cache(fsi, dev, B, Hkv, hd, max_seq, seed=9)
    q = torch.randn(B, Hq, hd, device=dev, generator=g).bfloat16()
    qi = F.rms_norm(torch.randn(B, 16, device=dev, generator=g), (16,)).bfloat16()
    # page 3 of sequence 5 gets sequence 5's own query as its key (certain to be selected)
    # and a page-table entry beyond the pool
    c.kp_cache[5, 3] = F.normalize(qi[5].float(), dim=-1)
    c.page_table[5, 3] = c.n_phys_pages + 7
    monkeypatch.setenv("FSI_CHECK", "1")
    with pytest.raises(IndexError):
        fsi.decode_step_attention(q, qi, c, pos=max_seq - 1, window=256, completed_pages=max_seq // 64, top_p=0.9,
                                  min_remote_blocks=0, max_remote_blocks=8, scale=0.125)
