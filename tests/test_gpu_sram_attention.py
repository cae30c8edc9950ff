"""GPU parity of the fused indexer-attention kernel (fsi_sram_indexer_attention,
replacing triton_fused_sram_indexer_attention, triton_ops.py:142-249,373-435).

Selection: the kernel's picks equal oracle.attention.sram_select's (fp32) on
every row whose probabilities have no near-tie at a decision (gap, mass or the
1e-4 floor within 1e-5).  Output: against sram_attention_f64 over the kernel's
own picks, rel-L2 <= 1e-5 (fp32), 1e-3 (fp16), 4e-3 (bf16): the kernel rounds
the probabilities to the storage dtype before the PV product, as the reference
does, and rounds the output once."""
import math

import pytest
import torch

from oracle import attention as A

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 4e-3}


def _decided_rows(probs, top_p, R):
    """(B, M) bool: rows whose greedy decisions are far from every threshold."""
    srt = probs.double().sort(dim=-1, descending=True).values
    cum = torch.cat([torch.zeros_like(srt[..., :1]), srt.cumsum(-1)[..., :-1]], dim=-1)
    gaps = (srt[..., :-1] - srt[..., 1:]).abs()
    # the mass gate only decides picks that clear the 1e-4 floor
    mass_near = ((cum[..., :R] - top_p).abs() < 1e-5) & (srt[..., :R] > 1e-4 - 1e-5)
    near = (gaps[..., :R] < 1e-5).any(-1) | mass_near.any(-1) | ((srt[..., :R] - 1e-4).abs() < 1e-5).any(-1)
    return ~near


def _run(fsi, dev, B, H, N, D, bs, R, top_p, dtype, seed, idx_dtype=None, scale=None, peaked=False):
    g = torch.Generator().manual_seed(seed)
    M = N // bs
    q, k, v = (torch.randn(B, H, N, D, generator=g).to(dtype) for _ in range(3))
    q16 = torch.randn(B, M, 16, generator=g)
    k16 = torch.randn(B, M, 16, generator=g)
    if peaked:
        q16 = q16 * 3.0
    q16 = q16.to(idx_dtype or dtype)
    k16 = k16.to(idx_dtype or dtype)
    out, sel = fsi.sram_indexer_attention(q.to(dev), k.to(dev), v.to(dev), q16.to(dev), k16.to(dev), scale=scale,
                                          top_p=top_p, max_remote_blocks=R, block_size=bs, return_selection=True)
    picks, probs = A.sram_select(q16, k16, top_p, R)
    sel = sel.cpu().long()
    ok = _decided_rows(probs, top_p, R)
    assert torch.equal(sel[ok], picks[ok])
    assert ok.float().mean() > 0.7
    ref = A.sram_attention_f64(q, k, v, sel, bs, scale if scale is not None else 1.0 / math.sqrt(D))
    err = (out.cpu().double() - ref).norm() / ref.norm()
    assert out.dtype == dtype and out.shape == q.shape
    assert float(err) <= TOL[dtype], float(err)
    return out, sel


@pytest.mark.parametrize("B,N,M,bs", [(64, 64, 4, 16), (32, 256, 16, 16), (16, 1024, 32, 32)])
def test_reference_benchmark_configs_fp16(fsi, dev, B, N, M, bs):
    """The three configs of the reference's SRAM benchmark (benchmark_a10g_full.py:320-331):
    4 heads, head_dim 32, fp16, max_remote 2, default top_p 0.8."""
    print(f"[case] sram B={B} N={N} blocks={M} bs={bs} fp16", flush=True)
    assert N // bs == M
    _run(fsi, dev, B, 4, N, 32, bs, 2, 0.8, torch.float16, seed=N)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,N,D,bs,R,top_p", [
    (2, 3, 40, 24, 8, 3, 0.5),      # odd head_dim, block 8
    (1, 2, 192, 64, 64, 2, 0.9),    # largest block
    (3, 1, 160, 128, 16, 6, 0.95),  # more picks than blocks with mass
    (2, 2, 96, 16, 32, 8, 1.0),     # max_remote above the remote block count
])
def test_shapes_and_dtypes(fsi, dev, dtype, B, H, N, D, bs, R, top_p):
    print(f"[case] sram B={B} H={H} N={N} D={D} bs={bs} R={R} {dtype}", flush=True)
    _run(fsi, dev, B, H, N, D, bs, R, top_p, dtype, seed=N + D, peaked=True)


def test_fp32_index_operands_with_half_attention(fsi, dev):
    _run(fsi, dev, 2, 2, 128, 32, 16, 3, 0.8, torch.float16, seed=9, idx_dtype=torch.float32, scale=0.2)


def test_single_block_attends_itself(fsi, dev):
    """N == block_size: no remote block, so every row is plain self attention."""
    out, sel = _run(fsi, dev, 2, 2, 16, 32, 16, 2, 0.8, torch.float32, seed=1)
    assert sel.eq(-1).all()


def test_many_blocks(fsi, dev):
    """1024 blocks of 2 tokens: the scoring and argmax loops stride over the workgroup."""
    _run(fsi, dev, 1, 2, 2048, 16, 2, 4, 0.6, torch.bfloat16, seed=5, peaked=True)


def test_reference_wrapper_and_errors(fsi, dev):
    q = torch.randn(1, 2, 64, 32, device=dev, dtype=torch.float16)
    q16 = torch.randn(1, 4, 16, device=dev, dtype=torch.float16)
    out = fsi.triton_fused_sram_indexer_attention(q, q, q, q16, q16, block_size=16)
    ref, _ = fsi.sram_indexer_attention(q, q, q, q16, q16, block_size=16, return_selection=True)
    assert torch.equal(out, ref)
    with pytest.raises(AssertionError):
        fsi.triton_fused_sram_indexer_attention(q, q, q, q16, q16, block_size=24)
    with pytest.raises(RuntimeError):
        fsi.triton_fused_sram_indexer_attention(q.cpu(), q.cpu(), q.cpu(), q16.cpu(), q16.cpu())
    with pytest.raises(RuntimeError):  # block_size above the kernel's limit of 64
        big = torch.randn(1, 1, 256, 8, device=dev)
        fsi.triton_fused_sram_indexer_attention(big, big, big, torch.randn(1, 2, 16, device=dev),
                                                torch.randn(1, 2, 16, device=dev), block_size=128)


def test_graph_replays(fsi, dev):
    """The MFMA kernel captured in a graph and replayed with eager work in between:
    every replay equals the eager result."""
    g = torch.Generator().manual_seed(4)
    B, H, N, D, bs = 4, 4, 256, 32, 32
    q, k, v = (torch.randn(B, H, N, D, generator=g).half().to(dev) for _ in range(3))
    q16, k16 = (torch.randn(B, N // bs, 16, generator=g).half().to(dev) for _ in range(2))
    with torch.no_grad():
        eager = fsi.sram_indexer_attention(q, k, v, q16, k16, block_size=bs, max_remote_blocks=2)
        outs = {}
        graph = torch.cuda.CUDAGraph()
        st = torch.cuda.Stream(dev)
        st.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(st), torch.cuda.graph(graph, stream=st):
            outs["o"] = fsi.sram_indexer_attention(q, k, v, q16, k16, block_size=bs, max_remote_blocks=2)
        torch.cuda.synchronize(dev)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize(dev)
            assert torch.equal(outs["o"], eager)
            torch.randn(1024, 1024, device=dev).sum().item()
