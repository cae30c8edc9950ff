"""GPU parity of block-sparse prefill attention (fsi_sparse_attn).

Both modes are compared with fp64 softmax attention under the oracle's key
weights: sparse_mask (FovealSparseAttention's local window OR listed pages,
attention.py:148-218) and block_list_weights (triton_foveal_sparse_attention,
triton_ops.py:26-93).  bf16 outputs: rel-L2 <= 2e-3.  The module forward also
passes through the bf16 library GEMMs of the four projections on each side, so
its bar is rel-L2 1e-2, as for decode_step."""
import math

import pytest
import torch

from oracle import attention as A
from oracle import indexer as IX
from oracle import pattention as Pt
from oracle import routing as R

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _qkv(B, Hq, Hkv, T, hd, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, T, hd, generator=g).bfloat16()
    k = torch.randn(B, Hkv, T, hd, generator=g).bfloat16()
    v = torch.randn(B, Hkv, T, hd, generator=g).bfloat16()
    return q, k, v, g


LR_CASES = [
    # B, Hq, Hkv, hd, T, block, window, capacity
    (2, 8, 2, 128, 512, 64, 128, 3),
    (1, 4, 4, 64, 256, 64, 64, 4),
    (2, 8, 1, 64, 320, 64, 1, 2),      # window of one key: the query itself
    (1, 32, 8, 128, 1024, 64, 256, 8),
    (2, 4, 2, 32, 100, 16, 24, 3),     # T not a multiple of 16 or 32
    (1, 2, 1, 16, 96, 32, 40, 2),      # head_dim 16
    (1, 6, 1, 64, 192, 64, 1000, 2),   # window beyond T; 6 heads per KV head (two workgroups)
    (2, 4, 2, 128, 256, 64, 64, 0),    # no remote pages at all
    (1, 8, 2, 128, 200, 64, 100, 3),   # T not a multiple of the 64-query block
    (2, 16, 2, 64, 384, 64, 128, 5),   # 8 query heads per KV head (two workgroups)
    (1, 4, 4, 128, 256, 64, 64, 70),   # more than 64 listed pages per block
    (1, 4, 1, 128, 512, 128, 200, 3),  # 128-token blocks: 4 chunks per listed block
]


@pytest.mark.parametrize("case", LR_CASES, ids=[f"c{i}" for i in range(len(LR_CASES))])
def test_local_remote_parity(fsi, dev, case):
    B, Hq, Hkv, hd, T, blk, W, cap = case
    print(f"[case] sparse_attention local_remote {case}", flush=True)
    q, k, v, g = _qkv(B, Hq, Hkv, T, hd, seed=sum(case))
    Qb = -(-T // blk)
    idx = torch.randint(0, Qb, (B, Qb, max(cap, 1)), generator=g, dtype=torch.int32)[:, :, :cap]
    cnt = torch.randint(0, cap + 1, (B, Qb), generator=g, dtype=torch.int32)
    if cap >= 2:
        idx[0, Qb - 1, :2] = torch.tensor([0, 0], dtype=torch.int32)  # a page listed twice counts once
        cnt[0, Qb - 1] = 2
    scale = 1.0 / math.sqrt(hd)
    out = fsi.sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev) if cap else None, cnt.to(dev), block=blk,
                               mode=0, window=W, scale=scale)
    mask = A.sparse_mask(B, T, W, blk, idx, cnt)
    ref = A.weighted_attention_f64(q, k, v, mask, scale)
    err = Pt.rel_l2(out.cpu().float(), ref.float())
    assert err <= TOL, err


BL_CASES = [
    # B, H, N, D, block_size, max_active
    (2, 4, 128, 64, 16, 4),
    (1, 2, 256, 128, 32, 5),
    (2, 3, 192, 16, 64, 2),
    (1, 8, 512, 128, 64, 8),
    (1, 2, 64, 32, 16, 6),
]


@pytest.mark.parametrize("case", BL_CASES, ids=[f"c{i}" for i in range(len(BL_CASES))])
def test_block_list_parity(fsi, dev, case):
    """triton_foveal_sparse_attention: every key of each listed block, no causal
    mask, a block listed twice counts twice, an empty list gives 0."""
    B, H, N, D, bs, mx = case
    print(f"[case] triton_foveal_sparse_attention {case}", flush=True)
    q, k, v, g = _qkv(B, H, H, N, D, seed=7 * sum(case))
    M = N // bs
    idx = torch.randint(0, M, (B, M, mx), generator=g, dtype=torch.int32)
    cnt = torch.randint(0, mx + 1, (B, M), generator=g, dtype=torch.int32)
    cnt[0, 0] = 0
    idx[0, 1, :2] = 1
    cnt[0, 1] = max(int(cnt[0, 1]), 2)
    out = fsi.triton_foveal_sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), cnt.to(dev),
                                             block_size=bs).cpu()
    assert out.is_contiguous() and out.shape == q.shape
    w = A.block_list_weights(B, N, bs, idx, cnt)
    ref = A.weighted_attention_f64(q, k, v, w, 1.0 / math.sqrt(D))
    assert torch.equal(out[0, :, :bs], torch.zeros(H, bs, D, dtype=torch.bfloat16))
    err = Pt.rel_l2(out.float(), ref.float())
    assert err <= TOL, err


# fp32 (FovealSparseAttention's default dtype): the fp32 MFMA kernel for pages
# of a power-of-two multiple of 64 and head_dim 64 / 128, the generic kernel for
# the other cases of the same lists.  fp32 bar: rel-L2 <= 1e-5 against fp64.
TOL_F32 = 1e-5


@pytest.mark.parametrize("case", LR_CASES, ids=[f"c{i}" for i in range(len(LR_CASES))])
def test_local_remote_parity_f32(fsi, dev, case):
    B, Hq, Hkv, hd, T, blk, W, cap = case
    print(f"[case] sparse_attention fp32 local_remote {case}", flush=True)
    q, k, v, g = _qkv(B, Hq, Hkv, T, hd, seed=sum(case) + 1)
    q, k, v = q.float(), k.float(), v.float()
    Qb = -(-T // blk)
    idx = torch.randint(0, Qb, (B, Qb, max(cap, 1)), generator=g, dtype=torch.int32)[:, :, :cap]
    cnt = torch.randint(0, cap + 1, (B, Qb), generator=g, dtype=torch.int32)
    if cap >= 2:
        idx[0, Qb - 1, :2] = torch.tensor([0, 0], dtype=torch.int32)
        cnt[0, Qb - 1] = 2
    scale = 1.0 / math.sqrt(hd)
    out = fsi.sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev) if cap else None, cnt.to(dev), block=blk,
                               mode=0, window=W, scale=scale)
    assert out.dtype == torch.float32
    mask = A.sparse_mask(B, T, W, blk, idx, cnt)
    ref = A.weighted_attention_f64(q, k, v, mask, scale)
    err = Pt.rel_l2(out.cpu(), ref.float())
    assert err <= TOL_F32, err


@pytest.mark.parametrize("case", BL_CASES, ids=[f"c{i}" for i in range(len(BL_CASES))])
def test_block_list_parity_f32(fsi, dev, case):
    B, H, N, D, bs, mx = case
    print(f"[case] triton_foveal_sparse_attention fp32 {case}", flush=True)
    q, k, v, g = _qkv(B, H, H, N, D, seed=7 * sum(case) + 1)
    q, k, v = q.float(), k.float(), v.float()
    M = N // bs
    idx = torch.randint(0, M, (B, M, mx), generator=g, dtype=torch.int32)
    cnt = torch.randint(0, mx + 1, (B, M), generator=g, dtype=torch.int32)
    cnt[0, 0] = 0
    idx[0, 1, :2] = 1
    cnt[0, 1] = max(int(cnt[0, 1]), 2)
    out = fsi.triton_foveal_sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), cnt.to(dev),
                                             block_size=bs).cpu()
    w = A.block_list_weights(B, N, bs, idx, cnt)
    ref = A.weighted_attention_f64(q, k, v, w, 1.0 / math.sqrt(D))
    assert torch.equal(out[0, :, :bs], torch.zeros(H, bs, D))
    err = Pt.rel_l2(out, ref.float())
    assert err <= TOL_F32, err


@pytest.mark.parametrize("hd", [64, 128])
def test_value_range_f32(fsi, dev, hd):
    """Scores spreading over tens of log2 units (the running max moves several
    times and the accumulators are rescaled) and values of very different size
    per KV head, fp32 end to end."""
    B, Hq, Hkv, T, blk, W, cap = 1, 8, 2, 640, 64, 192, 4
    g = torch.Generator().manual_seed(hd)
    q = torch.randn(B, Hq, T, hd, generator=g) * 2.0
    k = torch.randn(B, Hkv, T, hd, generator=g) * torch.linspace(0.1, 2.0, T).view(1, 1, T, 1)
    v = torch.randn(B, Hkv, T, hd, generator=g) * torch.tensor([1e-3, 1e3]).view(1, 2, 1, 1)
    Qb = T // blk
    idx = torch.randint(0, Qb, (B, Qb, cap), generator=g, dtype=torch.int32)
    cnt = torch.full((B, Qb), cap, dtype=torch.int32)
    scale = 1.0 / math.sqrt(hd)
    out = fsi.sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), cnt.to(dev), block=blk, mode=0,
                               window=W, scale=scale)
    ref = A.weighted_attention_f64(q, k, v, A.sparse_mask(B, T, W, blk, idx, cnt), scale)
    for hk in range(Hkv):  # per KV head group: values of 1e-3 and 1e3
        hs = slice(hk * (Hq // Hkv), (hk + 1) * (Hq // Hkv))
        err = Pt.rel_l2(out[:, hs].cpu(), ref[:, hs].float())
        assert err <= TOL_F32, (hk, err)


def test_strided_views_in_place(fsi, dev):
    """q, k, v as (B, T, H, hd) projections viewed (B, H, T, hd), output written
    into such a view."""
    B, Hq, Hkv, T, hd, blk = 2, 8, 2, 256, 64, 64
    g = torch.Generator().manual_seed(11)
    qs = torch.randn(B, T, Hq, hd, generator=g).bfloat16()
    ks = torch.randn(B, T, Hkv, hd, generator=g).bfloat16()
    vs = torch.randn(B, T, Hkv, hd, generator=g).bfloat16()
    idx = torch.tensor([[[0, 1], [0, 2], [1, 0], [2, 0]]] * B, dtype=torch.int32)
    cnt = torch.tensor([[0, 1, 2, 1]] * B, dtype=torch.int32)
    outs = torch.zeros(B, T, Hq, hd, dtype=torch.bfloat16, device=dev)
    fsi.sparse_attention(qs.to(dev).transpose(1, 2), ks.to(dev).transpose(1, 2), vs.to(dev).transpose(1, 2),
                         idx.to(dev), cnt.to(dev), block=blk, mode=0, window=70, scale=0.1,
                         out=outs.transpose(1, 2))
    mask = A.sparse_mask(B, T, 70, blk, idx, cnt)
    ref = A.weighted_attention_f64(qs.transpose(1, 2), ks.transpose(1, 2), vs.transpose(1, 2), mask, 0.1)
    err = Pt.rel_l2(outs.cpu().transpose(1, 2).float(), ref.float())
    assert err <= TOL, err


@pytest.mark.parametrize("hd", [64, 128])
def test_value_range_per_head(fsi, dev, hd):
    """The 64-query kernel takes V as fp16 scaled by a power of two per (sequence,
    KV head): heads whose values sit near the ends of the bf16 range, a head with
    one outlier 2^20 above the rest and an all-zero head all stay within the bf16
    bar, head by head, against fp64 attention."""
    B, Hq, Hkv, T, blk, W, cap = 2, 8, 4, 448, 64, 96, 3
    print(f"[case] sparse_attention value range hd={hd}", flush=True)
    q, k, v, g = _qkv(B, Hq, Hkv, T, hd, seed=31 + hd)
    v = v.float()
    v[:, 0] *= 1e30
    v[:, 1] *= 1e-30
    v[0, 2, 77, 5] = 2.0 ** 20
    v[1, 3] = 0.0
    v = v.bfloat16()
    Qb = -(-T // blk)
    idx = torch.randint(0, Qb, (B, Qb, cap), generator=g, dtype=torch.int32)
    cnt = torch.randint(0, cap + 1, (B, Qb), generator=g, dtype=torch.int32)
    scale = 1.0 / math.sqrt(hd)
    out = fsi.sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx.to(dev), cnt.to(dev), block=blk, mode=0,
                               window=W, scale=scale).cpu().float()
    ref = A.weighted_attention_f64(q, k, v, A.sparse_mask(B, T, W, blk, idx, cnt), scale).float()
    assert torch.equal(out[1, 6:8], torch.zeros_like(out[1, 6:8]))  # KV head 3 of sequence 1 is zero
    for b in range(B):
        for h in range(Hq):
            if b == 1 and h >= 6:
                continue
            err = Pt.rel_l2(out[b, h], ref[b, h])
            assert err <= TOL, (b, h, err)


def test_invalid_block_reported(fsi, dev, monkeypatch):
    q, k, v, _ = _qkv(1, 2, 1, 128, 64, seed=5)
    idx = torch.tensor([[[0], [5]]], dtype=torch.int32, device=dev)  # 2 blocks exist
    cnt = torch.tensor([[0, 1]], dtype=torch.int32, device=dev)
    monkeypatch.setenv("FSI_CHECK", "1")
    with pytest.raises(IndexError):
        fsi.sparse_attention(q.to(dev), k.to(dev), v.to(dev), idx, cnt, block=64, mode=0, window=64)


def test_prefill_forward_module(fsi, dev):
    """FovealSparseAttention.forward: route against the routing oracle on the
    module's own block scores, output against the CPU restatement of
    attention.py:180-269 under that route, distillation loss against the loss
    of the oracle's dense teacher mass."""
    from route_check import check_rows

    torch.manual_seed(0)
    B, T, D = 2, 1024, 256
    m = fsi.FovealSparseAttention(hidden_size=D, num_heads=8, num_kv_heads=2, head_dim=32, page_size=64,
                                  local_window_blocks=2, top_p=0.8, min_remote_pages=1, max_remote_pages=3,
                                  remote_capacity=4).to(torch.bfloat16)
    cpu = {kk: vv.clone() for kk, vv in m.state_dict().items()}
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, T, D, generator=g).bfloat16()
    md = m.to(dev)
    with torch.no_grad():
        out, aux = md(x.to(dev), compute_teacher_loss=True)
        xd = x.to(dev)
        qb = md.indexer.compute_query_16d(xd)[:, ::64]
        kb, _ = md.indexer.compute_kv_blocks_16d(xd)
        scores = md.indexer.compute_block_scores(qb, kb).cpu()
    route = aux["route"]
    ora = R.select_route(scores, causal=True, local_window_blocks=2, top_p=0.8, min_remote_blocks=1,
                         max_remote_blocks=3, remote_capacity=4)
    _, _, remote = R.route_masks(T // 64, T // 64, True, 2)
    assert not check_rows(route.remote_indices, route.remote_counts, ora, remote, 1e-6, 1e-5)

    mc = fsi.FovealSparseAttention(hidden_size=D, num_heads=8, num_kv_heads=2, head_dim=32, page_size=64,
                                   local_window_blocks=2, top_p=0.8, min_remote_pages=1, max_remote_pages=3,
                                   remote_capacity=4).to(torch.bfloat16)
    mc.load_state_dict(cpu)
    ref, teacher = A.prefill_forward(mc, x, route.remote_indices.cpu(), route.remote_counts.cpu())
    err = Pt.rel_l2(out.cpu().float(), ref.float())
    assert err <= 1e-2, err
    assert aux["additive_out"] is not None and out.shape == (B, T, D)
    ref_loss = IX.distillation_loss(scores, teacher, causal=True, temperature=mc.indexer.distill_temperature)
    assert math.isclose(float(aux["distill_loss"]), float(ref_loss), rel_tol=1e-2, abs_tol=1e-5)


def test_graph_replays_after_workspace_growth(fsi, dev):
    """The fp16 V^T path (three launches) captured in a graph on a side stream and
    replayed with eager work between replays: every replay equals the eager
    result, also after a larger eager call on the same stream has grown that
    stream's workspace (the captured buffer stays alive and untouched by others)."""
    B, Hq, Hkv, T, hd, blk, W, cap = 1, 8, 2, 512, 128, 64, 128, 3
    q, k, v, g = _qkv(B, Hq, Hkv, T, hd, seed=77)
    Qb = T // blk
    idx = torch.randint(0, Qb, (B, Qb, cap), generator=g, dtype=torch.int32).to(dev)
    cnt = torch.randint(0, cap + 1, (B, Qb), generator=g, dtype=torch.int32).to(dev)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    qb, kb, vb = (torch.randn(1, 8, 8192, hd, generator=g).bfloat16().to(dev) for _ in range(3))
    big_idx = torch.zeros(1, 8192 // blk, cap, dtype=torch.int32, device=dev)
    big_cnt = torch.zeros(1, 8192 // blk, dtype=torch.int32, device=dev)

    def call():
        return fsi.sparse_attention(q, k, v, idx, cnt, block=blk, mode=0, window=W, scale=0.09)

    with torch.no_grad():
        eager = call()
        st = torch.cuda.Stream(dev)
        st.wait_stream(torch.cuda.current_stream(dev))
        outs = {}
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(st):
            call()  # warm-up on the capture stream: its workspace exists before the capture
            torch.cuda.synchronize(dev)
            with torch.cuda.graph(graph, stream=st):
                outs["o"] = call()
            # a larger call on the same stream grows its workspace
            fsi.sparse_attention(qb, kb[:, :2], vb[:, :2], big_idx, big_cnt, block=blk, mode=0, window=W, scale=0.09)
        torch.cuda.synchronize(dev)
        # blocks of the sizes a freed workspace of this call would offer for reuse
        fill = [torch.full((n // 4,), 7, dtype=torch.int32, device=dev)
                for n in (1 << 20, 3 << 19, 1 << 21) for _ in range(8)]
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize(dev)
            assert torch.equal(outs["o"], eager)
            torch.randn(1024, 1024, device=dev).sum().item()
        assert all(bool((f == 7).all()) for f in fill)


GRAD_CASES = [
    # B, Hq, Hkv, hd, T, block, window, capacity, mode, dtype
    (2, 4, 2, 64, 256, 64, 96, 3, 0, torch.float32),
    (1, 8, 2, 128, 320, 64, 200, 4, 0, torch.bfloat16),     # T not a multiple of 64
    (2, 4, 4, 32, 192, 16, 40, 5, 0, torch.float32),        # 16-key blocks: four per tile
    (1, 6, 1, 96, 256, 128, 130, 2, 0, torch.bfloat16),     # head_dim 96 (padded to 128), 128-token blocks
    (2, 4, 2, 64, 256, 32, 0, 4, 1, torch.float32),         # block lists, repeated entries
    (1, 2, 2, 16, 128, 16, 0, 6, 1, torch.bfloat16),
    (2, 4, 2, 64, 200, 32, 0, 3, 1, torch.bfloat16),       # bf16 tile kernels: block lists, tiles over two blocks
    (1, 4, 4, 32, 256, 64, 100, 3, 0, torch.bfloat16),      # bf16 tile kernels at head_dim 32
]


@pytest.mark.parametrize("case", GRAD_CASES, ids=[f"g{i}" for i in range(len(GRAD_CASES))])
def test_sparse_attention_gradients(fsi, dev, case):
    """The HIP backward (fsi_sparse_attn_bwd) against fp64 autograd of softmax
    attention under the oracle's key weights (sparse_mask / block_list_weights):
    dq, dk, dv within rel-L2 2e-5 for fp32 inputs and 1e-2 for bf16 (gradients
    rounded to bf16)."""
    B, Hq, Hkv, hd, T, blk, W, cap, mode, dtype = case
    print(f"[case] sparse_attention backward {case}", flush=True)
    g = torch.Generator().manual_seed(T + hd + cap)
    q = torch.randn(B, Hq, T, hd, generator=g).to(dtype)
    k = torch.randn(B, Hkv, T, hd, generator=g).to(dtype)
    v = torch.randn(B, Hkv, T, hd, generator=g).to(dtype)
    dout = torch.randn(B, Hq, T, hd, generator=g).to(dtype)
    Qb = -(-T // blk)
    idx = torch.randint(0, Qb, (B, Qb, cap), generator=g, dtype=torch.int32)
    cnt = torch.randint(0, cap + 1, (B, Qb), generator=g, dtype=torch.int32)
    idx[0, Qb - 1, :2] = 0  # a block listed twice
    cnt[0, Qb - 1] = max(int(cnt[0, Qb - 1]), 2)
    cnt[0, 0] = 0
    scale = 1.0 / math.sqrt(hd)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    out = fsi.sparse_attention(qd, kd, vd, idx.to(dev), cnt.to(dev), block=blk, mode=mode, window=W, scale=scale)
    out.backward(dout.to(dev))
    w = A.sparse_mask(B, T, W, blk, idx, cnt) if mode == 0 else A.block_list_weights(B, T, blk, idx, cnt)
    q64, k64, v64 = (t.double().requires_grad_() for t in (q, k, v))
    ref = A.weighted_attention_f64(q64, k64, v64, w, scale)
    ref.backward(dout.double())
    tol = 2e-5 if dtype == torch.float32 else 1e-2
    assert Pt.rel_l2(out.detach().cpu().float(), ref.detach().float()) <= (1e-5 if dtype == torch.float32 else TOL)
    for name, got, want in (("dq", qd.grad, q64.grad), ("dk", kd.grad, k64.grad), ("dv", vd.grad, v64.grad)):
        assert got.dtype == dtype
        err = Pt.rel_l2(got.cpu().float(), want.float())
        print(f"  {name} rel-L2 {err:.2e}", flush=True)
        assert err <= tol, (name, err)


def test_sparse_attention_backward_strided_views(fsi, dev):
    """q, k, v as (B, T, H, hd) projections viewed (B, H, T, hd), as the module
    passes them: gradients land in the views' storage order."""
    B, Hq, Hkv, T, hd, blk = 1, 4, 2, 192, 64, 64
    g = torch.Generator().manual_seed(12)
    qs = torch.randn(B, T, Hq, hd, generator=g)
    ks = torch.randn(B, T, Hkv, hd, generator=g)
    vs = torch.randn(B, T, Hkv, hd, generator=g)
    idx = torch.tensor([[[0, 1], [0, 0], [1, 0]]], dtype=torch.int32)
    cnt = torch.tensor([[0, 1, 2]], dtype=torch.int32)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (qs, ks, vs))
    out = fsi.sparse_attention(qd.transpose(1, 2), kd.transpose(1, 2), vd.transpose(1, 2), idx.to(dev), cnt.to(dev),
                               block=blk, mode=0, window=70, scale=0.1)
    dout = torch.randn(B, Hq, T, hd, generator=g)
    out.backward(dout.to(dev))
    q64, k64, v64 = (t.double().requires_grad_() for t in (qs, ks, vs))
    ref = A.weighted_attention_f64(q64.transpose(1, 2), k64.transpose(1, 2), v64.transpose(1, 2),
                                   A.sparse_mask(B, T, 70, blk, idx, cnt), 0.1)
    ref.backward(dout.double())
    for got, want in ((qd.grad, q64.grad), (kd.grad, k64.grad), (vd.grad, v64.grad)):
        assert Pt.rel_l2(got.cpu().float(), want.float()) <= 2e-5


def test_prefill_module_backward_16k(fsi, dev):
    """FovealSparseAttention.forward + backward at 16384 tokens with the
    Llama-3-8B attention heads (32 / 8, head_dim 128): runs without any (T, T)
    tensor (a dense fp32 score tensor alone would take 32 GiB), gives finite
    gradients for every parameter, and the attention core's gradients equal the
    dense recompute's on a 1024-token slice of the same module (rel-L2 1e-2)."""
    torch.manual_seed(0)
    D, T = 4096, 16384
    m = fsi.FovealSparseAttention(hidden_size=D, num_heads=32, num_kv_heads=8, head_dim=128, page_size=64,
                                  local_window_blocks=16, top_p=0.9, min_remote_pages=0, max_remote_pages=32,
                                  remote_capacity=32).to(torch.bfloat16).to(dev)
    x = (torch.randn(1, T, D, device=dev) * 0.5).bfloat16().requires_grad_()
    torch.cuda.reset_peak_memory_stats(dev)
    out, aux = m(x)
    out.float().pow(2).mean().backward()
    peak = torch.cuda.max_memory_allocated(dev)
    print(f"16K forward + backward peak memory {peak / 2**30:.2f} GiB", flush=True)
    assert peak < 24 * 2**30
    assert torch.isfinite(x.grad.float()).all()
    for name, p in m.named_parameters():
        if p.grad is not None:
            assert torch.isfinite(p.grad.float()).all(), name
    assert m.q_proj.weight.grad is not None and float(m.q_proj.weight.grad.float().abs().sum()) > 0


def test_sparse_attention_backward_matches_dense_recompute(fsi, dev):
    """The HIP backward and the dense fp32 recompute (the path head_dim > 128
    keeps) give the same gradients on a routed 1024-token pattern (rel-L2 1e-2,
    bf16 outputs)."""
    att = fsi.attention
    B, Hq, Hkv, hd, T, blk, W = 1, 8, 2, 128, 1024, 64, 256
    g = torch.Generator().manual_seed(21)
    q, k, v, dout = (torch.randn(B, h, T, hd, generator=g).bfloat16().to(dev) for h in (Hq, Hkv, Hkv, Hq))
    Qb = T // blk
    scores = torch.randn(B, Qb, Qb, generator=g).to(dev)
    route = fsi.select_blocks(scores, causal=True, block_size=blk, local_window_blocks=W // blk, top_p=0.9,
                              min_remote_blocks=0, max_remote_blocks=8, remote_capacity=8)
    lists, counts = route.remote_indices, route.remote_counts
    with torch.no_grad():
        out = fsi.sparse_attention(q, k, v, lists, counts, block=blk, mode=0, window=W, scale=hd ** -0.5)
    hip = att._sparse_attention_bwd(q, k, v, out, dout, lists, counts, 8, blk, 0, W, hd ** -0.5)
    dense = att._sparse_attention_bwd_dense(q, k, v, dout, lists, counts, 8, blk, 0, W, hd ** -0.5)
    for a, b in zip(hip, dense):
        assert Pt.rel_l2(a.float().cpu(), b.float().cpu()) <= 1e-2
