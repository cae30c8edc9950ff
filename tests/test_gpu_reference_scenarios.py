"""The reference's own module tests, run on the GPU with the reference's
constructor arguments and default dtype (fp32), and checked against the CPU
oracle in fp64 — forward values and gradients:
  * tests/test_attention.py:10-35   prefill forward + teacher loss + backward
                                    (page 16, head_dim 16, GQA 4/2)
  * tests/test_attention.py:37-62   40 decode steps on a page-8, head_dim-16 cache
  * tests/test_block_matmul.py:10-44 BlockSparseLinear (block 32, bias) + backward
  * tests/test_block_matmul.py:46-65 BlockwiseMatMul2D (32 x 32 tiles) + backward
"""
import copy

import pytest
import torch

from oracle import attention as A
from oracle import blocksparse as BS
from oracle import indexer as IX
from oracle import pattention as Pt
from oracle import routing as R

pytestmark = pytest.mark.gpu

F64 = torch.float64


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def test_attention_prefill_and_loss(fsi, dev):
    torch.manual_seed(0)
    attn = fsi.FovealSparseAttention(hidden_size=64, num_heads=4, num_kv_heads=2, head_dim=16, page_size=16,
                                     local_window_blocks=2, index_dim=16, top_p=0.9, max_remote_pages=2)
    ref_m = copy.deepcopy(attn).double()
    attn = attn.to(dev)
    x = torch.randn(2, 64, 64)
    xd = x.to(dev).requires_grad_()
    out, aux = attn(xd, compute_teacher_loss=True)
    assert out.shape == (2, 64, 64) and out.dtype == torch.float32
    assert aux["route"].remote_counts.shape == (2, 4)
    assert aux["distill_loss"].item() >= 0.0
    (out.sum() + aux["distill_loss"]).backward()
    assert attn.q_proj.weight.grad is not None and attn.indexer.q_proj.weight.grad is not None

    # the same graph in fp64 on the CPU over the route the module chose
    # (attention.py:180-269: the indexer branch sees x detached)
    m = ref_m
    xr = x.double().requires_grad_()
    ri, rc = aux["route"].remote_indices.cpu(), aux["route"].remote_counts.cpu()
    q = m.q_proj(xr).view(2, 64, 4, 16).transpose(1, 2)
    k = m.k_proj(xr).view(2, 64, 2, 16).transpose(1, 2)
    v = m.v_proj(xr).view(2, 64, 2, 16).transpose(1, 2)
    att = A.weighted_attention_f64(q, k, v, A.sparse_mask(2, 64, m.local_window, 16, ri, rc), m.scale)
    ref_out = m.out_proj(att.transpose(1, 2).reshape(2, 64, 64))
    xdet = xr.detach()
    qi = IX.rms_norm16(m.indexer.q_proj(xdet))
    kb, vb = IX.pool_kv(m.indexer.k_proj(xdet), m.indexer.v_proj(xdet), 16, F64)
    scores = IX.block_scores(qi[:, ::16], kb, F64)
    ref_out = ref_out + m.indexer.out_proj(IX.additive_context(scores, vb, True, F64)).repeat_interleave(16, dim=1)
    with torch.no_grad():
        s = torch.matmul(q, k.repeat_interleave(2, dim=1).transpose(-2, -1)) * m.scale
        s = s.masked_fill(~torch.tril(torch.ones(64, 64, dtype=torch.bool)), float("-inf"))
        teacher = torch.softmax(s, dim=-1)[:, :, ::16].view(2, 4, 4, 4, 16).sum(-1).mean(1)
    ref_loss = IX.distillation_loss(scores, teacher, causal=True, acc=F64)
    (ref_out.sum() + ref_loss).backward()
    assert _rel(out, ref_out) <= 1e-5
    assert abs(float(aux["distill_loss"]) - float(ref_loss)) <= 1e-4 * max(1.0, float(ref_loss))
    assert _rel(xd.grad, xr.grad) <= 1e-4
    for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
        assert _rel(getattr(attn, name).weight.grad, getattr(ref_m, name).weight.grad) <= 1e-4, name
    assert _rel(attn.indexer.q_proj.weight.grad, ref_m.indexer.q_proj.weight.grad) <= 1e-4


def test_attention_kv_cache_decode(fsi, dev):
    torch.manual_seed(1)
    attn = fsi.FovealSparseAttention(hidden_size=32, num_heads=2, num_kv_heads=2, head_dim=16, page_size=8,
                                     local_window_blocks=2, index_dim=16, top_p=0.9, min_remote_pages=1,
                                     max_remote_pages=2)
    ref_m = copy.deepcopy(attn)
    attn = attn.to(dev)
    kv_cache = attn.init_kv_cache(batch_size=1, max_seq_len=48, device=dev)
    assert kv_cache.dtype == torch.float32 and not kv_cache.paged
    assert kv_cache.k_cache.shape == (1, 2, 48, 16)  # the reference's contiguous layout
    oracle = A.DecodeStepOracle(ref_m, batch=1, max_seq_len=48)
    for step in range(40):
        tok = torch.randn(1, 1, 32)
        out, dec_aux = attn.decode_step(tok.to(dev), kv_cache)
        ref, pages, _ = oracle.step(tok)
        assert out.shape == (1, 1, 32)
        assert dec_aux["selected_remote_pages"] == [list(p) for p in pages], step
        assert _rel(out, ref) <= 1e-5, step
    assert len(dec_aux["selected_remote_pages"][0]) >= 1


def test_block_sparse_linear_reference_scenario(fsi, dev):
    torch.manual_seed(2)
    linear = fsi.BlockSparseLinear(in_features=64, out_features=256, block_size=32, base_blocks=2, index_dim=16,
                                   top_p=0.5, max_remote_blocks=2, bias=True)
    assert linear.weight.dtype == torch.float32
    ref_m = copy.deepcopy(linear)
    linear = linear.to(dev)
    x = torch.randn(2, 4, 64)
    xd = x.to(dev).requires_grad_()
    out, aux = linear(xd, compute_teacher_loss=True)
    assert out.shape == (2, 4, 256)
    assert aux["mean_active_blocks"] <= 4
    assert aux["route"].remote_counts.max().item() <= 2
    assert aux["sparsity"] >= 0.5
    assert aux["distill_loss"].item() >= 0.0
    x_single = torch.randn(1, 1, 64, device=dev)
    _, aux_single = linear(x_single)
    assert aux_single["active_blocks_union"] <= 4
    (out.sum() + aux["distill_loss"]).backward()
    assert linear.weight.grad is not None and linear.bias.grad is not None
    assert linear.weight_to_k.weight.grad is not None

    # gradients of the sparse product: the oracle's gather -> F.linear -> scatter
    # in fp64 over the module's active set (block_matmul.py:215-232)
    route = aux["route"]
    cap = route.remote_indices.shape[-1]
    valid = torch.arange(cap, device=dev)[None, None] < route.remote_counts[..., None]
    sel = route.remote_indices[valid]
    mask = torch.zeros(8, dtype=torch.bool)
    mask[:2] = True
    mask[sel[sel >= 2].long().cpu()] = True
    active = torch.where(mask)[0]
    w = ref_m.weight.detach().double().requires_grad_()
    bias = ref_m.bias.detach().double().requires_grad_()
    xr = x.double().requires_grad_()
    y = BS.block_sparse_linear_f64(xr.reshape(8, 64), w, bias, active, 32)
    gy = torch.ones_like(y)
    y.backward(gy)
    # the module's product gradient alone: rerun the sparse GEMM op through autograd
    wd = linear.weight.detach().clone().requires_grad_()
    bd = linear.bias.detach().clone().requires_grad_()
    xd2 = x.to(dev).reshape(8, 64).requires_grad_()
    yd = fsi.block_sparse_linear(xd2, wd, bd, active.to(dev), 32)
    yd.backward(torch.ones_like(yd))
    assert _rel(yd, y) <= 1e-5
    assert _rel(xd2.grad, xr.grad.reshape(8, 64)) <= 1e-5
    assert _rel(wd.grad, w.grad) <= 1e-5 and _rel(bd.grad, bias.grad) <= 1e-5


def test_blockwise_matmul_2d_reference_scenario(fsi, dev):
    torch.manual_seed(3)
    matmul = fsi.BlockwiseMatMul2D(in_features=64, out_features=64, block_k=32, block_n=32, base_tiles_ratio=0.25,
                                   top_p=0.8)
    assert matmul.weight.dtype == torch.float32
    matmul = matmul.to(dev)
    x = torch.randn(2, 4, 64)
    xd = x.to(dev).requires_grad_()
    out, aux = matmul(xd, compute_teacher_loss=True)
    assert out.shape == (2, 4, 64)
    assert aux["total_tiles"] == 4
    assert aux["distill_loss"].item() >= 0.0
    (out.sum() + aux["distill_loss"]).backward()
    assert matmul.weight.grad is not None and matmul.tile_q.weight.grad is not None

    # routing vs the oracle given the module's scores; product and its gradients vs fp64
    with torch.no_grad():
        mask, probs, scores, tile_v = matmul.route_tiles(xd)
    ref = R.tile_route(scores.reshape(-1, 4).cpu(), 0.8, matmul.base_tiles)
    assert torch.equal(mask.cpu(), ref["mask"][0])
    w = matmul.weight.detach().cpu().double().requires_grad_()
    xr = x.double().reshape(8, 64).requires_grad_()
    em = BS.expand_tile_mask(mask.cpu(), 64, 64, 32, 32)
    y = xr @ (w * em).t()
    y.backward(torch.ones_like(y))
    wd = matmul.weight.detach().clone().requires_grad_()
    xd2 = x.to(dev).reshape(8, 64).requires_grad_()
    yd = fsi.blockwise_matmul(xd2, wd, mask, 32, 32)
    yd.backward(torch.ones_like(yd))
    assert _rel(yd, y) <= 1e-5 and _rel(xd2.grad, xr.grad) <= 1e-5 and _rel(wd.grad, w.grad) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("page,hd", [(8, 16), (16, 32), (32, 64), (64, 48)])
def test_dense_decode_attention_parity(fsi, dev, dtype, page, hd):
    """fsi_decode_attn_dense over the contiguous cache for page sizes and head
    dims outside the paged MFMA layout, against fp64 attention."""
    g = torch.Generator().manual_seed(page * 100 + hd)
    B, Hq, Hkv, S = 3, 8, 2, 40 * page
    c = fsi.FovealKVCache(B, S, Hkv, hd, 16, page, dev, dtype)
    assert not c.paged
    k = torch.randn(B, Hkv, S, hd, generator=g).to(dtype)
    v = torch.randn(B, Hkv, S, hd, generator=g).to(dtype)
    c.load_dense(k.to(dev), v.to(dev))
    q = torch.randn(B, Hq, hd, generator=g).to(dtype)
    pos, W = S - 3, 5 * page
    pages = [[0, 7, 3], [1], []]
    rp = torch.full((B, 3), -1, dtype=torch.int32)
    for b, p in enumerate(pages):
        rp[b, :len(p)] = torch.tensor(p, dtype=torch.int32)
    cnt = torch.tensor([len(p) for p in pages], dtype=torch.int32)
    out = fsi.decode_attention(q.to(dev), c, pos=pos, window=W, remote_pages=rp.to(dev),
                               remote_counts=cnt.to(dev), scale=hd ** -0.5)
    ref = A.decode_attention_f64(q.float(), k, v, pos, W, pages, page, hd ** -0.5)
    tol = 1e-5 if dtype == torch.float32 else 4e-3
    assert out.dtype == dtype and Pt.rel_l2(out.cpu().float(), ref.float()) <= tol


@pytest.mark.parametrize("hd,Hq,Hkv,page,W,pages_per_seq", [
    (128, 32, 8, 64, 1024, 20),   # the C4 head shape: 2304 keys in 18 splits per sequence
    (64, 8, 8, 64, 200, 3),       # one query head per KV head
    (128, 40, 2, 32, 96, 5),      # 20 query heads per KV head: two MFMA column blocks
    (64, 12, 3, 16, 0, 6),        # no window, pages only
])
def test_dense_decode_attention_f32_split(fsi, dev, hd, Hq, Hkv, page, W, pages_per_seq):
    """fp32 contiguous-cache decode on the split MFMA kernels (head_dim 64 / 128):
    per-sequence positions, pages listed twice and pages inside the window (both
    counted, attention.py:341-352), a sequence with no key at all, against fp64."""
    print(f"[case] dense decode fp32 hd={hd} Hq={Hq} Hkv={Hkv} page={page} W={W} pages={pages_per_seq}", flush=True)
    g = torch.Generator().manual_seed(hd + Hq + page + W)
    B, S = 4, 64 * page
    c = fsi.FovealKVCache(B, S, Hkv, hd, 16, page, dev, torch.float32)
    assert not c.paged
    k = torch.randn(B, Hkv, S, hd, generator=g)
    v = torch.randn(B, Hkv, S, hd, generator=g)
    c.load_dense(k.to(dev), v.to(dev))
    q = torch.randn(B, Hq, hd, generator=g)
    pos = [S - 1, S // 2 + 7, 3 * page - 1, -1]
    pages = []
    for b in range(B):
        done = max((pos[b] + 1) // page, 0)
        n = min(pages_per_seq, done) if b < 3 else 0
        lst = torch.randint(0, max(done, 1), (n,), generator=g).tolist()
        if n >= 2:
            lst[1] = lst[0]  # listed twice: counted twice
        pages.append(lst)
    cap = max(len(p) for p in pages) or 1
    rp = torch.full((B, cap), -1, dtype=torch.int32)
    for b, p in enumerate(pages):
        if p:
            rp[b, :len(p)] = torch.tensor(p, dtype=torch.int32)
    cnt = torch.tensor([len(p) for p in pages], dtype=torch.int32)
    pos_t = torch.tensor(pos, dtype=torch.int32)
    out = fsi.decode_attention(q.to(dev), c, pos=pos_t.to(dev), window=W, remote_pages=rp.to(dev),
                               remote_counts=cnt.to(dev), scale=hd ** -0.5).cpu()
    ref = A.decode_attention_f64(q, k, v, [max(p, -1) for p in pos], W, pages, page, hd ** -0.5)
    assert torch.equal(out[3], torch.zeros(Hq, hd))  # no key: 0
    assert Pt.rel_l2(out[:3], ref[:3].float()) <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("block,hd,mode", [(8, 16, 0), (16, 24, 0), (64, 64, 0), (8, 32, 1), (32, 100, 1)])
def test_generic_sparse_attention_parity(fsi, dev, dtype, block, hd, mode):
    """fsi_sparse_attn's generic kernel (fp32, and bf16 blocks / head dims the
    MFMA kernels do not tile) against fp64 attention under the same pattern."""
    g = torch.Generator().manual_seed(block * 7 + hd + mode)
    B, Hq, Hkv, T = 2, 4, 2, 8 * block
    q = torch.randn(B, Hq, T, hd, generator=g).to(dtype)
    k = torch.randn(B, Hkv, T, hd, generator=g).to(dtype)
    v = torch.randn(B, Hkv, T, hd, generator=g).to(dtype)
    Qb, cap = T // block, 3
    lists = torch.randint(0, Qb, (B, Qb, cap), generator=g, dtype=torch.int32)
    counts = torch.randint(0, cap + 1, (B, Qb), generator=g, dtype=torch.int32)
    W = 2 * block
    scale = hd ** -0.5
    out = fsi.sparse_attention(q.to(dev), k.to(dev), v.to(dev), lists.to(dev), counts.to(dev), block=block,
                               mode=mode, window=W, scale=scale)
    if mode == 0:
        wts = A.sparse_mask(B, T, W, block, lists, counts)
    else:
        wts = A.block_list_weights(B, T, block, lists, counts)
    ref = A.weighted_attention_f64(q.float(), k.float(), v.float(), wts, scale)
    tol = 1e-5 if dtype == torch.float32 else 4e-3
    assert out.dtype == dtype and Pt.rel_l2(out.cpu().float(), ref.float()) <= tol
