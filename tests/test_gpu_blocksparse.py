"""GPU parity of the block-sparse MFMA GEMM engine: column-block sparse linear,
2-D tile-sparse matmul, the Pattention prefill path, and the BlockSparseLinear /
BlockwiseMatMul2D modules.  bf16 bar: rel-L2 <= 2e-3 against fp64."""
import pytest
import torch

from oracle import blocksparse as BS
from oracle import pattention as P
from oracle import routing as R
from route_check import check_rows, tolerances

pytestmark = pytest.mark.gpu

TOL = 2e-3


def _rel(got, ref):
    return P.rel_l2(got.float().cpu(), ref.float())


BSL_CASES = [
    (1, 64, 256, 64, [3, 0], False),
    (100, 256, 512, 32, [15, 2, 7, 9], True),
    (300, 1000, 384, 128, [1, 2], True),
    (257, 128, 1024, 64, list(range(16)), False),
    (64, 512, 256, 64, [], True),
]


@pytest.mark.parametrize("M,K,N,bs,active,bias", BSL_CASES)
def test_block_sparse_linear(fsi, dev, M, K, N, bs, active, bias):
    print(f"[case] block_sparse_linear M={M} K={K} N={N} bs={bs} n_active={len(active)}", flush=True)
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    b = torch.randn(N, generator=g).bfloat16() if bias else None
    act = torch.tensor(active, dtype=torch.int32)
    out = fsi.triton_block_sparse_linear(x.to(dev), w.to(dev), None if b is None else b.to(dev), act.to(dev),
                                         block_size=bs).cpu()
    ref = BS.block_sparse_linear_f64(x, w, b, active, bs)
    inactive = torch.ones(N, dtype=torch.bool)
    for a in active:
        inactive[a * bs:(a + 1) * bs] = False
    assert torch.all(out[:, inactive] == 0)
    if active:
        assert _rel(out, ref) <= TOL


def test_block_sparse_linear_bad_block_reported(fsi, dev, monkeypatch):
    x = torch.randn(8, 64).bfloat16().to(dev)
    w = torch.randn(128, 64).bfloat16().to(dev)
    monkeypatch.setenv("FSI_CHECK", "1")
    with pytest.raises(IndexError):
        fsi.triton_block_sparse_linear(x, w, None, torch.tensor([5], dtype=torch.int32, device=dev), block_size=64)


BW_CASES = [
    (256, 512, 512, 128, 128, 0.25, 1),
    (384, 512, 256, 64, 64, 0.3, 3),
    (200, 256, 512, 64, 128, 0.5, 1),
    (512, 1024, 1024, 128, 128, 0.1, 4),
    (256, 512, 384, 32, 16, 0.3, 2),       # 32-wide k blocks, 8 n blocks per 128-column tile
    (130, 256, 320, 64, 32, 0.4, 1),       # ragged M and N (N % 128 == 64)
    (256, 8192, 256, 32, 128, 0.6, 1),     # ~150 active k blocks per tile: list read 64 at a time
    (128, 16384, 256, 32, 256, 0.05, 1),   # 512 k blocks: two rounds of the list build; 256-wide n blocks
    (384, 1024, 512, 128, 64, 0.0, 3),     # empty masks: every tile stores zeros
    (256, 512, 512, 64, 128, 1.0, 2),      # dense masks
    (96, 192, 96, 64, 48, 0.5, 1),         # n block dividing neither way: generic kernel
    (4608, 512, 2048, 128, 128, 0.3, 36),  # 576 tiles: heaviest-first tile order from the pre-pass
    (4096, 256, 2304, 32, 64, 0.25, 4),    # 576 tiles, 2 n blocks per tile, 8 m tiles per group
    (4200, 256, 2176, 64, 128, 0.5, 3),    # 561 tiles, ragged M, with the tile order
]


@pytest.mark.parametrize("M,K,N,bk,bn,density,groups", BW_CASES)
def test_blockwise_matmul(fsi, dev, M, K, N, bk, bn, density, groups):
    print(f"[case] blockwise_matmul M={M} K={K} N={N} tile={bk}x{bn} d={density} groups={groups}", flush=True)
    g = torch.Generator().manual_seed(K + N)
    x = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    T = (K // bk) * (N // bn)
    masks = torch.rand(groups, T, generator=g) < density
    rpg = -(-M // groups) if groups > 1 else M
    rpg = -(-rpg // 128) * 128 if groups > 1 else rpg
    out = fsi.blockwise_matmul(x.to(dev), w.to(dev), masks.to(dev), bk, bn, rows_per_group=rpg).cpu()
    ref = BS.blockwise_matmul_f64(x, w, masks, bk, bn, rpg)
    if not masks.any():
        assert torch.equal(out, torch.zeros_like(out))
        return
    assert _rel(out, ref) <= TOL


# fp32 (the reference modules' default dtype): the list-driven tile kernel on
# v_mfma_f32_16x16x4_f32 where the tiling fits it (k blocks of 16-multiples), the
# generic kernel otherwise (k blocks of 8, n blocks of 48, K = 1000).  fp32 bar:
# rel-L2 <= 1e-5 against fp64.
TOL_F32 = 1e-5


@pytest.mark.parametrize("M,K,N,bk,bn,density,groups", BW_CASES + [
    (256, 512, 384, 16, 16, 0.3, 2),       # 16-wide k blocks: one fp32 K-step each
    (192, 256, 256, 8, 64, 0.5, 1),        # 8-wide k blocks: generic kernel
])
def test_blockwise_matmul_f32(fsi, dev, M, K, N, bk, bn, density, groups):
    print(f"[case] blockwise_matmul fp32 M={M} K={K} N={N} tile={bk}x{bn} d={density} groups={groups}", flush=True)
    g = torch.Generator().manual_seed(K + N + 1)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.05
    T = (K // bk) * (N // bn)
    masks = torch.rand(groups, T, generator=g) < density
    rpg = -(-M // groups) if groups > 1 else M
    rpg = -(-rpg // 128) * 128 if groups > 1 else rpg
    out = fsi.blockwise_matmul(x.to(dev), w.to(dev), masks.to(dev), bk, bn, rows_per_group=rpg).cpu()
    assert out.dtype == torch.float32
    ref = BS.blockwise_matmul_f64(x, w, masks, bk, bn, rpg)
    if not masks.any():
        assert torch.equal(out, torch.zeros_like(out))
        return
    assert _rel(out, ref) <= TOL_F32


@pytest.mark.parametrize("M,K,N,bs,active,bias", BSL_CASES + [(130, 4096, 512, 16, [0, 5, 31], True)])
def test_block_sparse_linear_f32(fsi, dev, M, K, N, bs, active, bias):
    print(f"[case] block_sparse_linear fp32 M={M} K={K} N={N} bs={bs} n_active={len(active)}", flush=True)
    g = torch.Generator().manual_seed(M + K + 1)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.05
    b = torch.randn(N, generator=g) if bias else None
    act = torch.tensor(active, dtype=torch.int32)
    out = fsi.triton_block_sparse_linear(x.to(dev), w.to(dev), None if b is None else b.to(dev), act.to(dev),
                                         block_size=bs).cpu()
    ref = BS.block_sparse_linear_f64(x, w, b, active, bs)
    inactive = torch.ones(N, dtype=torch.bool)
    for a in active:
        inactive[a * bs:(a + 1) * bs] = False
    assert torch.all(out[:, inactive] == 0)
    if active:
        assert _rel(out, ref) <= TOL_F32


@pytest.mark.parametrize("M,rounding", [(300, "fused"), (512, "eager"), (256, "fp32")])
def test_pattention_prefill_gemm_path(fsi, dev, M, rounding):
    """M >= 256 with SwiGLU and down_proj-layout V takes the MFMA GEMM path."""
    print(f"[case] prefill gemm M={M} {rounding}", flush=True)
    g = torch.Generator().manual_seed(M)
    D, N_p = 512, 2048
    x = torch.randn(M, D, generator=g).bfloat16()
    kg = (torch.randn(N_p, D, generator=g) * 0.02).bfloat16()
    ku = (torch.randn(N_p, D, generator=g) * 0.02).bfloat16()
    wd = (torch.randn(D, N_p, generator=g) * 0.02).bfloat16()  # down_proj layout; v = wd.t()
    active = torch.tensor([5, 0, 31, 7, 12, 3], dtype=torch.int32)
    vt = wd.to(dev).t()
    got = fsi.pattention_forward(x.to(dev), kg.to(dev), ku.to(dev), vt, active.to(dev), 64, "swiglu", rounding).cpu()
    if rounding == "fp32":
        ref = P.pattention_fp32_act(x, kg, wd.t().contiguous(), ku, active, "swiglu", 64)
    else:
        ref = P.mlp_eval_forward(x, kg, ku, wd.t().contiguous(), active, 64, fused=(rounding == "fused"))
    assert _rel(got, ref) <= TOL


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_sparse_linear_module(fsi, dev, dtype):
    """BlockSparseLinear eval (block_matmul.py:131-282): the selected block set
    against the oracle's eval selection on the module's own scores (exact, except
    a token whose sorted mass sits within 1e-5 of top_p at its boundary), and the
    output against the oracle forward."""
    import copy

    torch.manual_seed(0)
    m = fsi.BlockSparseLinear(256, 1024, block_size=64, base_blocks=2, top_p=0.9, max_remote_blocks=4, bias=True,
                              dtype=dtype).eval()
    x = torch.randn(2, 5, 256).to(dtype)
    with torch.no_grad():
        ref, _ = BS.block_sparse_forward(m, x)
        md = copy.deepcopy(m).to(dev)
        out, aux = md(x.to(dev))
        kb, _ = md.get_block_keys_and_values()
        scores = md.indexer.compute_block_scores(md.indexer.compute_query_16d(x.to(dev)), kb.expand(2, -1, -1))
        active_gpu, _ = fsi.block_matmul._eval_active_blocks(scores, 2, 0.9, 4, 16)
    active_ora = BS.eval_active_blocks(scores.cpu(), 2, 0.9, 4, 16)
    assert aux["active_blocks_union"] == active_gpu.numel()
    if dtype == torch.float32:
        probs = torch.softmax(scores.cpu()[..., 2:].double(), dim=-1)
        cum = probs.sort(dim=-1, descending=True).values.cumsum(-1)
        near = bool(((cum - 0.9).abs() <= 1e-5).any())
        if not near:
            assert active_gpu.tolist() == active_ora.tolist()
        assert _rel(out, ref) <= 1e-5
    else:
        # bf16 probabilities tie often: per token, every ranked slot and count
        # equals the oracle's (block_matmul.py:169-185 is select_blocks with no
        # local window, K_min 0) except where bf16 values tie or the running mass
        # sits at top_p within bf16 rounding; the union is the GPU rows' union
        kw = dict(causal=False, local_window_blocks=0, top_p=0.9, min_remote_blocks=0, max_remote_blocks=4,
                  remote_capacity=4)
        with torch.no_grad():
            r = fsi.select_blocks(scores[..., 2:].contiguous(), **kw)
        ora = R.select_route(scores.cpu()[..., 2:].contiguous(), **kw)
        remote = torch.ones(scores.shape[1], 14, dtype=torch.bool)
        bad = check_rows(r.remote_indices, r.remote_counts, ora, remote, *tolerances(torch.bfloat16))
        assert not bad, bad
        union = set(range(2))
        for b in range(2):
            for t in range(5):
                union |= {int(i) + 2 for i in r.remote_indices[b, t, :int(r.remote_counts[b, t])].tolist()}
        assert active_gpu.tolist() == sorted(union)
        if torch.equal(r.remote_counts.cpu(), ora["remote_counts"]) and torch.equal(
                r.remote_indices.cpu(), ora["remote_indices"]):
            assert active_gpu.tolist() == active_ora.tolist()
        assert _rel(out, ref) <= 1e-2


def test_blockwise_matmul_module(fsi, dev):
    torch.manual_seed(1)
    m = fsi.BlockwiseMatMul2D(256, 512, block_k=64, block_n=64, base_tiles_ratio=0.1, top_p=0.5,
                              dtype=torch.bfloat16).eval()
    x = torch.randn(2, 3, 256).bfloat16()
    with torch.no_grad():
        md = m.to(dev)
        xd = x.to(dev)
        out, aux = md(xd)
        mask, probs, scores, tile_v = md.route_tiles(xd)
        ref = BS.blockwise_matmul_f64(x.reshape(-1, 256), m.weight.detach().cpu(), mask.cpu(), 64, 64, 6)
        ctx = (probs.to(tile_v.dtype).reshape(-1, m.total_tiles) @ tile_v).view(2, 3, 16)
        ref = ref.view(2, 3, 512) + md.out_proj(ctx).double().cpu()
    assert aux["active_tiles"] == int(mask.sum())
    assert _rel(out, ref) <= 1e-2


@pytest.mark.parametrize("bn,density,dtype", [(128, 0.25, torch.bfloat16), (64, 0.4, torch.bfloat16),
                                             (128, 0.0, torch.bfloat16), (64, 0.4, torch.float32)])
def test_blockwise_matmul_tile_order_matches_dispatch_order(fsi, dev, bn, density, dtype):
    """Above 512 output tiles the workspace receives a tile order, heaviest first
    inside each 128-row band; without a workspace the tiles run in dispatch order.
    Both give the same bits (each tile's result does not depend on the workgroup
    that computes it) and match the fp64 reference.  Group masks range from empty
    to dense."""
    print(f"[case] tile order bn={bn} density={density}", flush=True)
    from foveal_sparse_indexer_amd import _lib
    g = torch.Generator().manual_seed(bn + int(density * 100))
    M, K, N, bk, groups = 5120, 512, 2048, 64, 20
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) * 0.05).to(dtype)
    T = (K // bk) * (N // bn)
    dens = torch.linspace(0.0, 1.0, groups).unsqueeze(1) if density > 0 else torch.zeros(groups, 1)
    masks = torch.rand(groups, T, generator=g) < dens
    rpg = M // groups
    xd, wd, md = x.to(dev), w.to(dev), masks.to(dev)
    ordered = fsi.blockwise_matmul(xd, wd, md, bk, bn, rows_per_group=rpg)
    L = _lib.lib()
    m8 = md.to(torch.uint8).contiguous()
    plain = torch.empty_like(ordered)
    st = L.fsi_blockwise_matmul(xd.data_ptr(), K, wd.data_ptr(), K, m8.data_ptr(), groups, rpg, bk, bn, M, N, K,
                                _lib.dtype_code(xd.dtype, "blockwise_matmul"), plain.data_ptr(), N, None, 0,
                                _lib.stream_handle(dev))
    _lib.check(st, "blockwise_matmul")
    torch.cuda.synchronize(dev)
    assert torch.equal(ordered, plain)
    if masks.any():
        tol = TOL_F32 if dtype == torch.float32 else TOL
        assert _rel(ordered, BS.blockwise_matmul_f64(x, w, masks, bk, bn, rpg)) <= tol
    else:
        assert torch.equal(ordered.cpu(), torch.zeros(M, N, dtype=dtype))


def test_blockwise_matmul_graph_replays(fsi, dev):
    """The tile-sparse GEMM (k-block lists built on chip) captured in a graph and
    replayed with eager work in between, the mask changed in place between
    replays: every replay equals an eager call on the same mask."""
    g = torch.Generator().manual_seed(5)
    M, K, N, T = 256, 1024, 512, 128
    x = torch.randn(M, K, generator=g).bfloat16().to(dev)
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16().to(dev)
    masks = torch.rand(2, (K // T) * (N // T), generator=g) < 0.4
    mask = masks.to(dev)
    with torch.no_grad():
        outs = {}
        graph = torch.cuda.CUDAGraph()
        st = torch.cuda.Stream(dev)
        st.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(st), torch.cuda.graph(graph, stream=st):
            outs["y"] = fsi.blockwise_matmul(x, w, mask, T, T, rows_per_group=T)
        torch.cuda.synchronize(dev)
        for r in range(3):
            if r == 2:
                mask.copy_((torch.rand(2, (K // T) * (N // T), generator=g) < 0.7).to(dev))
            graph.replay()
            torch.cuda.synchronize(dev)
            eager = fsi.blockwise_matmul(x, w, mask, T, T, rows_per_group=T)
            assert torch.equal(outs["y"], eager)
            torch.randn(1024, 1024, device=dev).sum().item()  # eager work between replays
