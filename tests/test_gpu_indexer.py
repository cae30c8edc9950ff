"""GPU parity of the indexer-representation kernels (rms_norm, block pooling,
block scores, additive context) and of the FovealIndexer module.

fp32: within 1e-6 relative (+1e-7 absolute) of the oracle; bf16: within one
bf16 ulp per element (rounding of values the CPU and GPU compute a few fp32 ulp
apart can land on either side)."""
import pytest
import torch

from oracle import indexer as IX
from oracle import routing as R

pytestmark = pytest.mark.gpu


def _close(got, ref, rtol=1e-6, atol=1e-7):
    got, ref = got.cpu(), ref.cpu()
    assert got.dtype == ref.dtype and got.shape == ref.shape
    if ref.dtype == torch.bfloat16:
        d = (got.float() - ref.float()).abs()
        assert bool((d <= ref.float().abs() * 2.0 ** -7 + 1e-30).all()), float(d.max())
    else:
        assert torch.allclose(got, ref, rtol=rtol, atol=atol), float((got - ref).abs().max())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_index_rms_norm(fsi, dev, dtype):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(3, 77, 16, generator=g) * 2).to(dtype)
    _close(fsi.index_rms_norm(x.to(dev)), IX.rms_norm16(x))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("bs", [4, 64])
def test_pool_kv(fsi, dev, dtype, bs):
    g = torch.Generator().manual_seed(bs)
    B, N = 2, bs * 9
    k = (torch.randn(B, N, 16, generator=g) * 0.7).to(dtype)
    v = torch.randn(B, N, 16, generator=g).to(dtype)
    from foveal_sparse_indexer_amd import _lib

    kd, vd = k.to(dev), v.to(dev)  # keep the device copies alive until the kernel has run
    kb = torch.empty(B, 9, 16, dtype=dtype, device=dev)
    vb = torch.empty_like(kb)
    st = _lib.lib().fsi_index_pool_kv(kd.data_ptr(), vd.data_ptr(), _lib.dtype_code(dtype, "t"), B, N, 16, bs,
                                      kb.data_ptr(), vb.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, "pool")
    rk, rv = IX.pool_kv(k, v, bs)
    _close(kb, rk)
    _close(vb, rv)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_block_scores(fsi, dev, dtype):
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 70, 16, generator=g).to(dtype)
    k = torch.randn(2, 300, 16, generator=g).to(dtype)
    _close(fsi.block_scores(q.to(dev), k.to(dev)), IX.block_scores(q, k))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("causal", [True, False])
def test_additive_context(fsi, dev, dtype, causal):
    from foveal_sparse_indexer_amd import _lib

    g = torch.Generator().manual_seed(6)
    B, Qb, Nb = 2, 33, 40
    s = (torch.randn(B, Qb, Nb, generator=g) * 2).to(dtype)
    v = torch.randn(B, Nb, 16, generator=g).to(dtype)
    sd, vd = s.to(dev), v.to(dev)
    ctx = torch.empty(B, Qb, 16, dtype=dtype, device=dev)
    st = _lib.lib().fsi_additive_context(sd.data_ptr(), vd.data_ptr(), _lib.dtype_code(dtype, "t"), B, Qb, Nb, 16,
                                         int(causal), ctx.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, "ctx")
    ref = IX.additive_context(s, v, causal)
    got = ctx.cpu()
    if dtype == torch.bfloat16:
        err = (got.float() - ref.float()).norm() / ref.float().norm()
        assert float(err) <= 2e-3
    else:
        assert torch.allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_foveal_indexer_module(fsi, dev):
    """compute_query_16d / compute_kv_blocks_16d / compute_block_scores / route /
    additive_stream against the oracle composed with the same projections.  The
    D -> 16 projections are library GEMMs whose fp32 summation order differs
    from the CPU's, so the comparison allows 2e-5 relative."""
    torch.manual_seed(0)
    m = fsi.FovealIndexer(hidden_size=64, block_size=8, local_window_blocks=2, top_p=0.9, max_remote_blocks=4,
                          remote_capacity=4).eval()
    x = torch.randn(2, 64, 64)
    with torch.no_grad():
        md = m.to(dev)
        xd = x.to(dev)
        q = md.compute_query_16d(xd)
        kb, vb = md.compute_kv_blocks_16d(xd)
        qb = q[:, ::8]
        s = md.compute_block_scores(qb, kb)
        route = md.route(s)
        add = md.additive_stream(s, vb)
        mc = m.cpu()
        rq = IX.rms_norm16(mc.q_proj(x))
        rk, rv = IX.pool_kv(mc.k_proj(x), mc.v_proj(x), 8)
    _close(q, rq, 2e-5, 2e-6)
    _close(kb, rk, 2e-5, 2e-6)
    _close(vb, rv, 2e-5, 2e-6)
    rs = IX.block_scores(rq[:, ::8], rk)
    assert torch.allclose(s.cpu(), rs, rtol=1e-5, atol=1e-6)
    ora = R.select_route(s.cpu(), causal=True, local_window_blocks=2, top_p=0.9, max_remote_blocks=4,
                         remote_capacity=4)
    from route_check import check_rows

    _, _, remote = R.route_masks(8, 8, True, 2)
    assert not check_rows(route.remote_indices, route.remote_counts, ora, remote, 1e-6, 1e-5)
    ref_add = mc.out_proj(IX.additive_context(s.cpu(), vb.cpu(), True)).repeat_interleave(8, dim=1)
    assert torch.allclose(add.cpu(), ref_add, rtol=1e-4, atol=1e-7)
    assert add.shape == (2, 64, 64)


def test_block_sparse_linear_gradients_bf16(fsi, dev):
    """The bf16 MFMA forward of block_sparse_linear records autograd: gradients of
    x, weight and bias match the fp64 gather -> linear -> scatter product
    (block_matmul.py:215-232) on the active column blocks."""
    g = torch.Generator().manual_seed(4)
    w = (torch.randn(256, 128, generator=g) * 0.1).bfloat16()
    b = torch.randn(256, generator=g).bfloat16()
    x = torch.randn(40, 128, generator=g).bfloat16()
    active = torch.tensor([0, 3], dtype=torch.int32)
    wd, bd, xd = (t.to(dev).requires_grad_() for t in (w, b, x))
    y = fsi.block_sparse_linear(xd, wd, bd, active.to(dev), 64)
    dy = torch.randn(40, 256, generator=g).bfloat16()
    y.backward(dy.to(dev))
    wr, br, xr = (t.double().requires_grad_() for t in (w, b, x))
    cols = torch.cat([torch.arange(0, 64), torch.arange(192, 256)])
    yr = torch.zeros(40, 256, dtype=torch.float64)
    yr[:, cols] = xr @ wr[cols].t() + br[cols]
    yr.backward(dy.double())
    for got, want in ((y, yr), (xd.grad, xr.grad), (wd.grad, wr.grad), (bd.grad, br.grad)):
        err = (got.detach().double().cpu() - want).norm() / want.norm()
        assert err <= 1e-2
    assert not wd.grad[64:192].any() and not bd.grad[64:192].any()
