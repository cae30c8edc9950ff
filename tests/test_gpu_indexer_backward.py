"""GPU parity of the indexer backward kernels (fsi_index_rms_norm_bwd,
fsi_index_pool_kv_bwd, fsi_block_scores_bwd, fsi_additive_context_bwd,
fsi_masked_softmax_bwd) against fp64 autograd of the oracle restatement, and the
reference's own gradient test (tests/test_indexer.py:63-101) run on the GPU.

Inputs are drawn in the test dtype and the oracle runs in fp64 on the same
values.  Tolerances (relative L2 over the gradient tensor): fp32 <= 1e-5 for the
kernels, 1e-4 for the module (library GEMMs in the projections); bf16 <= 1e-2
(the forward's bf16 rounding points move the operands by up to 2^-9)."""
import pytest
import torch

from oracle import indexer as IX
from oracle import routing as R

pytestmark = pytest.mark.gpu

F64 = torch.float64
DTYPES = [torch.float32, torch.bfloat16]
IDS = ["f32", "bf16"]


def _tol(dtype):
    return 1e-5 if dtype == torch.float32 else 1e-2


def _rel(got, ref):
    got, ref = got.detach().cpu().double(), ref.detach().cpu().double()
    assert got.shape == ref.shape
    return ((got - ref).norm() / ref.norm().clamp_min(1e-300)).item()


def _leaf(t, dev=None):
    return (t.to(dev) if dev is not None else t.double()).detach().requires_grad_()


def _rand(shape, g, dtype, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_index_rms_norm_backward(fsi, dev, dtype):
    g = torch.Generator().manual_seed(0)
    x = _rand((3, 77, 16), g, dtype, 2.0)
    dy = _rand((3, 77, 16), g, dtype)
    xg = _leaf(x, dev)
    fsi.index_rms_norm(xg).backward(dy.to(dev))
    xr = _leaf(x)
    IX.rms_norm16(xr).backward(dy.double())
    assert xg.grad.dtype == dtype
    assert _rel(xg.grad, xr.grad) <= _tol(dtype)


@pytest.mark.parametrize("bs", [1, 8, 64, 100])
@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_pool_kv_backward(fsi, dev, dtype, bs):
    g = torch.Generator().manual_seed(bs)
    k = _rand((2, bs * 5, 16), g, dtype)
    v = _rand((2, bs * 5, 16), g, dtype)
    gk = _rand((2, 5, 16), g, dtype)
    gv = _rand((2, 5, 16), g, dtype)
    kg, vg = _leaf(k, dev), _leaf(v, dev)
    kb, vb = fsi.core._PoolKVFn.apply(kg, vg, bs)
    ((kb * gk.to(dev)).sum() + (vb * gv.to(dev)).sum()).backward()
    kr, vr = _leaf(k), _leaf(v)
    rkb, rvb = IX.pool_kv(kr, vr, bs, F64)
    ((rkb * gk.double()).sum() + (rvb * gv.double()).sum()).backward()
    assert _rel(kg.grad, kr.grad) <= _tol(dtype)
    assert _rel(vg.grad, vr.grad) <= _tol(dtype)
    # only the keys used: the value gradient is exactly zero
    kg2, vg2 = _leaf(k, dev), _leaf(v, dev)
    fsi.core._PoolKVFn.apply(kg2, vg2, bs)[0].sum().backward()
    assert vg2.grad is None or not vg2.grad.any()


@pytest.mark.parametrize("Q,N", [(37, 70), (130, 200), (1, 1), (64, 64)])
@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_block_scores_backward(fsi, dev, dtype, Q, N):
    g = torch.Generator().manual_seed(Q * 1000 + N)
    q = _rand((2, Q, 16), g, dtype)
    k = _rand((2, N, 16), g, dtype)
    ds = _rand((2, Q, N), g, dtype)
    qg, kg = _leaf(q, dev), _leaf(k, dev)
    fsi.block_scores(qg, kg).backward(ds.to(dev))
    qr, kr = _leaf(q), _leaf(k)
    IX.block_scores(qr, kr, F64).backward(ds.double())
    assert _rel(qg.grad, qr.grad) <= _tol(dtype)
    assert _rel(kg.grad, kr.grad) <= _tol(dtype)


@pytest.mark.parametrize("Q,N", [(70, 130), (130, 70), (3, 1), (200, 200)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_additive_context_backward(fsi, dev, dtype, causal, Q, N):
    g = torch.Generator().manual_seed(Q + N + causal)
    s = _rand((2, Q, N), g, dtype, 2.0)
    v = _rand((2, N, 16), g, dtype)
    dc = _rand((2, Q, 16), g, dtype)
    sg, vg = _leaf(s, dev), _leaf(v, dev)
    ctx = fsi.core._AdditiveContextFn.apply(sg, vg, causal)
    ctx.backward(dc.to(dev))
    sr, vr = _leaf(s), _leaf(v)
    IX.additive_context(sr, vr, causal, F64).backward(dc.double())
    assert _rel(sg.grad, sr.grad) <= _tol(dtype)
    assert _rel(vg.grad, vr.grad) <= _tol(dtype)
    if causal:  # masked entries (key >= query block) get exactly zero
        qi = torch.arange(Q).view(Q, 1)
        ni = torch.arange(N).view(1, N)
        assert not sg.grad.cpu()[:, (ni >= qi)].any()


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_masked_softmax_backward(fsi, dev, dtype):
    g = torch.Generator().manual_seed(5)
    s = _rand((3, 5, 300), g, dtype, 3.0)
    mask = torch.rand(5, 300, generator=g) > 0.3
    mask[2] = False  # an all-masked row
    dp = _rand((3, 5, 300), g, dtype)
    sg = _leaf(s, dev)
    fsi.masked_softmax(sg, mask.to(dev)).backward(dp.to(dev))
    sr = _leaf(s)
    R.masked_probs(sr, mask.expand(3, 5, 300), F64).backward(dp.double())
    assert _rel(sg.grad, sr.grad) <= _tol(dtype)
    assert not sg.grad[:, 2].any() and not sg.grad.cpu()[:, ~mask].any()
    # 2-D scores go through the (B*Q, 1, N) view
    s2, m2, d2 = _rand((7, 50), g, dtype), torch.rand(7, 50, generator=g) > 0.5, _rand((7, 50), g, dtype)
    sg2 = _leaf(s2, dev)
    fsi.masked_softmax(sg2, m2.to(dev)).backward(d2.to(dev))
    sr2 = _leaf(s2)
    R.masked_probs(sr2, m2, F64).backward(d2.double())
    assert _rel(sg2.grad, sr2.grad) <= _tol(dtype)


@pytest.mark.parametrize("hidden,seq,block", [(32, 32, 16), (64, 256, 16), (48, 512, 64)])
def test_foveal_indexer_gradients(fsi, dev, hidden, seq, block):
    """tests/test_indexer.py:63-101 on the GPU, with every gradient compared to
    the same graph built from the oracle functions on the CPU (fp32 model, fp64
    oracle)."""
    torch.manual_seed(hidden + seq)
    m = fsi.FovealIndexer(hidden_size=hidden, index_dim=16, block_size=block, local_window_blocks=1, top_p=0.9,
                          use_additive_stream=True)
    x = torch.randn(2, seq, hidden)
    nb = seq // block
    teacher = torch.rand(2, nb, nb)
    teacher[0, 0, 0] = 1.0

    md = fsi.FovealIndexer(hidden_size=hidden, index_dim=16, block_size=block, local_window_blocks=1, top_p=0.9,
                           use_additive_stream=True)
    md.load_state_dict(m.state_dict())
    md = md.to(dev)
    xd = x.to(dev).requires_grad_()
    q_16d = md.compute_query_16d(xd)
    assert q_16d.shape == (2, seq, 16)
    k_b, v_b = md.compute_kv_blocks_16d(xd)
    assert k_b.shape == (2, nb, 16) and v_b.shape == (2, nb, 16)
    scores = md.compute_block_scores(q_16d[:, ::block], k_b)
    assert scores.shape == (2, nb, nb)
    md.route(scores)  # routing consumes detached scores
    add_out = md.additive_stream(scores, v_b)
    assert add_out.shape == (2, seq, hidden)
    distill = md.distillation_loss(scores, teacher.to(dev))
    assert distill.item() >= 0.0
    (add_out.sum() + distill).backward()

    mr = m.double()
    xr = x.double().requires_grad_()
    rq = IX.rms_norm16(mr.q_proj(xr))
    rk, rv = IX.pool_kv(mr.k_proj(xr), mr.v_proj(xr), block, F64)
    rs = IX.block_scores(rq[:, ::block], rk, F64)
    radd = mr.out_proj(IX.additive_context(rs, rv, True, F64)).repeat_interleave(block, dim=1)
    rdist = IX.distillation_loss(rs, teacher.double(), causal=True, temperature=mr.distill_temperature, acc=F64)
    (radd.sum() + rdist).backward()

    assert _rel(add_out, radd) <= 1e-4
    assert abs(distill.item() - rdist.item()) <= 1e-4 * max(1.0, abs(rdist.item()))
    assert _rel(xd.grad, xr.grad) <= 1e-4
    for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
        got = getattr(md, name).weight.grad
        assert got is not None, name
        assert _rel(got, getattr(mr, name).weight.grad) <= 1e-4, name


def test_block_sparse_linear_block_keys_backward(fsi, dev):
    """BlockSparseLinear.get_block_keys_and_values (block_matmul.py:109-128) is
    differentiable in the weight and its two 16-D projections."""
    torch.manual_seed(1)
    lin = fsi.BlockSparseLinear(128, 256, block_size=64).to(dev, torch.bfloat16)
    kb, vb = lin.get_block_keys_and_values()
    assert kb.shape == (1, 4, 16) and vb.shape == (1, 4, 16)
    (kb.float().sum() + vb.float().square().sum()).backward()
    assert lin.weight.grad is not None and lin.weight.grad.abs().sum() > 0
    assert lin.weight_to_k.weight.grad is not None and lin.weight_to_v.weight.grad is not None
