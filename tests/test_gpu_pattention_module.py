"""FovealPattentionMLP module contract on the GPU beyond the kernels:
  * eval-mode gradients reach the input (the reference's eval path runs F.linear
    on detached weight copies, foveal_pattention.py:115-122, 278-288) and no weight;
  * the packed-weight copy follows weight changes made through `.data`
    (invalidate_packed_weights), load_state_dict and module moves;
  * the reference's cache attributes _cached_kg / _cached_ku / _cached_v;
  * NaN router scores rank first, as torch.topk ranks them, and every slot of the
    active list is written.
"""
import pytest
import torch

from oracle import pattention as P
from oracle import routing as R

pytestmark = pytest.mark.gpu


def _mlp(fsi, dev, dtype=torch.bfloat16, D=256, N_p=1024, base=2, remote=6, seed=0):
    torch.manual_seed(seed)
    m = fsi.FovealPattentionMLP(hidden_dim=D, intermediate_dim=N_p, base_blocks=base, remote_blocks=remote,
                                dtype=dtype).to(dev).eval()
    with torch.no_grad():
        for p in (m.k_gate, m.k_up, m.v):
            p.normal_(0.0, 0.05)
    return m


def _cpu(m):
    return {k: v.detach().cpu() for k, v in m.state_dict().items()}


@pytest.mark.parametrize("dtype,M", [(torch.bfloat16, 8), (torch.bfloat16, 300), (torch.float32, 12)])
def test_eval_input_gradient(fsi, dev, dtype, M):
    m = _mlp(fsi, dev, dtype)
    x = torch.randn(M, 1, 256, dtype=dtype)
    xd = x.to(dev).requires_grad_()
    out = m(xd)
    assert out.grad_fn is not None
    dy = torch.randn(M, 1, 256, dtype=dtype)
    out.backward(dy.to(dev))
    assert m.k_gate.grad is None and m.v.grad is None  # the reference's eval path detaches the weights
    sd = _cpu(m)
    active = m._cached_active_blocks.cpu()
    idx = P.channel_index(active, 64)
    xr = x.reshape(M, 256).double().requires_grad_()
    kg, ku, v = sd["k_gate"].double()[idx], sd["k_up"].double()[idx], sd["v"].double()[idx]
    g, u = xr @ kg.t(), xr @ ku.t()
    yr = (torch.nn.functional.silu(g) * u) @ v
    yr.backward(dy.reshape(M, 256).double())
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert P.rel_l2(xd.grad.reshape(M, 256).cpu(), xr.grad) <= tol
    assert P.rel_l2(out.detach().reshape(M, 256).cpu(), yr.detach()) <= tol


def test_packed_weights_follow_data_writes_and_state_dict(fsi, dev):
    m = _mlp(fsi, dev)
    x = torch.randn(8, 1, 256).bfloat16()
    with torch.no_grad():
        m(x.to(dev))
        assert m._packed is not None
        m.k_gate.data.mul_(2.0)  # no version bump: the packed copy must be refreshed explicitly
        m.invalidate_packed_weights()
        out = m(x.to(dev)).cpu()
    sd = _cpu(m)
    active = m._cached_active_blocks.cpu()
    ref = P.mlp_eval_forward(x.reshape(8, 256), sd["k_gate"], sd["k_up"], sd["v"], active, 64, fused=True)
    assert P.rel_l2(out.reshape(8, 256), ref) <= 2e-3
    # load_state_dict drops the packed copy by itself
    m2 = _mlp(fsi, dev, seed=5)
    with torch.no_grad():
        m(x.to(dev))
        m.load_state_dict(m2.state_dict())
        m.set_active_blocks(active)
        out = m(x.to(dev)).cpu()
    sd = _cpu(m2)
    ref = P.mlp_eval_forward(x.reshape(8, 256), sd["k_gate"], sd["k_up"], sd["v"], active, 64, fused=True)
    assert P.rel_l2(out.reshape(8, 256), ref) <= 2e-3


def test_reference_cache_attributes(fsi, dev):
    m = _mlp(fsi, dev)
    assert m._cached_kg is None and m._cached_v is None
    x = torch.randn(4, 1, 256, device=dev).bfloat16()
    with torch.no_grad():
        m(x)
    idx = (m._cached_active_blocks.long()[:, None] * 64 + torch.arange(64, device=dev)).flatten()
    assert torch.equal(m._cached_kg, m.k_gate[idx]) and torch.equal(m._cached_ku, m.k_up[idx])
    assert torch.equal(m._cached_v, m.v[idx]) and m._cached_v.is_contiguous()
    m._cached_kg = None  # the reference's way to force re-routing
    assert m._cached_active_blocks is None and m._cached_ku is None
    with pytest.raises(AttributeError):
        m._cached_kg = torch.zeros(1)


def test_router_nan_scores_rank_first(fsi, dev):
    """Blocks whose key is NaN score NaN; torch.topk ranks NaN above every number,
    so they come first (in block order) and every slot is a valid block id."""
    m = _mlp(fsi, dev, D=128, N_p=640, base=2, remote=5)
    with torch.no_grad():
        m.block_keys_16d[7] = float("nan")
        m.block_keys_16d[4] = float("nan")
        x = torch.randn(3, 128, device=dev).bfloat16()
        active = fsi.mlp_pooled_route(x, m.q_proj_16d.weight, m.block_keys_16d, 2, 5).cpu()
    assert active[:4].tolist() == [0, 1, 4, 7]
    assert len(set(active.tolist())) == 7 and int(active.min()) >= 0 and int(active.max()) < 10
