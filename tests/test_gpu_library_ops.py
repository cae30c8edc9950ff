"""torch.library registration on the GPU: torch.library.opcheck (schema, fake
tensor, AOT dispatch with dynamic shapes) on the hot-path ops with real inputs,
and torch.compile (aot_eager, whole graph) of a routed decode step and of a
differentiable indexer loss, compared with eager execution (same kernels, so
the results are identical)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bf(*shape, scale=1.0, seed=0, dev="cuda"):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(*shape, device=dev, generator=g) * scale).bfloat16()


def _cases(dev):
    ops = torch.ops.fsi
    g = torch.Generator(device=dev).manual_seed(1)
    s = torch.randn(2, 8, 32, device=dev, generator=g)
    x = _bf(16, 256, seed=2)
    kg, ku, v = _bf(512, 256, scale=0.05, seed=3), _bf(512, 256, scale=0.05, seed=4), _bf(512, 128, scale=0.05, seed=5)
    active = torch.tensor([5, 0, 2], dtype=torch.int32, device=dev)
    q = _bf(2, 4, 128, 64, seed=6)
    kv = _bf(2, 2, 128, 64, seed=7)
    lists = torch.randint(0, 4, (2, 4, 2), dtype=torch.int32, device=dev, generator=g)
    counts = torch.randint(0, 3, (2, 4), dtype=torch.int32, device=dev, generator=g)
    return [
        (ops.route_from_scores, (s, True, 1, 0.9, 0, 4, 4, None, None, None, 0)),
        (ops.score_and_route, (_bf(2, 6, 16, seed=8), _bf(1, 40, 16, seed=9), False, 0, 0.9, 0, 8, 8, True)),
        (ops.pattention, (x, kg, ku, v, active, 64, 0, 1, False)),
        (ops.mlp_router, (x, _bf(16, 256, seed=10), _bf(8, 16, seed=11), 2, 3, 1.0, True)),
        (ops.swiglu, (x, _bf(16, 256, seed=12), "fused")),
        (ops.block_sparse_linear, (x, kg, None, active, 64)),
        (ops.blockwise_matmul, (x, kg, (torch.rand(1, 4 * 8, device=dev, generator=g) < 0.5).to(torch.uint8), 64, 64,
                                16)),
        (ops.tile_route, (torch.randn(7, 48, device=dev, generator=g), 0.5, 2, 3)),
        (ops.sparse_attention, (q, kv, kv, lists, counts, 2, 32, 0, 32, 0.125)),
        (ops.sram_indexer_attention, (q.half(), q.half(), q.half(), _bf(2, 8, 16, seed=13).half(),
                                      _bf(2, 8, 16, seed=14).half(), 0.125, 0.8, 2, 16, True)),
    ]


@pytest.mark.parametrize("i", range(10))
def test_opcheck(fsi, dev, i):
    op, args = _cases(dev)[i]
    print(f"[case] opcheck {op}", flush=True)
    torch.library.opcheck(op, args, test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))


def test_compiled_decode_step_matches_eager(fsi, dev):
    """Router + packed Pattention decode of one 8B-shaped-down layer, compiled as one graph."""
    torch.manual_seed(0)
    m = fsi.FovealPattentionMLP(hidden_dim=512, intermediate_dim=2048, block_size=64, base_blocks=2, remote_blocks=6,
                                dtype=torch.bfloat16).to(dev).eval()
    packed = fsi.pack_pattention_weights(m.k_gate.detach(), m.k_up.detach(), m.v.detach(), 64)
    x = _bf(16, 512, seed=3)

    def step(x):
        active = torch.ops.fsi.mlp_router(x, m.q_proj_16d.weight, m.block_keys_16d, 2, 6, 1.0, False)[0]
        return torch.ops.fsi.pattention_packed(x, packed.buf, active, 2048, 512, 64, 1)

    with torch.no_grad():
        eager = step(x)
        compiled = torch.compile(step, backend="aot_eager", fullgraph=True)(x)
    assert torch.equal(eager, compiled)


def test_compiled_indexer_loss_backward_matches_eager(fsi, dev):
    """block_scores -> masked_softmax -> weighted sum, differentiated through the
    HIP forward and backward ops, eager vs compiled."""
    torch.manual_seed(1)
    q0 = torch.randn(2, 6, 16, device=dev)
    k0 = torch.randn(2, 10, 16, device=dev)
    w = torch.randn(2, 6, 10, device=dev)
    mask = torch.rand(2, 6, 10, device=dev) < 0.7

    def loss_fn(q, k):
        s = fsi.block_scores(q, k)
        p = fsi.masked_softmax(s, mask)
        return (p * w).sum()

    grads = []
    for fn in (loss_fn, torch.compile(loss_fn, backend="aot_eager")):
        q = q0.clone().requires_grad_()
        k = k0.clone().requires_grad_()
        loss = fn(q, k)
        loss.backward()
        grads.append((loss.detach(), q.grad, k.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)
