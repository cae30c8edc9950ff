"""Pins of the indexer-representation oracle against brute force and closed
forms (CPU only)."""
import math

import pytest
import torch

from oracle import indexer as IX


def test_rms_norm16_brute_force():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 16, generator=g) * 3
    y = IX.rms_norm16(x)
    for r in range(5):
        row = [float(v) for v in x[r]]
        rms = math.sqrt(sum(v * v for v in row) / 16 + 1.1920928955078125e-07)
        for c in range(16):
            assert abs(float(y[r, c]) - row[c] / rms) <= 1e-6 * max(1.0, abs(row[c] / rms))


def test_pool_kv_brute_force_and_unit_norm():
    g = torch.Generator().manual_seed(1)
    B, N, bs = 2, 12, 4
    k = torch.randn(B, N, 16, generator=g)
    v = torch.randn(B, N, 16, generator=g)
    kb, vb = IX.pool_kv(k, v, bs)
    assert kb.shape == (B, 3, 16) and vb.shape == (B, 3, 16)
    for b in range(B):
        for blk in range(3):
            toks = range(blk * bs, (blk + 1) * bs)
            normed = []
            for t in toks:
                row = k[b, t].double()
                normed.append(row / torch.sqrt((row * row).mean() + 1.1920928955078125e-07))
            m = sum(normed) / bs
            ref = m / m.norm()
            assert torch.allclose(kb[b, blk].double(), ref, atol=1e-6)
            assert torch.allclose(vb[b, blk].double(), v[b, list(toks)].double().mean(0), atol=1e-6)
    assert torch.allclose(kb.norm(dim=-1), torch.ones(B, 3), atol=1e-6)


def test_block_scores_are_cosine_over_four():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 5, 16, generator=g)
    k = torch.randn(2, 9, 16, generator=g)
    s = IX.block_scores(q, k)
    ref = torch.einsum("bqd,bkd->bqk", q.double(), k.double())
    ref = ref / (q.double().norm(dim=-1)[..., None] * k.double().norm(dim=-1)[:, None, :]) / 4.0
    assert torch.allclose(s.double(), ref, atol=1e-6)
    # bf16: operands rounded after normalising, product rounded, then / 4
    sb = IX.block_scores(q.bfloat16(), k.bfloat16())
    assert sb.dtype == torch.bfloat16
    assert torch.allclose(sb.double(), ref, atol=2e-3)


def test_additive_context_brute_force():
    g = torch.Generator().manual_seed(3)
    s = torch.randn(1, 4, 6, generator=g)
    v = torch.randn(1, 6, 16, generator=g)
    ctx = IX.additive_context(s, v, causal=True)
    assert torch.all(ctx[0, 0] == 0)  # query block 0 sees no complete block
    for q in range(1, 4):
        w = [math.exp(float(s[0, q, p])) for p in range(q)]
        z = sum(w)
        ref = sum((w[p] / z) * v[0, p].double() for p in range(q))
        assert torch.allclose(ctx[0, q].double(), ref, atol=1e-6)
    full = IX.additive_context(s, v, causal=False)
    w = torch.softmax(s[0].double(), -1)
    assert torch.allclose(full[0].double(), w @ v[0].double(), atol=1e-6)


@pytest.mark.parametrize("causal", [True, False])
def test_indexer_gradients_match_finite_differences(causal):
    """The backward oracle is autograd of the fp64 restatement; gradcheck pins
    it against central differences for every differentiable input."""
    from oracle import indexer as IX
    from oracle import routing as R

    g = torch.Generator().manual_seed(3)
    f64 = dict(dtype=torch.float64)
    x = torch.randn(2, 5, 16, generator=g, **f64).requires_grad_()
    assert torch.autograd.gradcheck(lambda t: IX.rms_norm16(t), (x,))
    k = torch.randn(2, 12, 16, generator=g, **f64).requires_grad_()
    v = torch.randn(2, 12, 16, generator=g, **f64).requires_grad_()
    assert torch.autograd.gradcheck(lambda a, b: IX.pool_kv(a, b, 4, torch.float64), (k, v))
    q = torch.randn(2, 4, 16, generator=g, **f64).requires_grad_()
    kb = torch.randn(2, 3, 16, generator=g, **f64).requires_grad_()
    assert torch.autograd.gradcheck(lambda a, b: IX.block_scores(a, b, torch.float64), (q, kb))
    s = torch.randn(2, 4, 3, generator=g, **f64).requires_grad_()
    vb = torch.randn(2, 3, 16, generator=g, **f64).requires_grad_()
    assert torch.autograd.gradcheck(lambda a, b: IX.additive_context(a, b, causal, torch.float64), (s, vb))
    mask = torch.rand(2, 4, 3, generator=g) > 0.4
    mask[0, 1] = False  # an all-masked row
    assert torch.autograd.gradcheck(lambda a: R.masked_probs(a, mask, torch.float64), (s,))
