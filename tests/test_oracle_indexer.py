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


def _distill_case(g, B, Q, N, kind):
    s = torch.randn(B, Q, N, generator=g, dtype=torch.float64) * 2
    t = torch.rand(B, Q, N, generator=g, dtype=torch.float64) - 0.2  # some negative teacher mass
    t[0, -1] = 0.0  # a row whose teacher mass vanishes -> uniform target
    if kind == "explicit":
        mask = torch.rand(B, Q, N, generator=g) > 0.4
        mask[0, 0] = False  # a row without a valid block
        return s, t, mask, False
    return s, t, None, kind == "causal"


@pytest.mark.parametrize("kind", ["causal", "full", "explicit"])
@pytest.mark.parametrize("temperature", [0.5, 1.0, 2.0])
def test_distillation_loss_brute_force(kind, temperature):
    from oracle import brute

    g = torch.Generator().manual_seed(7)
    B, Q, N = 2, 6, 9
    s, t, mask, causal = _distill_case(g, B, Q, N, kind)
    got = IX.distillation_loss(s, t, mask, causal=causal, temperature=temperature, acc=torch.float64)
    if mask is None:
        valid = (torch.arange(N)[None] < torch.arange(Q)[:, None]) if causal else torch.ones(Q, N, dtype=torch.bool)
        valid = valid[None].expand(B, Q, N)
    else:
        valid = mask
    rows_s = s.reshape(B * Q, N).tolist()
    rows_t = t.reshape(B * Q, N).tolist()
    rows_v = valid.reshape(B * Q, N).tolist()
    ref, per_row = brute.distill_loss_rows(rows_s, rows_t, rows_v, temperature)
    assert abs(float(got) - ref) <= 1e-12 * max(1.0, abs(ref))
    if kind != "full":
        assert any(r is None for r in per_row)  # the empty rows are excluded, not averaged as 0


def test_distillation_loss_closed_forms():
    g = torch.Generator().manual_seed(3)
    s = torch.randn(1, 4, 11, generator=g, dtype=torch.float64)
    p = torch.softmax(s, dim=-1)
    # teacher = student distribution: the loss is the mean entropy of the rows
    ent = -(p * p.log()).sum(-1).mean()
    got = IX.distillation_loss(s, p * 3.0, causal=False, acc=torch.float64)  # unnormalised teacher mass
    assert abs(float(got) - float(ent)) <= 1e-12
    # zero teacher: uniform target, loss = logsumexp(z) - mean(z)
    z = s / 0.7
    ref = (torch.logsumexp(z, -1) - z.mean(-1)).mean()
    got = IX.distillation_loss(s, torch.zeros_like(s), causal=False, temperature=0.7, acc=torch.float64)
    assert abs(float(got) - float(ref)) <= 1e-12
    # one query block, causal: no valid row, zero loss with zero gradient
    s1 = torch.randn(1, 1, 5, dtype=torch.float64, requires_grad=True)
    loss = IX.distillation_loss(s1, torch.rand(1, 1, 5, dtype=torch.float64), causal=True, acc=torch.float64)
    loss.backward()
    assert float(loss) == 0.0 and not s1.grad.any()


def test_distillation_loss_gradcheck():
    g = torch.Generator().manual_seed(5)
    s = torch.randn(2, 4, 6, generator=g, dtype=torch.float64, requires_grad=True)
    t = torch.rand(2, 4, 6, generator=g, dtype=torch.float64)
    t[1, 2] = 0.0
    for causal in (True, False):
        assert torch.autograd.gradcheck(
            lambda x: IX.distillation_loss(x, t, causal=causal, temperature=1.3, acc=torch.float64), (s,))
