"""Pins the Pattention oracle (CPU) against closed forms: with every block
active the Pattention MLP equals dense SwiGLU; with any active set it equals
dense SwiGLU with the inactive channels zeroed."""
import pytest
import torch

from oracle import pattention as P


def _weights(D, N_p, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    kg = (torch.randn(N_p, D, generator=g) * 0.05).to(dtype)
    ku = (torch.randn(N_p, D, generator=g) * 0.05).to(dtype)
    v = (torch.randn(N_p, D, generator=g) * 0.05).to(dtype)
    x = torch.randn(12, D, generator=g).to(dtype)
    return x, kg, ku, v


@pytest.mark.parametrize("fused", [False, True])
def test_all_blocks_equals_dense_swiglu_fp32(fused):
    x, kg, ku, v = _weights(64, 256, torch.float32)
    active = torch.arange(4)
    out = P.mlp_eval_forward(x, kg, ku, v, active, 64, fused=fused)
    ref = P.dense_swiglu_f64(x, kg, ku, v)
    assert P.rel_l2(out, ref) < 1e-6


def test_sparse_equals_masked_dense_fp32():
    x, kg, ku, v = _weights(64, 512, torch.float32, seed=1)
    active = torch.tensor([5, 0, 3])
    mask = torch.zeros(512)
    for b in active.tolist():
        mask[b * 64:(b + 1) * 64] = 1
    out = P.mlp_eval_forward(x, kg, ku, v, active, 64, fused=False)
    assert P.rel_l2(out, P.dense_swiglu_f64(x, kg, ku, v, mask)) < 1e-6
    # the reference fallback and fp32-act forms agree with the same closed form
    out2 = P.pattention_eager(x, kg, v, ku, active, "swiglu", 64)
    out3 = P.pattention_fp32_act(x, kg, v, ku, active, "swiglu", 64)
    assert P.rel_l2(out2, P.dense_swiglu_f64(x, kg, ku, v, mask)) < 1e-6
    assert P.rel_l2(out3, P.dense_swiglu_f64(x, kg, ku, v, mask)) < 1e-6


def test_bf16_rounding_points_distinct_but_close():
    x, kg, ku, v = _weights(128, 512, torch.bfloat16, seed=2)
    active = torch.tensor([1, 6, 2])
    exact = P.dense_swiglu_f64(x.float(), kg.float(), ku.float(), v.float(),
                               torch.repeat_interleave(torch.tensor([0, 1, 1, 0, 0, 0, 1, 0.]), 64))
    eager = P.mlp_eval_forward(x, kg, ku, v, active, 64, fused=False)
    fused = P.mlp_eval_forward(x, kg, ku, v, active, 64, fused=True)
    # each bf16 path sits near the exact result; the modes differ from each other
    assert P.rel_l2(eager, exact) < 1e-2
    assert P.rel_l2(fused, exact) < 1e-2
    assert not torch.equal(eager, fused)


def test_swiglu_forms():
    g = torch.randn(1000).bfloat16()
    u = torch.randn(1000).bfloat16()
    e = P.swiglu_eager(g, u)
    f = P.swiglu_fused(g, u)
    ref = (g.double() * torch.sigmoid(g.double()) * u.double())
    assert (f.double() - ref).abs().max() <= ref.abs().max() * 2 ** -7
    # eager rounds silu(g) first: identical to rounding twice
    assert torch.equal(e, (torch.nn.functional.silu(g.float()).bfloat16().float() * u.float()).bfloat16())


def test_activations_closed_form():
    x, kg, ku, v = _weights(32, 128, torch.float32, seed=3)
    for act, fn in [("relu", lambda g: g.clamp_min(0)), ("relu2", lambda g: g.clamp_min(0) ** 2),
                    ("silu", lambda g: g * torch.sigmoid(g)),
                    ("gelu", lambda g: 0.5 * g * (1 + torch.erf(g / 2 ** 0.5)))]:
        out = P.pattention_eager(x, kg, v, None, None, act, 64)
        ref = fn(x.double() @ kg.double().t()) @ v.double()
        assert P.rel_l2(out, ref) < 1e-6, act
