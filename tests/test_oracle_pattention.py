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


def test_swiglu_bwd_matches_autograd_fp64():
    """The closed-form SwiGLU gradient of the reference's Triton backward
    (pattention_triton.py:63-71) equals autograd through F.silu(g) * u."""
    from oracle import pattention as P

    g = torch.randn(257, dtype=torch.float64, requires_grad=True)
    u = torch.randn(257, dtype=torch.float64, requires_grad=True)
    dout = torch.randn(257, dtype=torch.float64)
    (torch.nn.functional.silu(g) * u).backward(dout)
    dg, du = P.swiglu_bwd_f64(dout, g.detach(), u.detach())
    assert torch.allclose(dg, g.grad, rtol=1e-12, atol=1e-14)
    assert torch.allclose(du, u.grad, rtol=1e-12, atol=1e-14)
    # special cases: g = 0 -> dg = dout * u / 2, du = 0
    z = torch.zeros(3, dtype=torch.float64)
    dg0, du0 = P.swiglu_bwd_f64(torch.ones(3), z, torch.tensor([2.0, -4.0, 1.0]))
    assert torch.allclose(dg0, torch.tensor([1.0, -2.0, 0.5], dtype=torch.float64)) and torch.all(du0 == 0)


@pytest.mark.parametrize("base,remote,temp", [(2, 6, 1.0), (1, 3, 0.5), (0, 4, 2.0)])
def test_train_forward_closed_form(base, remote, temp):
    """train_forward (foveal_pattention.py:292-307, 328-342) against brute force:
    per-token rms-normed 16-D queries, the active set = base blocks + the top
    `remote` token-mean scores, dense SwiGLU in fp64 with the inactive channels
    zeroed, plus softmax(scores / T) @ block_keys through out_proj."""
    import math

    import __graft_entry__

    fi = __graft_entry__.load_package()
    torch.manual_seed(base * 10 + remote)
    H, I, bs, T = 64, 512, 64, 5
    m = fi.FovealPattentionMLP(hidden_dim=H, intermediate_dim=I, block_size=bs, base_blocks=base,
                               remote_blocks=remote, temperature=temp, dtype=torch.float64).train()
    with torch.no_grad():
        m.block_keys_16d.normal_()
    x = torch.randn(T, H, dtype=torch.float64)
    out, active = P.train_forward(m, x)

    Wq, K16, Wo = m.q_proj_16d.weight.detach(), m.block_keys_16d.detach(), m.out_proj_16d.weight.detach()
    nb = I // bs
    scores = torch.zeros(T, nb, dtype=torch.float64)
    add = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        q = [sum(Wq[i, d].item() * x[t, d].item() for d in range(H)) for i in range(16)]
        r = math.sqrt(sum(v * v for v in q) / 16)
        q = [v / r for v in q]
        s = [sum(q[i] * K16[j, i].item() for i in range(16)) / 4.0 for j in range(nb)]
        scores[t] = torch.tensor(s, dtype=torch.float64)
        e = [math.exp((v - max(s)) / temp) for v in s]
        p = [v / sum(e) for v in e]
        c = [sum(p[j] * K16[j, i].item() for j in range(nb)) for i in range(16)]
        add[t] = torch.tensor([sum(Wo[h, i].item() * c[i] for i in range(16)) for h in range(H)], dtype=torch.float64)
    mean = scores.mean(0)
    rem = sorted(range(base, nb), key=lambda j: -mean[j].item())[:remote]
    assert active[:base].tolist() == list(range(base)) and sorted(active[base:].tolist()) == sorted(rem)
    mask = torch.zeros(I, dtype=torch.float64)
    for b in active.tolist():
        mask[b * bs:(b + 1) * bs] = 1
    want = P.dense_swiglu_f64(x, m.k_gate.detach(), m.k_up.detach(), m.v.detach(), mask) + add
    assert torch.allclose(out.detach(), want, rtol=1e-10, atol=1e-10)


def test_dense_block_targets_brute_force():
    """The teacher-target oracle (train_foveal_pattention_speedrun.py:176-185)
    against explicit loops in fp64: |silu(g) u| block means times the block
    mean of W_down's column norms, softmax over blocks / T."""
    import math

    g0 = torch.Generator().manual_seed(11)
    M, D, I, bs, T = 3, 8, 64, 32, 0.05
    h = torch.randn(M, D, generator=g0, dtype=torch.float64)
    gw = torch.randn(I, D, generator=g0, dtype=torch.float64) * 0.3
    uw = torch.randn(I, D, generator=g0, dtype=torch.float64) * 0.3
    dw = torch.randn(D, I, generator=g0, dtype=torch.float64)
    P_ = P.dense_block_targets(h, gw, uw, dw, bs, T)
    nb = I // bs
    for m in range(M):
        e = []
        for b in range(nb):
            a = n = 0.0
            for i in range(b * bs, (b + 1) * bs):
                gv = sum(h[m, d].item() * gw[i, d].item() for d in range(D))
                uv = sum(h[m, d].item() * uw[i, d].item() for d in range(D))
                a += abs(gv / (1 + math.exp(-gv)) * uv)
                n += math.sqrt(sum(dw[d, i].item() ** 2 for d in range(D)))
            e.append(a / bs * n / bs / T)
        mx = max(e)
        z = sum(math.exp(v - mx) for v in e)
        want = torch.tensor([math.exp(v - mx) / z for v in e])
        assert torch.allclose(P_[m].double(), want.double(), rtol=1e-5, atol=1e-7)
    assert torch.allclose(P_.sum(-1), torch.ones(M), atol=1e-6)


def test_calibrate_offline_svd_oracle_invariants():
    """The calibration oracle (foveal_pattention.py:175-255) against facts the
    mathematics fixes: orthonormal q rows spanning the top eigenvectors of X^T X,
    explained variance from the eigenvalues, the ridge normal equations, and the
    teacher targets against brute-force block energies."""
    g0 = torch.Generator().manual_seed(4)
    D, I, bs = 24, 128, 32
    X = torch.randn(200, D, generator=g0, dtype=torch.float64) * torch.linspace(3, 0.2, D, dtype=torch.float64)
    kg = torch.randn(I, D, generator=g0, dtype=torch.float64) * 0.2
    ku = torch.randn(I, D, generator=g0, dtype=torch.float64) * 0.2
    v = torch.randn(I, D, generator=g0, dtype=torch.float64) * 0.2
    q, keys, met = P.calibrate_offline_svd(kg, ku, v, X, 16, bs, 1, 2, 0.5, 1e-2)
    assert torch.allclose(q @ q.T, torch.eye(16, dtype=torch.float64), atol=1e-10)
    evals, evecs = torch.linalg.eigh(X.T @ X)
    top = evecs[:, -16:]
    assert torch.allclose(q.T @ (q @ top), top, atol=1e-8)  # same subspace
    assert abs(met["top16_explained_variance"] - (evals[-16:].sum() / evals.sum()).item()) < 1e-10
    Z, target = met["Z"], met["target"]
    resid = (Z.T @ Z + 1e-2 * torch.eye(16, dtype=torch.float64)) @ keys.T - Z.T @ target
    assert resid.abs().max() < 1e-9
    t, b = 7, 2  # one target entry by brute force
    e = []
    for blk in range(I // bs):
        a = sum(abs(torch.nn.functional.silu(X[t] @ kg[j]) * (X[t] @ ku[j])) for j in range(blk * bs, (blk + 1) * bs))
        e.append(a / bs * v[blk * bs:(blk + 1) * bs].pow(2).sum().sqrt())
    e = torch.stack(e) / 0.5
    assert torch.allclose(target[t], torch.softmax(e, 0), atol=1e-12)
    assert met["calib_active_blocks"][0] == 0 and len(met["calib_active_blocks"]) == 3
