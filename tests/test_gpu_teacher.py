"""GPU parity of the dense block-energy teacher targets (fsi_dense_block_targets,
dense_block_targets, compute_teacher_dense_block_targets) against the CPU
oracle of train_foveal_pattention_speedrun.py:154-189 in bf16 (the reference's
tensors and rounding points).  Tolerance per probability: 1e-2 relative
(+1e-6 absolute): the energies are bf16 values whose last bit can differ with
the summation order of the block means, a relative change of 2^-8 of the logit."""
from types import SimpleNamespace

import pytest
import torch
from torch import nn

from oracle import pattention as P

pytestmark = pytest.mark.gpu


def _close(got, want):
    got, want = got.float().cpu(), want.float().cpu()
    assert got.shape == want.shape
    err = (got - want).abs()
    assert torch.all(err <= want.abs() * 1e-2 + 1e-6), float((err / want.abs().clamp_min(1e-6)).max())
    assert torch.allclose(got.sum(-1), torch.ones(got.shape[:-1]), atol=1e-5)


# lead shape, D, I, block, temperature: small-M kernel, DMA kernel, K % 32 != 0, 3-D input
CASES = [
    ((5,), 256, 1024, 64, 0.01),
    ((300,), 512, 2048, 32, 0.005),
    ((257,), 264, 1536, 128, 0.01),
    ((2, 100), 256, 896, 64, 0.02),
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_dense_block_targets_parity(fsi, dev, case):
    lead, D, I, bs, T = case
    g = torch.Generator().manual_seed(D + I)
    h = torch.randn(*lead, D, generator=g).bfloat16()
    gw = (torch.randn(I, D, generator=g) * D ** -0.5).bfloat16()
    uw = (torch.randn(I, D, generator=g) * D ** -0.5).bfloat16()
    dw = (torch.randn(D, I, generator=g) * (0.5 + torch.rand(1, I, generator=g)) * 0.05).bfloat16()
    got = fsi.dense_block_targets(h.to(dev), gw.to(dev), uw.to(dev), dw.to(dev), bs, T)
    assert got.dtype == torch.float32 and got.shape == (*lead, I // bs)
    want = P.dense_block_targets(h, gw, uw, dw, bs, T)
    _close(got, want)


def test_dense_block_targets_errors(fsi, dev):
    h = torch.randn(4, 64, device=dev, dtype=torch.bfloat16)
    w = torch.randn(256, 64, device=dev, dtype=torch.bfloat16)
    wd = torch.randn(64, 256, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        fsi.dense_block_targets(h, w, w, wd, block_size=48)
    with pytest.raises(TypeError):
        fsi.dense_block_targets(h.float(), w, w, wd)
    with pytest.raises(ValueError):
        fsi.dense_block_targets(h, w, w, wd.t().contiguous()[:, :64])
    assert fsi.dense_block_targets(h[:0], w, w, wd).shape == (0, 4)


class _Layer(nn.Module):
    def __init__(self, D, I):
        super().__init__()
        self.post_attention_layernorm = nn.RMSNorm(D, eps=1e-6)
        self.mlp = nn.Module()
        self.mlp.gate_proj = nn.Linear(D, I, bias=False)
        self.mlp.up_proj = nn.Linear(D, I, bias=False)
        self.mlp.down_proj = nn.Linear(I, D, bias=False)
        self.mix = nn.Linear(D, D, bias=False)

    def forward(self, x):
        return x + torch.tanh(self.mix(x))


class _Model(nn.Module):
    """A stand-in decoder with the attributes the teacher code reads
    (embed, layers[i].post_attention_layernorm / .mlp, hidden states)."""

    def __init__(self, D, I, n_layers):
        super().__init__()
        self.embed = nn.Embedding(50, D)
        self.layers = nn.ModuleList([_Layer(D, I) for _ in range(n_layers)])

    def forward(self, ids, output_hidden_states=False):
        x = self.embed(ids)
        hs = [x]
        for layer in self.layers:
            x = layer(x)
            hs.append(x)
        return SimpleNamespace(last_hidden_state=x, hidden_states=hs)


def test_compute_teacher_dense_block_targets(fsi, dev):
    torch.manual_seed(0)
    D, I = 128, 512
    teacher = nn.Module()
    teacher.model = _Model(D, I, 17)
    teacher = teacher.to(dev, torch.bfloat16)
    ids = torch.randint(0, 50, (2, 40), device=dev)
    t_rep, t_mid, targets = fsi.compute_teacher_dense_block_targets(teacher, ids, [3, 10], block_size=64,
                                                                     temperature=0.01)
    out = teacher.model(ids, output_hidden_states=True)
    assert torch.equal(t_rep, out.last_hidden_state) and torch.equal(t_mid, out.hidden_states[16])
    assert len(targets) == 2
    for l_idx, got in zip([3, 10], targets):
        layer = teacher.model.layers[l_idx]
        norm_h = layer.post_attention_layernorm(out.hidden_states[l_idx]).cpu()
        mlp = layer.mlp
        want = P.dense_block_targets(norm_h, mlp.gate_proj.weight.cpu(), mlp.up_proj.weight.cpu(),
                                     mlp.down_proj.weight.cpu(), 64, 0.01)
        assert got.shape == (2, 40, I // 64)
        _close(got, want)
