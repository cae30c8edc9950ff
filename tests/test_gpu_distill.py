"""FovealIndexer.distillation_loss (foveal_indexer/core.py:315-353) on the HIP
kernels of csrc/distill.hip against the oracle restatement (fp64 autograd):
loss value and gradient in the student scores, for the causal, full and
explicit-mask valid sets, fp32 and bf16 scores, several temperatures, rows
whose teacher mass vanishes and rows without a valid block."""
import pytest
import torch

from oracle import indexer as IX

pytestmark = pytest.mark.gpu

F64 = torch.float64


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind,temperature", [("causal", 1.0), ("full", 0.5), ("explicit", 2.0), ("causal", 3.0)])
@pytest.mark.parametrize("shape", [(2, 7, 7), (1, 33, 300), (3, 64, 64)])
def test_distillation_loss_matches_oracle(fsi, dev, dtype, kind, temperature, shape):
    B, Q, N = shape
    g = torch.Generator().manual_seed(B * 1000 + Q + N)
    s = (torch.randn(B, Q, N, generator=g) * 2).to(dtype)
    t = torch.rand(B, Q, N, generator=g) - 0.1
    t[0, Q // 2] = 0.0  # vanishing teacher mass -> uniform target
    mask = None
    if kind == "explicit":
        mask = torch.rand(B, Q, N, generator=g) > 0.5
        mask[0, 0] = False
    m = fsi.FovealIndexer(hidden_size=32, causal=(kind == "causal"), distill_temperature=temperature)
    sd = s.to(dev).requires_grad_()
    loss = m.distillation_loss(sd, t.to(dev), None if mask is None else mask.to(dev))
    loss.backward()
    sr = s.to(F64).requires_grad_()
    ref = IX.distillation_loss(sr, t.to(F64), mask, causal=(kind == "causal"), temperature=temperature, acc=F64)
    ref.backward()
    assert loss.dtype == torch.float32 and loss.dim() == 0
    assert abs(float(loss) - float(ref)) <= 2e-6 * max(1.0, abs(float(ref)))
    tol = 2e-6 if dtype == torch.float32 else 8e-3  # bf16: the gradient is rounded to bf16
    assert sd.grad.dtype == dtype
    assert _rel(sd.grad, sr.grad) <= tol
    if kind == "causal":
        assert not sd.grad[:, 0].any()  # query block 0 has no candidate block


def test_distillation_loss_no_valid_rows(fsi, dev):
    """One causal query block: no candidates anywhere; the loss is a zero of the
    scores' dtype with a zero gradient (core.py:351-353)."""
    m = fsi.FovealIndexer(hidden_size=32, causal=True)
    s = torch.randn(2, 1, 5, device=dev, dtype=torch.bfloat16, requires_grad=True)
    loss = m.distillation_loss(s, torch.rand(2, 1, 5, device=dev))
    loss.backward()
    assert float(loss) == 0.0 and loss.dtype == torch.bfloat16
    assert not s.grad.any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_distillation_loss_all_false_mask(fsi, dev, dtype):
    """An explicit valid mask with no valid entry: the reference's scores.sum() * 0,
    a zero in the scores' dtype with a zero gradient (core.py:351-353)."""
    m = fsi.FovealIndexer(hidden_size=32, causal=False)
    s = torch.randn(2, 3, 5, device=dev, dtype=dtype, requires_grad=True)
    mask = torch.zeros(2, 3, 5, dtype=torch.bool, device=dev)
    loss = m.distillation_loss(s, torch.rand(2, 3, 5, device=dev), mask)
    loss.backward()
    assert float(loss) == 0.0 and loss.dtype == dtype
    assert not s.grad.any()


def test_distillation_loss_broadcast_mask_and_teacher(fsi, dev):
    """A (Q, N) valid mask and a teacher broadcast over the batch."""
    g = torch.Generator().manual_seed(11)
    s = torch.randn(3, 8, 20, generator=g)
    t = torch.rand(8, 20, generator=g)
    mask = torch.rand(8, 20, generator=g) > 0.3
    m = fsi.FovealIndexer(hidden_size=32, causal=False)
    sd = s.to(dev).requires_grad_()
    loss = m.distillation_loss(sd, t.to(dev).expand(3, 8, 20), mask.to(dev))
    loss.backward()
    sr = s.to(F64).requires_grad_()
    ref = IX.distillation_loss(sr, t.to(F64).expand(3, 8, 20), mask, causal=False, acc=F64)
    ref.backward()
    assert abs(float(loss) - float(ref)) <= 2e-6 * max(1.0, abs(float(ref)))
    assert _rel(sd.grad, sr.grad) <= 2e-6
