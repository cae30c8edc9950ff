"""GPU parity of model conversion: calibrate_offline_svd
(foveal_pattention.py:175-255) against the fp64 oracle, and a checkpoint loaded
from local safetensors running the Pattention forward.

Singular vectors carry an arbitrary sign per component, so the calibration is
compared through sign-invariant quantities: router scores on held-out tokens
(rel-L2 <= 1e-3 for an fp32 module, 3e-2 for bf16 parameters), explained
variance (1e-5 absolute), KL (1e-3 relative) and the calibrated active set."""
import json

import pytest
import torch
import torch.nn.functional as F

from oracle import pattention as P

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm()).item()


def _setup(dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    H, I = 256, 2048
    kg = (torch.randn(I, H, generator=g) * H ** -0.5).to(dtype)
    ku = (torch.randn(I, H, generator=g) * H ** -0.5).to(dtype)
    v = (torch.randn(I, H, generator=g) * H ** -0.5 * (0.2 + torch.rand(I, 1, generator=g))).to(dtype)
    spec = torch.linspace(4.0, 0.1, H)
    X = torch.randn(3072, H, generator=g) * spec
    Xh = torch.randn(64, H, generator=g) * spec
    return kg, ku, v, X, Xh


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_calibrate_offline_svd_parity(fsi, dev, dtype):
    kg, ku, v, X, Xh = _setup(dtype)
    m = fsi.FovealPattentionMLP(hidden_dim=256, intermediate_dim=2048, block_size=64, base_blocks=2,
                                remote_blocks=6, temperature=0.05, dtype=dtype).to(dev)
    with torch.no_grad():
        m.k_gate.copy_(kg)
        m.k_up.copy_(ku)
        m.v.copy_(v)
    met = m.calibrate_offline_svd(X.to(dev))
    q, keys, ref = P.calibrate_offline_svd(kg, ku, v, X, 16, 64, 2, 6, 0.05, 1e-2)
    assert abs(met["top16_explained_variance"] - ref["top16_explained_variance"]) < 1e-5
    assert abs(met["initial_kl_divergence"] - ref["initial_kl_divergence"]) <= 1e-3 * ref["initial_kl_divergence"] + 1e-6
    with torch.no_grad():
        got = m.compute_router_scores(Xh.to(dev, dtype)).float()
    want = F.rms_norm(Xh.double() @ q.T, (16,)) @ keys.T / 4.0
    assert _rel(got, want) <= (1e-3 if dtype == torch.float32 else 3e-2)
    assert met["num_blocks"] == 32 and met["active_blocks"] == 8
    mean = ref["scores"].mean(0)[2:].sort(descending=True).values
    if (mean[5] - mean[6]).item() > 1e-3:  # no near-tie at the top-k boundary
        assert met["calib_active_blocks"] == ref["calib_active_blocks"]
    assert m._cached_active_blocks.cpu().tolist() == met["calib_active_blocks"]
    assert m.q_proj_16d.weight.dtype == dtype and m.block_keys_16d.dtype == dtype


def test_loaded_checkpoint_forward(fsi, dev, tmp_path):
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(1)
    H, I = 256, 1024
    t = {}
    for i in range(2):
        t[f"model.layers.{i}.mlp.gate_proj.weight"] = (torch.randn(I, H, generator=g) * 0.05).bfloat16()
        t[f"model.layers.{i}.mlp.up_proj.weight"] = (torch.randn(I, H, generator=g) * 0.05).bfloat16()
        t[f"model.layers.{i}.mlp.down_proj.weight"] = (torch.randn(H, I, generator=g) * 0.05).bfloat16()
    save_file(t, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": H, "intermediate_size": I,
                                                      "num_hidden_layers": 2}))
    ms = fsi.load_foveal_pattention_mlps(tmp_path, block_size=64, base_blocks=4, remote_blocks=4, device=dev)
    x = torch.randn(2, 24, H, generator=g).bfloat16()
    for i, m in ms.items():
        m.eval()
        assert m.k_gate.device.type == "cuda"
        active = torch.tensor([0, 1, 2, 3, 9, 12, 5, 15], dtype=torch.int32)
        m.set_active_blocks(active)
        with torch.no_grad():
            out = m(x.to(dev))
        ref = P.mlp_eval_forward(x.reshape(-1, H), t[f"model.layers.{i}.mlp.gate_proj.weight"],
                                 t[f"model.layers.{i}.mlp.up_proj.weight"],
                                 t[f"model.layers.{i}.mlp.down_proj.weight"].t(), active, 64, fused=True)
        assert P.rel_l2(out.cpu().reshape(-1, H), ref) <= 2e-3
