"""Oracle for the block-sparse Pattention MLP — TEST INFRASTRUCTURE ONLY.

Restates, with the same torch CPU ops in the same order (so bf16 rounding
lands at the same points as the reference):
  * FovealPattentionMLP eval body       foveal_indexer/foveal_pattention.py:115-122 (gather),
                                        :329-335 (3x F.linear + SwiGLU)
  * _pytorch_pattention_fallback        foveal_indexer/pattention_triton.py:280-311
  * _pattention_fused_kernel numerics   foveal_indexer/pattention_triton.py:153-201
                                        (fp32 accumulation, act cast to V dtype, fp32 acc)
  * _swiglu_fwd_kernel numerics         foveal_indexer/pattention_triton.py:40-47
  * _swiglu_bwd_kernel                  foveal_indexer/pattention_triton.py:49-71 (closed form, fp64)
  * FovealPattentionMLP training forward foveal_indexer/foveal_pattention.py:292-307, 328-342
  * dense block-energy teacher targets  archive/hy_mt2/llm_pattention/train_foveal_pattention_speedrun.py:176-185
  * calibrate_offline_svd               foveal_indexer/foveal_pattention.py:175-255 (fp64)
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor


def rel_l2(a: Tensor, b: Tensor) -> float:
    a64, b64 = a.double(), b.double()
    return float((a64 - b64).norm() / b64.norm().clamp_min(1e-300))


def channel_index(active: Tensor, block_n: int) -> Tensor:
    """Row ids of the active channels, block-major (foveal_pattention.py:118)."""
    a = torch.as_tensor(active).reshape(-1, 1).to(torch.int64)
    return (a * block_n + torch.arange(block_n, dtype=torch.int64)).reshape(-1)


def swiglu_eager(g: Tensor, u: Tensor) -> Tensor:
    """`F.silu(kg) * ku` (foveal_pattention.py:284): silu and product each rounded."""
    return F.silu(g) * u


def swiglu_fused(g: Tensor, u: Tensor) -> Tensor:
    """silu(g) * u in fp32, one rounding to g's dtype (pattention_triton.py:40-47)."""
    gf, uf = g.float(), u.float()
    return (gf * torch.sigmoid(gf) * uf).to(g.dtype)


def mlp_eval_forward(x2d: Tensor, k_gate: Tensor, k_up: Tensor, v: Tensor, active: Tensor, block_n: int,
                     fused: bool) -> Tensor:
    """Eval forward of FovealPattentionMLP over a fixed active set
    (foveal_pattention.py:119-121 gather, :329-335 body)."""
    rows = channel_index(active, block_n)
    kg_act, ku_act, v_act = k_gate[rows], k_up[rows], v[rows]
    g = F.linear(x2d, kg_act)
    u = F.linear(x2d, ku_act)
    act = swiglu_fused(g, u) if fused else swiglu_eager(g, u)
    return F.linear(act, v_act.t())


def _activation(name: str, g: Tensor, u: Tensor | None) -> Tensor:
    if name == "swiglu":
        return F.silu(g) * u
    if name == "silu":
        return F.silu(g)
    if name == "gelu":
        return F.gelu(g)
    if name == "relu":
        return F.relu(g)
    if name == "relu2":
        return F.relu(g) ** 2
    return g


def pattention_eager(x: Tensor, k_gate: Tensor, v: Tensor, k_up: Tensor | None, active: Tensor | None,
                     activation: str, block_n: int) -> Tensor:
    """The reference's PyTorch fallback (pattention_triton.py:280-311)."""
    x2d = x.reshape(-1, x.shape[-1])
    if active is not None:
        rows = channel_index(active, block_n)
        k_gate, v = k_gate[rows], v[rows]
        if k_up is not None:
            k_up = k_up[rows]
    g = torch.matmul(x2d, k_gate.t())
    u = torch.matmul(x2d, k_up.t()) if k_up is not None else None
    out = torch.matmul(_activation(activation, g, u), v)
    return out.reshape(*x.shape[:-1], v.shape[-1])


def pattention_fp32_act(x: Tensor, k_gate: Tensor, v: Tensor, k_up: Tensor | None, active: Tensor | None,
                        activation: str, block_n: int) -> Tensor:
    """Numerics of the fused kernel (pattention_triton.py:153-201): gate/up
    accumulate in fp32, the activation runs in fp32 and is cast to V's dtype,
    the V contraction accumulates in fp32 and the result is cast to x's dtype.
    GeLU is the exact erf form (the fallback's F.gelu, :300)."""
    x2d = x.reshape(-1, x.shape[-1])
    N_p = k_gate.shape[0]
    if active is not None:
        rows = channel_index(active, block_n)
        valid = rows < N_p  # the kernel masks rows beyond N_p (pattention_triton.py:151)
        rows = rows[valid]
        k_gate, v = k_gate[rows], v[rows]
        if k_up is not None:
            k_up = k_up[rows]
    xf = x2d.double()
    g = (xf @ k_gate.double().t()).float()
    u = (xf @ k_up.double().t()).float() if k_up is not None else None
    act = _activation(activation, g, u).to(v.dtype)
    out = (act.double() @ v.double()).float().to(x.dtype)
    return out.reshape(*x.shape[:-1], v.shape[-1])


def dense_swiglu_f64(x2d: Tensor, k_gate: Tensor, k_up: Tensor, v: Tensor, channel_mask: Tensor | None = None) -> Tensor:
    """Exact dense SwiGLU (silu(x Wg^T) * (x Wu^T)) Wd^T in fp64, optionally with
    the inactive channels zeroed — the closed form a sparse Pattention must equal."""
    xf = x2d.double()
    g = xf @ k_gate.double().t()
    u = xf @ k_up.double().t()
    h = g * torch.sigmoid(g) * u
    if channel_mask is not None:
        h = h * channel_mask.double()
    return h @ v.double()


def swiglu_bwd_f64(dout: Tensor, g: Tensor, u: Tensor):
    """(dg, du) of silu(g) * u in fp64 (pattention_triton.py:63-71):
    s = sigmoid(g); du = dout * g s; dg = dout * u * s (1 + g (1 - s))."""
    d, gg, uu = dout.double(), g.double(), u.double()
    sg = torch.sigmoid(gg)
    return d * uu * sg * (1.0 + gg * (1.0 - sg)), d * gg * sg


def train_forward(m, x: Tensor, active: Tensor | None = None):
    """FovealPattentionMLP.forward in training mode (foveal_pattention.py:292-307,
    328-342) with torch CPU ops in the reference's order, on the module's own
    parameters (autograd-capable): returns (out, active_blocks).  `active`, when
    given, replaces the top-k selection (to check the arithmetic after routing
    on its own)."""
    D = x.shape[-1]
    x_2d = x.reshape(-1, D)
    q_16 = F.rms_norm(m.q_proj_16d(x_2d), (m.index_dim,))
    scores = torch.matmul(q_16, m.block_keys_16d.t()) / math.sqrt(m.index_dim)
    _, top_remote = torch.topk(scores.mean(dim=0)[m.base_blocks:], k=m.remote_blocks)
    if active is None:
        active = torch.cat([torch.arange(m.base_blocks, dtype=torch.int32),
                            (top_remote + m.base_blocks).to(torch.int32)])
    indices = (active.view(-1, 1).to(torch.int64) * m.block_size + m.offsets).flatten()
    kg_proj = F.linear(x_2d, m.k_gate[indices])
    ku_proj = F.linear(x_2d, m.k_up[indices])
    act = F.silu(kg_proj) * ku_proj
    out_patt = F.linear(act, m.v[indices].t())
    soft = F.softmax(scores / m.temperature, dim=-1)
    add = m.out_proj_16d(torch.matmul(soft, m.block_keys_16d))
    return (out_patt + add).reshape(x.shape), active


def dense_block_targets(norm_h: Tensor, gate_w: Tensor, up_w: Tensor, down_w: Tensor, block_size: int,
                        temperature: float) -> Tensor:
    """P_target of compute_teacher_dense_block_targets
    (train_foveal_pattention_speedrun.py:176-185) with torch CPU ops in the
    inputs' dtype (bf16 models: the same rounding points as the reference)."""
    g = F.silu(F.linear(norm_h, gate_w))
    u = F.linear(norm_h, up_w)
    act = g * u
    nb = act.shape[-1] // block_size
    dw_norms = down_w.norm(dim=0).view(nb, block_size).mean(dim=-1)
    act_blocks = act.abs().view(*act.shape[:-1], nb, block_size).mean(dim=-1)
    energy = act_blocks * dw_norms
    return F.softmax(energy.float() / temperature, dim=-1)


def calibrate_offline_svd(k_gate: Tensor, k_up: Tensor, v: Tensor, X: Tensor, index_dim: int, block_size: int,
                          base_blocks: int, remote_blocks: int, temperature: float, ridge_lambda: float):
    """FovealPattentionMLP.calibrate_offline_svd (foveal_pattention.py:175-255)
    in fp64: returns (q_proj weight (16, D), block keys (nb, 16), metrics).
    v is the logical (intermediate, hidden) V = W_down^T."""
    X = X.double().reshape(-1, k_gate.shape[1])
    _, S, Vh = torch.linalg.svd(X, full_matrices=False)
    V16 = Vh[:index_dim].T
    Z = F.rms_norm(X @ V16, (index_dim,))
    kg, ku, vv = k_gate.double(), k_up.double(), v.double()
    A = F.silu(X @ kg.T) * (X @ ku.T)
    nb = kg.shape[0] // block_size
    energies = [A[:, b * block_size:(b + 1) * block_size].abs().mean(dim=-1)
                * vv[b * block_size:(b + 1) * block_size].norm() for b in range(nb)]
    target = F.softmax(torch.stack(energies, dim=-1) / temperature, dim=-1)
    reg = ridge_lambda * torch.eye(index_dim, dtype=torch.float64)
    keys = torch.linalg.solve(Z.T @ Z + reg, Z.T @ target).T
    scores = Z @ keys.T / math.sqrt(index_dim)
    kl = F.kl_div(F.softmax(scores / temperature, dim=-1).log(), target, reduction="batchmean").item()
    _, top = torch.topk(scores.mean(dim=0)[base_blocks:], k=remote_blocks)
    active = torch.cat([torch.arange(base_blocks), top + base_blocks]).to(torch.int32)
    metrics = {"top16_explained_variance": ((S[:index_dim] ** 2).sum() / (S ** 2).sum()).item(),
               "initial_kl_divergence": kl, "calib_active_blocks": active.tolist(), "Z": Z, "target": target,
               "scores": scores}
    return V16.T, keys, metrics
