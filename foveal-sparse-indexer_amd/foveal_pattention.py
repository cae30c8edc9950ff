"""FovealPattentionMLP on MI355X: drop-in for foveal_indexer/foveal_pattention.py.

Same constructor, parameter names (state_dict compatible), eval routing,
active-block cache and forward signature as the reference
(foveal_pattention.py:54-352).  Differences by design:
  * No gathered weight copies: the reference slices the active rows of k_gate,
    k_up and v into contiguous caches (set_active_blocks, :115-122); here the
    HIP kernels stream those rows from the full tensors by block index, so the
    cache holds only the int32 block list.
  * bf16 rounding follows the reference's GPU path when use_fused_kernel=True
    (fused SwiGLU, one rounding of silu(g)*u; :281-282) and its eager path
    otherwise (silu(g) and the product rounded separately; :283-284).
  * Training mode follows the reference's per-token routing and additive stream
    with library GEMMs around the HIP SwiGLU forward / backward kernels.
"""
from __future__ import annotations

import json
import math
from pathlib import Path
from typing import Any, Dict, Iterable, List, Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _lib
from .pattention import (
    FusedSwiGLUFunction,
    PACKED_PREFILL_MIN_M,
    PackedPattentionWeights,
    dense_block_targets,
    _weights_key,
    pack_pattention_weights,
    packed_decode_supported,
    pattention_decode_packed,
    pattention_forward,
    triton_fused_swiglu,
    unpack_pattention_weights,
)


def mlp_pooled_route(
    x2d: Tensor,
    q_proj_weight: Tensor,
    block_keys: Tensor,
    base_blocks: int,
    remote_blocks: int,
    score_scale: float = 1.0,
    return_scores: bool = False,
):
    """Eval-mode pooled routing (foveal_pattention.py:310-321) on the GPU.

    Returns the int32 active block list [0..base) ++ (topk(s[base:]) + base);
    with return_scores, also the (n_blocks,) fp32 router scores."""
    what = "mlp_router"
    dev = _lib.require_gpu(x2d, q_proj_weight, block_keys, what=what)
    dt = x2d.dtype
    if q_proj_weight.dtype != dt or block_keys.dtype != dt:
        raise TypeError(f"{what}: dtype mismatch {dt}/{q_proj_weight.dtype}/{block_keys.dtype}")
    _lib.dtype_code(dt, what)
    if x2d.stride(-1) != 1:
        x2d = x2d.contiguous()
    wq = q_proj_weight.contiguous()
    keys = block_keys.contiguous()
    n_blocks = keys.shape[0]
    if remote_blocks > n_blocks - base_blocks:
        # torch.topk: "selected index k out of range" (foveal_pattention.py:314)
        raise RuntimeError(f"{what}: selected index k out of range ({remote_blocks} > {n_blocks - base_blocks})")
    active, scores = _mlp_router_op(x2d, wq, keys, int(base_blocks), int(remote_blocks), float(score_scale),
                                    bool(return_scores))
    if return_scores:
        return active, scores
    return active


@_lib.fsi_op("mlp_router", lambda x2d, wq, keys, base_blocks, remote_blocks, score_scale, want_scores: (
    x2d.new_empty((base_blocks + remote_blocks,), dtype=torch.int32),
    x2d.new_empty((keys.shape[0] if want_scores else 0,), dtype=torch.float32)))
def _mlp_router_op(x2d: Tensor, wq: Tensor, keys: Tensor, base_blocks: int, remote_blocks: int, score_scale: float,
                   want_scores: bool) -> Tuple[Tensor, Tensor]:
    """fsi_mlp_router: (active blocks int32, router scores fp32 (n_blocks,) or empty)."""
    what = "mlp_router"
    dev = x2d.device
    M, D = x2d.shape
    index_dim = wq.shape[0]
    n_blocks = keys.shape[0]
    active = torch.empty(base_blocks + remote_blocks, dtype=torch.int32, device=dev)
    scores = torch.empty(n_blocks if want_scores else 0, dtype=torch.float32, device=dev)
    stream = _lib.stream_handle(dev)
    L = _lib.lib()
    ws = _lib.workspace(dev, L.fsi_mlp_router_workspace_size(D, n_blocks), stream)
    st = L.fsi_mlp_router(x2d.data_ptr(), x2d.stride(0), M, D, wq.data_ptr(), index_dim, keys.data_ptr(), n_blocks,
                          base_blocks, remote_blocks, score_scale, _lib.dtype_code(x2d.dtype, what),
                          active.data_ptr(), scores.data_ptr() if want_scores else None, ws.data_ptr(), ws.numel(),
                          stream)
    _lib.check(st, what)
    return active, scores


class _EvalPattentionFn(torch.autograd.Function):
    """The eval-mode forward of FovealPattentionMLP with a gradient for its input.

    The reference's eval path runs F.linear on detached copies of the active
    rows (foveal_pattention.py:115-122, 278-288), so autograd reaches x but no
    weight.  Forward: the HIP decode / prefill kernels.  Backward, for
    h = act(g, u), g = x K_g,S^T, u = x K_u,S^T, y = h V_S:
        dh = dy V_S^T;  (dg, du) = swiglu_bwd(dh, g, u);  dx = dg K_g,S + du K_u,S
    with g, u recomputed, library GEMMs on the active rows and the HIP SwiGLU
    backward kernel."""

    @staticmethod
    def forward(ctx, x_2d: Tensor, module: "FovealPattentionMLP", active_blocks: Tensor) -> Tensor:
        ctx.module = module
        ctx.save_for_backward(x_2d, active_blocks)
        return module._eval_compute(x_2d, active_blocks)

    @staticmethod
    def backward(ctx, dy: Tensor):
        m = ctx.module
        x_2d, active_blocks = ctx.saved_tensors
        kg, ku, v = m._active_rows(active_blocks)
        g = F.linear(x_2d, kg)
        u = F.linear(x_2d, ku)
        dh = F.linear(dy.to(x_2d.dtype), v)
        dg, du = FusedSwiGLUFunction.backward(_SavedGU(g, u), dh)
        dx = F.linear(dg, kg.t().contiguous()) + F.linear(du, ku.t().contiguous())
        return dx, None, None


class _SavedGU:
    """Stand-in autograd context holding (g, u) for FusedSwiGLUFunction.backward."""

    def __init__(self, g: Tensor, u: Tensor):
        self.saved_tensors = (g.contiguous(), u.contiguous())


class FovealPattentionMLP(nn.Module):
    """Foveal block-sparse SwiGLU Pattention layer (foveal_pattention.py:54-352)."""

    _released = False  # pack-in-place inference mode (release_unpacked_weights)

    def __init__(
        self,
        hidden_dim: int = 2048,
        intermediate_dim: int = 6144,
        block_size: int = 64,
        base_blocks: int = 4,
        remote_blocks: int = 20,
        index_dim: int = 16,
        temperature: float = 1.0,
        dtype: torch.dtype = torch.bfloat16,
        use_fused_kernel: bool = True,
    ):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.block_size = block_size
        self.num_blocks = intermediate_dim // block_size
        self.base_blocks = base_blocks
        self.remote_blocks = remote_blocks
        self.total_active_blocks = base_blocks + remote_blocks
        self.active_channels = self.total_active_blocks * block_size
        self.index_dim = index_dim
        self.temperature = temperature
        self.dtype = dtype
        self.use_fused_kernel = use_fused_kernel

        self.k_gate = nn.Parameter(torch.empty(intermediate_dim, hidden_dim, dtype=dtype))
        self.k_up = nn.Parameter(torch.empty(intermediate_dim, hidden_dim, dtype=dtype))
        # v is logically (N_p, D) as in the reference; its storage is the row-major
        # (D, N_p) down_proj layout, which the decode kernel streams in full lines.
        self.v = nn.Parameter(torch.empty(hidden_dim, intermediate_dim, dtype=dtype).t())
        self.q_proj_16d = nn.Linear(hidden_dim, index_dim, bias=False, dtype=dtype)
        self.block_keys_16d = nn.Parameter(torch.empty(self.num_blocks, index_dim, dtype=dtype))
        self.out_proj_16d = nn.Linear(index_dim, hidden_dim, bias=False, dtype=dtype)
        self.register_buffer("offsets", torch.arange(block_size, dtype=torch.int64))

        self._cached_active_blocks: Optional[Tensor] = None
        self._gathered: Optional[tuple] = None
        # Decode (up to 64 tokens) and prefill (256 tokens and more) calls in bf16
        # stream a copy of k_gate, k_up and v repacked into the MFMA operand layout,
        # rebuilt whenever a weight tensor is replaced or modified in place.  It holds
        # as many bytes as the three weights; set pack_decode_weights = False to run
        # from the parameters directly.
        self.pack_decode_weights = True
        self._packed: Optional[PackedPattentionWeights] = None
        self.reset_parameters()

    # -- cache state machine (foveal_pattention.py:108-122) -----------------
    def clear_cache(self) -> None:
        """Forget the active block list; the next eval call routes again and, as the
        reference re-gathers the active rows from the current weights
        (foveal_pattention.py:108-122, 310-322), rebuilds the packed copy, so weight
        writes that bypass the version counters (`.data` assignments) are seen.  In
        the pack-in-place mode the packed copy is the weights and stays."""
        self._cached_active_blocks = None
        self._gathered = None
        if not self._released:
            self._packed = None

    def _gathered_rows(self, which: int) -> Optional[Tensor]:
        """Contiguous detached copies of the active rows of (k_gate, k_up, v), made
        only when a caller reads _cached_kg / _cached_ku / _cached_v (the kernels
        never use them), memoised for the current active set."""
        blocks = self._cached_active_blocks
        if blocks is None:
            return None
        g = getattr(self, "_gathered", None)
        if g is None or g[0] is not blocks:
            g = (blocks, *self._active_rows(blocks))
            self._gathered = g
        return g[1 + which]

    def _active_rows(self, blocks: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
        """Detached contiguous rows of k_gate, k_up and v for the given blocks,
        from the parameters or, once they are released, from the packed copy."""
        if self._released:
            return unpack_pattention_weights(self._packed, blocks.reshape(-1).to(torch.int64))
        idx = (blocks.view(-1, 1).to(torch.int64) * self.block_size + self.offsets).flatten()
        return (self.k_gate.detach().index_select(0, idx), self.k_up.detach().index_select(0, idx),
                self.v.detach().index_select(0, idx))

    def _cache_attr_set(self, value) -> None:
        # The reference's caches are plain attributes that callers reset with None
        # to force re-routing (foveal_pattention.py:101-112); anything else is refused.
        if value is not None:
            raise AttributeError("the active-row caches are derived from the active block list; "
                                 "use set_active_blocks() to change them")
        self.clear_cache()

    _cached_kg = property(lambda self: self._gathered_rows(0), _cache_attr_set)
    _cached_ku = property(lambda self: self._gathered_rows(1), _cache_attr_set)
    _cached_v = property(lambda self: self._gathered_rows(2), _cache_attr_set)

    def invalidate_packed_weights(self) -> None:
        """Drop the packed copy of k_gate / k_up / v; the next bf16 eval call repacks.
        Needed after writing the weights through `.data` (such writes do not bump
        the tensors' version counters, which is how in-place changes through the
        parameters themselves are detected).  load_state_dict and module moves
        call it."""
        if self._released:
            raise RuntimeError("the packed copy is the only copy of k_gate / k_up / v "
                               "(release_unpacked_weights); call unpack_weights() first")
        self._packed = None

    # -- pack-in-place inference mode ----------------------------------------
    def release_unpacked_weights(self) -> int:
        """Keep only the packed copy of k_gate, k_up and v and free the parameters'
        storage: decode and prefill read nothing else, so an inference-only
        model holds the MLP weights once instead of twice (336 MiB less per
        Llama-3-8B layer).  Returns the bytes released.

        While released: eval forward runs for bf16 tokens of any count (65..255
        tokens in 64-token pieces of the decode kernels) and still gives input
        gradients; state_dict() returns the weights unpacked from the packed copy,
        and _cached_kg / _cached_ku / _cached_v are unpacked on demand; a module
        move (.to, .cuda, ...) and load_state_dict unpack first.  Training
        forward, fp32 input, calibrate_offline_svd and reset_parameters raise
        until unpack_weights() restores the parameters (bit-exact)."""
        if self._released:
            return 0
        what = "release_unpacked_weights"
        _lib.require_gpu(self.k_gate, what=what)
        if self.k_gate.dtype != torch.bfloat16:
            raise TypeError(f"{what}: bfloat16 weights required, not {self.k_gate.dtype}")
        n_ch = self.total_active_blocks * self.block_size
        for m in (1, PACKED_PREFILL_MIN_M):
            if not packed_decode_supported(m, self.hidden_dim, self.v.shape[1], self.intermediate_dim,
                                           self.block_size, n_ch):
                raise ValueError(f"{what}: the packed kernels do not take this layer's shape "
                                 f"(hidden {self.hidden_dim}, intermediate {self.intermediate_dim}, "
                                 f"block {self.block_size}, {n_ch} active channels)")
        self._packed_weights()
        freed = 0
        for p in (self.k_gate, self.k_up, self.v):
            freed += p.numel() * p.element_size()
            p.data = torch.empty(0, dtype=p.dtype, device=p.device)
        self._released = True
        self._gathered = None
        return freed

    def unpack_weights(self) -> None:
        """Leave the pack-in-place mode: rebuild k_gate, k_up and v from the packed
        copy (bit-exact; v in its down_proj storage order), which stays valid."""
        if not self._released:
            return
        kg, ku, v = unpack_pattention_weights(self._packed)
        self.k_gate.data = kg
        self.k_up.data = ku
        self.v.data = v.t().contiguous().t()
        self._released = False
        self._packed.key = _weights_key(self.k_gate, self.k_up, self.v)

    def _require_unpacked(self, what: str) -> None:
        if self._released:
            raise RuntimeError(f"{what} needs k_gate / k_up / v, which release_unpacked_weights() freed; "
                               "call unpack_weights() first")

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        if self._released:
            kg, ku, v = unpack_pattention_weights(self._packed)
            destination[prefix + "k_gate"] = kg
            destination[prefix + "k_up"] = ku
            destination[prefix + "v"] = v

    def _load_from_state_dict(self, *args, **kwargs):
        self.unpack_weights()
        self.invalidate_packed_weights()
        self._gathered = None
        return super()._load_from_state_dict(*args, **kwargs)

    def _apply(self, fn, *args, **kwargs):
        self.unpack_weights()
        self.invalidate_packed_weights()
        self._gathered = None
        return super()._apply(fn, *args, **kwargs)

    def set_active_blocks(self, active_blocks: Tensor) -> None:
        """Fix the active block list used by later eval calls until clear_cache()."""
        active_blocks = torch.as_tensor(active_blocks)
        if active_blocks.device.type == "cpu" and active_blocks.numel() > 0:
            lo, hi = int(active_blocks.min()), int(active_blocks.max())
            if lo < 0 or hi >= self.num_blocks:
                raise IndexError(f"active block index out of range [0, {self.num_blocks}): min {lo}, max {hi}")
        self._cached_active_blocks = active_blocks.reshape(-1).to(device=self.k_gate.device,
                                                                  dtype=torch.int32).contiguous()
        self._gathered = None

    def reset_parameters(self) -> None:
        self._require_unpacked("reset_parameters")
        std = self.hidden_dim ** -0.5
        nn.init.normal_(self.k_gate, std=std)
        nn.init.normal_(self.k_up, std=std)
        nn.init.normal_(self.v, std=std)
        nn.init.normal_(self.q_proj_16d.weight, std=std)
        nn.init.normal_(self.block_keys_16d, std=self.index_dim ** -0.5)
        nn.init.normal_(self.out_proj_16d.weight, std=1e-3)

    @classmethod
    def from_dense_mlp(
        cls,
        dense_mlp: nn.Module,
        block_size: int = 64,
        base_blocks: int = 4,
        remote_blocks: int = 20,
        index_dim: int = 16,
        temperature: float = 1.0,
        use_fused_kernel: bool = True,
    ) -> "FovealPattentionMLP":
        """Exact reparameterisation K_gate = W_gate, K_up = W_up, V = W_down^T
        (foveal_pattention.py:133-173)."""
        hidden_dim = dense_mlp.gate_proj.in_features
        intermediate_dim = dense_mlp.gate_proj.out_features
        dtype = dense_mlp.gate_proj.weight.dtype
        device = dense_mlp.gate_proj.weight.device
        patt = cls(hidden_dim=hidden_dim, intermediate_dim=intermediate_dim, block_size=block_size,
                   base_blocks=base_blocks, remote_blocks=remote_blocks, index_dim=index_dim,
                   temperature=temperature, dtype=dtype, use_fused_kernel=use_fused_kernel).to(device)
        with torch.no_grad():
            patt.k_gate = nn.Parameter(dense_mlp.gate_proj.weight.data)
            patt.k_up = nn.Parameter(dense_mlp.up_proj.weight.data)
            patt.v = nn.Parameter(dense_mlp.down_proj.weight.data.t())
            nn.init.zeros_(patt.out_proj_16d.weight)
        return patt

    @torch.no_grad()
    def _dense_block_mass_f32(self, X: Tensor, chunk: int = 4096) -> Tensor:
        """E[t, b] = mean_{j in b} |silu(x_t k_gate_j) (x_t k_up_j)| * ||V_b||_F in fp32
        (foveal_pattention.py:201-213), token chunks bounding the (tokens, I)
        activation to `chunk` rows."""
        nb, bs = self.num_blocks, self.block_size
        kg, ku = self.k_gate.float(), self.k_up.float()
        v_norm = self.v.float().reshape(nb, bs, -1).norm(dim=(1, 2))
        out = torch.empty(X.shape[0], nb, dtype=torch.float32, device=X.device)
        for t0 in range(0, X.shape[0], chunk):
            xc = X[t0:t0 + chunk]
            a = F.silu(xc @ kg.t()) * (xc @ ku.t())
            out[t0:t0 + chunk] = a.abs().reshape(xc.shape[0], nb, bs).mean(dim=-1) * v_norm
        return out

    @torch.no_grad()
    def calibrate_offline_svd(self, features: Tensor, ridge_lambda: float = 1e-2) -> Dict[str, Any]:
        """Offline router calibration (foveal_pattention.py:175-255), in fp32 on the
        module's device: q_proj_16d = top-16 right singular vectors of the
        calibration tokens, teacher block energies of the dense SwiGLU, block keys
        by closed-form ridge regression of the rms-normed 16-D projections onto
        the teacher softmax, then the calibration top-k set as the active blocks.
        The SVD, the fp32 products and the solve are library calls (torch.linalg,
        hipBLASLt): this is a one-time conversion step.  Singular vectors carry an
        arbitrary sign per component; the router scores do not depend on it."""
        self._require_unpacked("calibrate_offline_svd")
        _lib.require_gpu(self.k_gate, what="calibrate_offline_svd")
        device = self.k_gate.device
        orig_dtype = self.k_gate.dtype
        X = features.to(device=device, dtype=torch.float32).reshape(-1, self.hidden_dim)
        _, S, Vh = torch.linalg.svd(X, full_matrices=False)
        if Vh.shape[0] < self.index_dim:
            pad = torch.randn(self.index_dim - Vh.shape[0], self.hidden_dim, device=device)
            Vh = torch.cat([Vh, pad], dim=0)
        V16 = Vh[: self.index_dim, :].T
        self.q_proj_16d.weight.data.copy_(V16.T.to(dtype=orig_dtype))
        Z = F.rms_norm(X @ V16, (self.index_dim,))
        teacher_target = F.softmax(self._dense_block_mass_f32(X) / self.temperature, dim=-1)
        reg = ridge_lambda * torch.eye(self.index_dim, device=device)
        block_keys = torch.linalg.solve(Z.T @ Z + reg, Z.T @ teacher_target).T
        self.block_keys_16d.data.copy_(block_keys.to(dtype=orig_dtype))

        scores = (Z @ block_keys.T) / math.sqrt(self.index_dim)
        student_probs = F.softmax(scores / self.temperature, dim=-1)
        kl = F.kl_div(student_probs.log(), teacher_target, reduction="batchmean").item()
        _, top_rem = torch.topk(scores.mean(dim=0)[self.base_blocks:], k=self.remote_blocks)
        calib_active = torch.cat([torch.arange(self.base_blocks, device=device, dtype=torch.int32),
                                  (top_rem + self.base_blocks).to(torch.int32)])
        self.set_active_blocks(calib_active)
        total_var = (S ** 2).sum().item()
        top16_var = (S[: self.index_dim] ** 2).sum().item()
        return {
            "top16_explained_variance": top16_var / max(total_var, 1e-12),
            "initial_kl_divergence": kl,
            "num_blocks": self.num_blocks,
            "active_blocks": self.total_active_blocks,
            "calib_active_blocks": calib_active.tolist(),
            "sparsity_pct": (1.0 - self.total_active_blocks / self.num_blocks) * 100.0,
        }

    def compute_router_scores(self, x: Tensor) -> Tensor:
        """Per-token router scores rms_norm(q_proj(x)) @ K_16^T / sqrt(16)
        (foveal_pattention.py:257-262); reported in router info only."""
        q_16 = F.rms_norm(self.q_proj_16d(x), (self.index_dim,))
        return torch.matmul(q_16, self.block_keys_16d.t()) / math.sqrt(self.index_dim)

    def _decode_packed(self, x_2d: Tensor, active_blocks: Tensor) -> bool:
        return (self.pack_decode_weights and x_2d.dtype == torch.bfloat16 and self.k_gate.dtype == torch.bfloat16
                and packed_decode_supported(x_2d.shape[0], self.hidden_dim, self.v.shape[1], self.intermediate_dim,
                                            self.block_size, active_blocks.numel() * self.block_size))

    def _packed_weights(self) -> PackedPattentionWeights:
        if self._released:
            return self._packed
        key = _weights_key(self.k_gate, self.k_up, self.v)
        if self._packed is None or self._packed.key != key:
            self._packed = None
            self._packed = pack_pattention_weights(self.k_gate.detach(), self.k_up.detach(), self.v.detach(),
                                                   self.block_size)
            self._packed.key = key
        return self._packed

    def _rounding(self) -> str:
        return "fused" if self.use_fused_kernel else "eager"

    def _eval_compute(self, x_2d: Tensor, active_blocks: Tensor) -> Tensor:
        """y = (silu(x K_g,S^T) * (x K_u,S^T)) V_S over the active blocks S on the
        HIP kernels: packed weights for bf16 decode / prefill shapes, the
        parameters in place otherwise."""
        with torch.no_grad():
            if self._released:
                if x_2d.dtype != torch.bfloat16:
                    self._require_unpacked(f"eval forward of {x_2d.dtype} tokens")
                M = x_2d.shape[0]
                if 64 < M < PACKED_PREFILL_MIN_M:  # neither decode nor prefill shape: 64-token pieces
                    return torch.cat([pattention_decode_packed(x_2d[i:i + 64], self._packed, active_blocks,
                                                               rounding=self._rounding())
                                      for i in range(0, M, 64)])
                return pattention_decode_packed(x_2d, self._packed, active_blocks, rounding=self._rounding())
            if self._decode_packed(x_2d, active_blocks):
                return pattention_decode_packed(x_2d, self._packed_weights(), active_blocks,
                                                rounding=self._rounding())
            return pattention_forward(x_2d, self.k_gate, self.k_up, self.v, active_blocks, self.block_size,
                                      activation="swiglu", rounding=self._rounding())

    def _train_forward(self, x_2d: Tensor, orig_shape, return_router_info: bool):
        """Training forward (foveal_pattention.py:292-307, 328-342): per-token
        router scores, top-k of their token mean over the remote blocks, the
        active rows gathered from the parameters, three library GEMMs with the
        HIP SwiGLU (forward and backward kernels) between them, and the additive
        16-D stream softmax(scores / T) @ block_keys -> out_proj_16d.  Gradients
        reach k_gate, k_up, v (active rows), q_proj_16d, block_keys_16d and
        out_proj_16d as in the reference."""
        _lib.require_gpu(x_2d, what="FovealPattentionMLP training forward")
        scores = self.compute_router_scores(x_2d)
        mean_scores = scores.mean(dim=0)
        _, top_remote = torch.topk(mean_scores[self.base_blocks:], k=self.remote_blocks)
        if self.base_blocks > 0:
            active_blocks = torch.cat([
                torch.arange(self.base_blocks, device=x_2d.device, dtype=torch.int32),
                (top_remote + self.base_blocks).to(torch.int32),
            ])
        else:
            active_blocks = top_remote.to(torch.int32)
        indices = (active_blocks.view(-1, 1).to(torch.int64) * self.block_size + self.offsets).flatten()
        kg_proj = F.linear(x_2d, self.k_gate[indices])
        ku_proj = F.linear(x_2d, self.k_up[indices])
        if self.use_fused_kernel:
            act = triton_fused_swiglu(kg_proj, ku_proj)
        else:
            act = F.silu(kg_proj) * ku_proj
        out_patt = F.linear(act, self.v[indices].t())
        soft = F.softmax(scores / self.temperature, dim=-1)
        context_16d = torch.matmul(soft, self.block_keys_16d)
        out = (out_patt + self.out_proj_16d(context_16d)).reshape(*orig_shape)
        if return_router_info:
            return out, {
                "scores": scores,
                "active_blocks": active_blocks,
                "sparsity": (1.0 - self.total_active_blocks / self.num_blocks) * 100.0,
            }
        return out

    def forward(self, x: Tensor, return_router_info: bool = False):
        if self.training:
            self._require_unpacked("training forward")
            return self._train_forward(x.reshape(-1, x.shape[-1]), x.shape, return_router_info)
        orig_shape = x.shape
        D = orig_shape[-1]
        x_2d = x.reshape(-1, D)
        is_prefill = (len(orig_shape) >= 3 and orig_shape[-2] > 1) or (
            len(orig_shape) == 2 and orig_shape[0] > 1 and self.training)

        fast = self._cached_active_blocks is not None and not is_prefill
        if self._cached_active_blocks is None:
            active = mlp_pooled_route(x_2d, self.q_proj_16d.weight, self.block_keys_16d, self.base_blocks,
                                      self.remote_blocks)
            self._cached_active_blocks = active
        active_blocks = self._cached_active_blocks
        if torch.is_grad_enabled() and x_2d.requires_grad:
            out = _EvalPattentionFn.apply(x_2d, self, active_blocks).reshape(*orig_shape)
        else:
            out = self._eval_compute(x_2d, active_blocks).reshape(*orig_shape)
        if return_router_info:
            if fast:
                return out, {"active_blocks": active_blocks}
            return out, {
                "scores": self.compute_router_scores(x_2d),
                "active_blocks": active_blocks,
                "sparsity": (1.0 - self.total_active_blocks / self.num_blocks) * 100.0,
            }
        return out


def release_unpacked_weights(model: nn.Module) -> int:
    """Pack-in-place inference mode for every FovealPattentionMLP in `model`
    (FovealPattentionMLP.release_unpacked_weights); returns the bytes released."""
    return sum(m.release_unpacked_weights() for m in model.modules() if isinstance(m, FovealPattentionMLP))


def sparsify_model_with_foveal_pattention(
    model: nn.Module,
    layers_to_sparsify: Optional[List[int]] = None,
    block_size: int = 64,
    base_blocks: int = 4,
    remote_blocks: int = 20,
    index_dim: int = 16,
    temperature: float = 1.0,
    use_fused_kernel: bool = True,
) -> nn.Module:
    """Replace `model.model.layers[i].mlp` with FovealPattentionMLP (foveal_pattention.py:355-387)."""
    layers = getattr(model, "model", model).layers
    targets = layers_to_sparsify if layers_to_sparsify is not None else list(range(len(layers)))
    for idx in targets:
        if hasattr(layers[idx], "mlp"):
            dense_mlp = layers[idx].mlp
            layers[idx].mlp = FovealPattentionMLP.from_dense_mlp(
                dense_mlp, block_size=block_size, base_blocks=base_blocks, remote_blocks=remote_blocks,
                index_dim=index_dim, temperature=temperature, use_fused_kernel=use_fused_kernel)
            del dense_mlp
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return model


def compute_teacher_dense_block_targets(
    teacher: nn.Module,
    b_ids: Tensor,
    target_layers: list,
    block_size: int = 64,
    temperature: float = 1.0,
) -> Tuple[Tensor, Tensor, List[Tensor]]:
    """Teacher representations and dense block-energy targets for KL
    distillation (archive/hy_mt2/llm_pattention/train_foveal_pattention_speedrun.py:154-189):
    one no-grad teacher forward with hidden states, then for every target
    layer the block targets of its MLP input (post_attention_layernorm of the
    layer's input hidden state) on the fused HIP kernel.  Returns
    (last hidden state, hidden state 16, [P_target per layer]) as the reference."""
    with torch.no_grad():
        t_out = teacher.model(b_ids, output_hidden_states=True)
        t_rep = t_out.last_hidden_state
        t_mid = t_out.hidden_states[16]
        targets = []
        for l_idx in target_layers:
            layer = teacher.model.layers[l_idx]
            mlp = layer.mlp
            norm_h = layer.post_attention_layernorm(t_out.hidden_states[l_idx])
            targets.append(dense_block_targets(norm_h, mlp.gate_proj.weight, mlp.up_proj.weight,
                                               mlp.down_proj.weight, block_size, temperature))
    return t_rep, t_mid, targets


def load_foveal_pattention_mlps(
    checkpoint_dir,
    layers: Optional[Iterable[int]] = None,
    block_size: int = 64,
    base_blocks: int = 4,
    remote_blocks: int = 20,
    index_dim: int = 16,
    temperature: float = 1.0,
    use_fused_kernel: bool = True,
    device=None,
    layer_prefix: str = "model.layers.",
) -> Dict[int, FovealPattentionMLP]:
    """FovealPattentionMLP modules for the MLPs of a local Llama-style Hugging
    Face checkpoint (config.json + *.safetensors, optionally sharded with
    model.safetensors.index.json), built the way from_dense_mlp
    (foveal_pattention.py:133-173) and sparsify_model_with_foveal_pattention
    (:355-387) build them from a loaded model, without instantiating the model:
    each layer's gate_proj / up_proj / down_proj tensors are read with
    safetensors straight onto `device` and become k_gate, k_up and v (v keeps
    down_proj's (hidden, intermediate) storage, the layout the kernels stream).
    The router's q_proj_16d and block_keys_16d get the module's random
    initialisation and out_proj_16d is zero, as in from_dense_mlp."""
    from safetensors import safe_open

    path = Path(checkpoint_dir)
    cfg = json.loads((path / "config.json").read_text())
    hidden, inter, n_layers = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    index = path / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text())["weight_map"]
    else:
        weight_map = {}
        for f in sorted(path.glob("*.safetensors")):
            with safe_open(str(f), framework="pt") as h:
                weight_map.update({k: f.name for k in h.keys()})
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    targets = list(range(n_layers)) if layers is None else list(layers)
    handles: Dict[str, Any] = {}
    out: Dict[int, FovealPattentionMLP] = {}
    try:
        for i in targets:
            if not 0 <= i < n_layers:
                raise IndexError(f"layer {i} outside [0, {n_layers})")
            w = {}
            for p in ("gate", "up", "down"):
                name = f"{layer_prefix}{i}.mlp.{p}_proj.weight"
                if name not in weight_map:
                    raise KeyError(f"{name} not found in {path}")
                f = weight_map[name]
                if f not in handles:
                    handles[f] = safe_open(str(path / f), framework="pt", device=str(dev))
                w[p] = handles[f].get_tensor(name)
            if (tuple(w["gate"].shape) != (inter, hidden) or tuple(w["up"].shape) != (inter, hidden)
                    or tuple(w["down"].shape) != (hidden, inter)):
                raise ValueError(f"layer {i}: gate {tuple(w['gate'].shape)}, up {tuple(w['up'].shape)}, "
                                 f"down {tuple(w['down'].shape)} do not match config ({hidden}, {inter})")
            with torch.device("meta"):
                m = FovealPattentionMLP(hidden_dim=hidden, intermediate_dim=inter, block_size=block_size,
                                        base_blocks=base_blocks, remote_blocks=remote_blocks, index_dim=index_dim,
                                        temperature=temperature, dtype=w["gate"].dtype,
                                        use_fused_kernel=use_fused_kernel)
            m = m.to_empty(device=dev)
            with torch.no_grad():
                m.k_gate = nn.Parameter(w["gate"])
                m.k_up = nn.Parameter(w["up"])
                m.v = nn.Parameter(w["down"].t())
                m.offsets.copy_(torch.arange(block_size, dtype=torch.int64))
                nn.init.normal_(m.q_proj_16d.weight, std=hidden ** -0.5)
                nn.init.normal_(m.block_keys_16d, std=index_dim ** -0.5)
                nn.init.zeros_(m.out_proj_16d.weight)
            out[i] = m
    finally:
        handles.clear()
    return out
