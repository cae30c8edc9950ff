"""16-D Foveal Indexer on MI355X: drop-in for foveal_indexer/core.py.

Same names, signatures, defaults and return structures as the reference
(`Route` core.py:23-33, `masked_softmax` :36-43, `select_blocks` :46-160,
`FovealIndexer` :163-353).  Softmax, ranking, prefix mass, counts, scoring,
pooling and the additive-stream contraction run in the HIP library
(csrc/routing.hip, csrc/indexer.hip); the D -> 16 projections are library
GEMMs (nn.Linear).  masked_softmax and the FovealIndexer representations
(compute_query_16d, compute_kv_blocks_16d, compute_block_scores,
additive_stream) are differentiable through HIP backward kernels, as the
reference's dual-gradient training needs (tests/test_indexer.py:63-101);
select_blocks / route take no gradient (the reference detaches the scores).

Differences by design:
  * equal probabilities are ranked lower index first (torch.sort leaves their
    order unspecified);
  * select_blocks handles up to 65536 blocks per row and
    min(max(K_max, capacity), blocks) <= 256 (RuntimeError beyond);
  * scores must be float32 or bfloat16.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch
from torch import Tensor, nn

from . import _lib


@dataclass
class Route:
    """Routing decisions for foveal block selection (core.py:23-33)."""

    remote_indices: Tensor  # (B, Q_blocks, remote_capacity) int32
    remote_counts: Tensor  # (B, Q_blocks) int32
    base_indices: Optional[Tensor]  # (B, Q_blocks, max_base_blocks) int32
    base_counts: Optional[Tensor]  # (B, Q_blocks) int32
    block_scores: Tensor  # (B, Q_blocks, total_blocks)
    cap_rate: Tensor
    mean_remote_blocks: Tensor
    base_only_rate: Tensor


def _as_3d(scores: Tensor, what: str) -> Tensor:
    if scores.dim() != 3:
        raise ValueError(f"{what}: expected (B, Q_blocks, total_blocks) scores, got {tuple(scores.shape)}")
    return scores.contiguous()


@_lib.fsi_op("masked_softmax", lambda s3, m8: torch.empty_like(s3))
def _masked_softmax_op(s3: Tensor, m8: Tensor) -> Tensor:
    """s3: contiguous (B, Q, N) scores; m8: uint8 mask view over (B, Q, N)."""
    what = "masked_softmax"
    dev = s3.device
    code = _lib.dtype_code(s3.dtype, what)
    out = torch.empty_like(s3)
    B, Q, N = s3.shape
    st = _lib.lib().fsi_masked_softmax(s3.data_ptr(), code, B, Q, N, m8.data_ptr(), m8.stride(0), m8.stride(1),
                                       m8.stride(2), out.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return out


@_lib.fsi_op("masked_softmax_bwd", lambda s3, g, m8: torch.empty_like(s3))
def _masked_softmax_bwd_op(s3: Tensor, g: Tensor, m8: Tensor) -> Tensor:
    what = "masked_softmax backward"
    dev = _lib.require_gpu(g, s3, what=what)
    gc = g.to(s3.dtype).contiguous()
    ds = torch.empty_like(s3)
    B, Q, N = s3.shape
    st = _lib.lib().fsi_masked_softmax_bwd(s3.data_ptr(), gc.data_ptr(), _lib.dtype_code(s3.dtype, what), B, Q, N,
                                           m8.data_ptr(), m8.stride(0), m8.stride(1), m8.stride(2), ds.data_ptr(),
                                           _lib.stream_handle(dev))
    _lib.check(st, what)
    return ds


class _MaskedSoftmaxFn(torch.autograd.Function):
    """fsi_masked_softmax with fsi_masked_softmax_bwd as its gradient."""

    @staticmethod
    def forward(ctx, s3: Tensor, m8: Tensor) -> Tensor:
        ctx.save_for_backward(s3, m8)
        return _masked_softmax_op(s3, m8)

    @staticmethod
    def backward(ctx, g: Tensor):
        s3, m8 = ctx.saved_tensors
        return _masked_softmax_bwd_op(s3, g, m8), None


def masked_softmax(scores: Tensor, mask: Tensor) -> Tensor:
    """Softmax over `mask` with masked entries and all-masked rows exactly zero,
    computed in fp32 and returned in the scores' dtype (core.py:36-43).
    scores: (..., N); mask: bool, broadcastable to scores.  Differentiable in
    the scores."""
    what = "masked_softmax"
    dev = _lib.require_gpu(scores, mask, what=what)
    _lib.dtype_code(scores.dtype, what)
    shape = scores.shape
    if scores.dim() == 0:
        raise ValueError(f"{what}: scores must have at least one dimension")
    N = shape[-1]
    m = torch.broadcast_to(mask.to(device=dev, dtype=torch.bool), shape)
    if scores.dim() == 3:
        s3 = scores.contiguous()
    else:
        s3 = scores.contiguous().reshape(-1, 1, N)
        m = m.reshape(-1, 1, N)
    m8 = m.view(torch.uint8)  # bool and uint8 share the element size; strides carry over
    return _MaskedSoftmaxFn.apply(s3, m8).reshape(shape)


def _per_row(value, B: int, Qb: int, dtype: torch.dtype, dev: torch.device):
    """Scalar -> (python value, None); tensor -> (None, contiguous (B*Qb,) device tensor)."""
    if isinstance(value, Tensor):
        if value.numel() == 1:
            return value.reshape(()).item(), None
        t = torch.broadcast_to(value.to(device=dev, dtype=dtype), (B, Qb)).contiguous().reshape(-1)
        return None, t
    return value, None


def _route_tables(B: int, Qb: int, causal: bool, local_window_blocks: int, dev: torch.device):
    """Base / local block tables of select_blocks (core.py:125-145)."""
    if local_window_blocks <= 0:
        return None, None
    if causal:
        width = local_window_blocks + 1
        offs = torch.arange(width, device=dev)
        qb = torch.arange(Qb, device=dev)
        start = (qb - local_window_blocks).clamp_min(0)
        n_local = qb - start + 1
        base = torch.where(offs[None] < n_local[:, None], start[:, None] + offs[None], torch.zeros_like(offs[None]))
        return base[None].expand(B, -1, -1).to(torch.int32), n_local[None].expand(B, -1).to(torch.int32)
    base = torch.arange(local_window_blocks, device=dev, dtype=torch.int32)[None, None].expand(B, Qb, -1)
    return base, torch.full((B, Qb), local_window_blocks, device=dev, dtype=torch.int32)


def _route_stats(counts: Tensor, max_remote, dev: torch.device):
    kmax_t = torch.as_tensor(max_remote, device=dev, dtype=torch.int64)
    cap_rate = torch.where(kmax_t > 0, (counts >= kmax_t).float().mean(),
                           counts.new_zeros((), dtype=torch.float32))
    return cap_rate, counts.float().mean(), (counts == 0).float().mean()


def _route_fake(scores, causal, local_window_blocks, top_p, k_min, k_max, capacity, p_rows, kmin_rows, kmax_rows,
                kmax_bound):
    B, Qb, _ = scores.shape
    return (scores.new_empty((B, Qb, capacity), dtype=torch.int32), scores.new_empty((B, Qb), dtype=torch.int32))


@_lib.fsi_op("route_from_scores", _route_fake)
def _route_op(scores: Tensor, causal: bool, local_window_blocks: int, top_p: float, k_min: int, k_max: int,
              capacity: int, p_rows: Optional[Tensor], kmin_rows: Optional[Tensor], kmax_rows: Optional[Tensor],
              kmax_bound: int) -> Tuple[Tensor, Tensor]:
    """fsi_route_from_scores: (indices (B, Qb, capacity), counts (B, Qb)) int32."""
    what = "select_blocks"
    dev = scores.device
    B, Qb, Nb = scores.shape
    indices = torch.empty((B, Qb, capacity), dtype=torch.int32, device=dev)
    counts = torch.empty((B, Qb), dtype=torch.int32, device=dev)
    st = _lib.lib().fsi_route_from_scores(
        scores.data_ptr(), _lib.dtype_code(scores.dtype, what), B, Qb, Nb, int(causal), local_window_blocks, top_p,
        k_min, k_max, capacity, _lib.ptr(p_rows), _lib.ptr(kmin_rows), _lib.ptr(kmax_rows), kmax_bound,
        indices.data_ptr(), counts.data_ptr(), None, _lib.stream_handle(dev))
    _lib.check(st, what)
    return indices, counts


def select_blocks(
    block_scores: Tensor,
    *,
    causal: bool = True,
    block_size: int = 64,
    local_window_blocks: int = 0,
    top_p: float | Tensor = 0.95,
    min_remote_blocks: int | Tensor = 0,
    max_remote_blocks: int | Tensor = 16,
    remote_capacity: int = 16,
) -> Route:
    """Adaptive top-p mass routing over block scores (core.py:46-160)."""
    what = "select_blocks"
    dev = _lib.require_gpu(block_scores, what=what)
    scores = _as_3d(block_scores.detach(), what)
    code = _lib.dtype_code(scores.dtype, what)
    B, Qb, Nb = scores.shape
    p_val, p_rows = _per_row(top_p, B, Qb, torch.float32, dev)
    kmin_val, kmin_rows = _per_row(min_remote_blocks, B, Qb, torch.int32, dev)
    kmax_val, kmax_rows = _per_row(max_remote_blocks, B, Qb, torch.int32, dev)
    kmax_bound = int(kmax_rows.max().item()) if kmax_rows is not None and kmax_rows.numel() else 0
    indices, counts = _route_op(scores, bool(causal), int(local_window_blocks),
                                float(p_val if p_val is not None else 0.0), int(kmin_val if kmin_val is not None else 0),
                                int(kmax_val if kmax_val is not None else 0), int(remote_capacity), p_rows, kmin_rows,
                                kmax_rows, kmax_bound)
    base_indices, base_counts = _route_tables(B, Qb, causal, local_window_blocks, dev)
    cap_rate, mean_remote, base_only = _route_stats(counts, max_remote_blocks, dev)
    return Route(remote_indices=indices, remote_counts=counts, base_indices=base_indices, base_counts=base_counts,
                 block_scores=block_scores, cap_rate=cap_rate, mean_remote_blocks=mean_remote,
                 base_only_rate=base_only)


def _score_route_fake(q3, k3, causal, local_window_blocks, top_p, k_min, k_max, capacity, want_mass):
    B, Q, _ = q3.shape
    return (q3.new_empty((B, Q, capacity), dtype=torch.int32), q3.new_empty((B, Q), dtype=torch.int32),
            q3.new_empty((B, Q) if want_mass else (0,), dtype=torch.float32))


@_lib.fsi_op("score_and_route", _score_route_fake)
def _score_route_op(q3: Tensor, k3: Tensor, causal: bool, local_window_blocks: int, top_p: float, k_min: int,
                    k_max: int, capacity: int, want_mass: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """fsi_score_and_route: (indices, counts, mass ((B, Q) fp32, or empty without want_mass))."""
    what = "score_and_route"
    dev = q3.device
    B, Q, d = q3.shape
    Bk, N, _ = k3.shape
    indices = torch.empty((B, Q, capacity), dtype=torch.int32, device=dev)
    counts = torch.empty((B, Q), dtype=torch.int32, device=dev)
    mass = torch.empty((B, Q) if want_mass else (0,), dtype=torch.float32, device=dev)
    st = _lib.lib().fsi_score_and_route(
        q3.data_ptr(), k3.data_ptr(), _lib.dtype_code(q3.dtype, what), B, Q, N, d, 0 if Bk == 1 else N * d,
        int(causal), local_window_blocks, top_p, k_min, k_max, capacity, indices.data_ptr(), counts.data_ptr(),
        mass.data_ptr() if want_mass else None, _lib.stream_handle(dev))
    _lib.check(st, what)
    return indices, counts, mass


def score_and_route(
    q: Tensor,
    k: Tensor,
    *,
    causal: bool = False,
    local_window_blocks: int = 0,
    top_p: float = 0.95,
    min_remote_blocks: int = 0,
    max_remote_blocks: int = 16,
    remote_capacity: int = 16,
    return_mass: bool = False,
):
    """Fused fp32 cosine scoring + select_blocks without materialising scores.

    Equivalent to select_blocks(normalize(q) . normalize(k)^T / sqrt(d)) with
    every step in fp32 (the fp32 form of compute_block_scores, core.py:254-266).
    q: (B, Q, 16) or (Q, 16); k: (B, N, 16), (1, N, 16) or (N, 16) (shared).
    Returns (indices (B, Q, capacity) int32, counts (B, Q) int32[, mass (B, Q) fp32])."""
    what = "score_and_route"
    dev = _lib.require_gpu(q, k, what=what)
    if q.dtype != k.dtype:
        raise TypeError(f"{what}: q {q.dtype} and k {k.dtype} differ")
    code = _lib.dtype_code(q.dtype, what)
    q3 = (q if q.dim() == 3 else q.unsqueeze(0)).contiguous()
    k3 = (k if k.dim() == 3 else k.unsqueeze(0)).contiguous()
    B, Q, d = q3.shape
    Bk, N, dk = k3.shape
    if dk != d or Bk not in (1, B):
        raise ValueError(f"{what}: q {tuple(q3.shape)} and k {tuple(k3.shape)} do not match")
    indices, counts, mass = _score_route_op(q3, k3, bool(causal), int(local_window_blocks), float(top_p),
                                            int(min_remote_blocks), int(max_remote_blocks), int(remote_capacity),
                                            bool(return_mass))
    if return_mass:
        return indices, counts, mass
    return indices, counts


class FovealIndexer(nn.Module):
    """Modular 16-dimensional Foveal Indexer (core.py:163-353)."""

    def __init__(
        self,
        hidden_size: int,
        index_dim: int = 16,
        block_size: int = 64,
        local_window_blocks: int = 8,
        top_p: float = 0.95,
        min_remote_blocks: int = 0,
        max_remote_blocks: int = 16,
        remote_capacity: int = 16,
        causal: bool = True,
        use_additive_stream: bool = True,
        distill_temperature: float = 1.0,
    ):
        super().__init__()
        self.hidden_size = hidden_size
        self.index_dim = index_dim
        self.block_size = block_size
        self.local_window_blocks = local_window_blocks
        self.top_p = top_p
        self.min_remote_blocks = min_remote_blocks
        self.max_remote_blocks = max_remote_blocks
        self.remote_capacity = remote_capacity
        self.causal = causal
        self.use_additive_stream = use_additive_stream
        self.distill_temperature = distill_temperature

        self.q_proj = nn.Linear(hidden_size, index_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, index_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, index_dim, bias=False)
        self.out_proj = nn.Linear(index_dim, hidden_size, bias=False)
        nn.init.normal_(self.q_proj.weight, std=hidden_size ** -0.5)
        nn.init.normal_(self.k_proj.weight, std=hidden_size ** -0.5)
        nn.init.normal_(self.v_proj.weight, std=hidden_size ** -0.5)
        nn.init.normal_(self.out_proj.weight, std=1e-3)

    def compute_query_16d(self, x: Tensor) -> Tensor:
        """rms_norm(q_proj(x)) (core.py:214-222)."""
        what = "compute_query_16d"
        q = self.q_proj(x)
        return index_rms_norm(q, what)

    def compute_kv_blocks_16d(self, x: Tensor) -> tuple[Tensor, Tensor]:
        """Pooled, normalised 16-D keys and mean values per block (core.py:224-250)."""
        what = "compute_kv_blocks_16d"
        if x.ndim == 2:
            x = x.unsqueeze(0)
        batch, n_elements, _ = x.shape
        if n_elements % self.block_size != 0:
            raise ValueError(f"Element length {n_elements} must be divisible by block_size={self.block_size}")
        k_lin = self.k_proj(x)
        v_lin = self.v_proj(x)
        _lib.require_gpu(k_lin, v_lin, what=what)
        _lib.dtype_code(k_lin.dtype, what)
        return _PoolKVFn.apply(k_lin.contiguous(), v_lin.contiguous(), self.block_size)

    def compute_block_scores(self, q_blocks: Tensor, k_blocks: Tensor) -> Tensor:
        """Cosine / sqrt(index_dim) block scores (core.py:254-266)."""
        return block_scores(q_blocks, k_blocks)

    def route(
        self,
        block_scores: Tensor,
        top_p: Optional[float] = None,
        max_remote_blocks: Optional[int] = None,
        min_remote_blocks: Optional[int] = None,
    ) -> Route:
        """Adaptive top-p routing with this module's settings (core.py:268-286)."""
        return select_blocks(
            block_scores.detach(),
            causal=self.causal,
            block_size=self.block_size,
            local_window_blocks=self.local_window_blocks,
            top_p=self.top_p if top_p is None else top_p,
            min_remote_blocks=self.min_remote_blocks if min_remote_blocks is None else min_remote_blocks,
            max_remote_blocks=self.max_remote_blocks if max_remote_blocks is None else max_remote_blocks,
            remote_capacity=self.remote_capacity,
        )

    def additive_stream(self, block_scores: Tensor, v_blocks: Tensor) -> Tensor:
        """Soft 16-D read over the valid blocks, projected to hidden_size and
        repeated over each block's elements (core.py:288-312)."""
        what = "additive_stream"
        _lib.require_gpu(block_scores, v_blocks, what=what)
        if block_scores.dtype != v_blocks.dtype:
            raise TypeError(f"{what}: scores {block_scores.dtype} and values {v_blocks.dtype} differ")
        _lib.dtype_code(v_blocks.dtype, what)
        s = _as_3d(block_scores, what)
        v = v_blocks.contiguous()
        B, Qb, Nb = s.shape
        if tuple(v.shape) != (B, Nb, self.index_dim):
            raise ValueError(f"{what}: values {tuple(v.shape)} != {(B, Nb, self.index_dim)}")
        context = _AdditiveContextFn.apply(s, v, self.causal)
        out_blocks = self.out_proj(context)
        return out_blocks.repeat_interleave(self.block_size, dim=1)

    def distillation_loss(
        self,
        student_scores: Tensor,
        teacher_block_mass: Tensor,
        valid_mask: Optional[Tensor] = None,
    ) -> Tensor:
        """Block-level KL loss of the student scores against the teacher block
        mass (core.py:315-353), on the fused HIP kernels of csrc/distill.hip:
        a masked log-softmax cross-entropy against the teacher mass renormalised
        over the valid blocks (uniform when that mass vanishes), averaged over
        the rows that have a valid block.  Without `valid_mask` the valid set is
        the causal set (key block < query block) or every block.  Differentiable
        in the student scores (the teacher is a constant target)."""
        what = "distillation_loss"
        s = student_scores
        if s.dim() != 3:
            raise ValueError(f"{what}: expected (B, Q_blocks, total_blocks) scores, got {tuple(s.shape)}")
        dev = _lib.require_gpu(s, teacher_block_mass, valid_mask, what=what)
        t = teacher_block_mass
        if t.dtype not in (torch.float32, torch.bfloat16):
            t = t.float()
        t = torch.broadcast_to(t, s.shape).contiguous()
        if valid_mask is None:
            mode, m8 = (1 if self.causal else 0), None
            no_rows = self.causal and s.shape[1] <= 1
        else:
            mode = 2
            vm = valid_mask.to(device=dev, dtype=torch.bool)
            m8 = torch.broadcast_to(vm, s.shape).view(torch.uint8)
            # the loss comes back in fp32; only the no-valid-entry result (scores.sum() * 0)
            # carries the scores' dtype, so only a non-fp32 caller needs the (syncing) check
            no_rows = s.dtype != torch.float32 and not bool(vm.any())
        loss = _DistillKLFn.apply(s.contiguous(), t, mode, m8, float(self.distill_temperature))
        if no_rows:
            # no query block has a candidate: the reference returns scores.sum() * 0
            return loss.to(s.dtype)
        return loss


@_lib.fsi_op("distill_kl", lambda s, t, mode, m8, temperature: (s.new_empty((), dtype=torch.float32),
                                                                   s.new_empty((1,), dtype=torch.int32)))
def _distill_kl_op(s: Tensor, t: Tensor, mode: int, m8: Optional[Tensor], temperature: float) -> Tuple[Tensor, Tensor]:
    """fsi_distill_kl_fwd: (loss () fp32, rows averaged (1,) int32)."""
    what = "distillation_loss"
    dev = s.device
    B, Q, N = s.shape
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    n_rows = torch.empty(1, dtype=torch.int32, device=dev)
    ws = _lib.workspace(dev, L.fsi_distill_kl_workspace_size(B, Q), stream)
    ms = m8.stride() if m8 is not None else (0, 0, 0)
    st = L.fsi_distill_kl_fwd(s.data_ptr(), _lib.dtype_code(s.dtype, what), t.data_ptr(),
                              _lib.dtype_code(t.dtype, what), B, Q, N, mode, _lib.ptr(m8), ms[0], ms[1], ms[2],
                              temperature, loss.data_ptr(), n_rows.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, what)
    return loss, n_rows


@_lib.fsi_op("distill_kl_bwd", lambda s, t, mode, m8, temperature, g, n_rows: torch.empty_like(s))
def _distill_kl_bwd_op(s: Tensor, t: Tensor, mode: int, m8: Optional[Tensor], temperature: float, g: Tensor,
                       n_rows: Tensor) -> Tensor:
    what = "distillation_loss backward"
    dev = s.device
    B, Q, N = s.shape
    ds = torch.empty_like(s)
    g32 = g.detach().to(device=dev, dtype=torch.float32).reshape(1).contiguous()
    ms = m8.stride() if m8 is not None else (0, 0, 0)
    st = _lib.lib().fsi_distill_kl_bwd(s.data_ptr(), _lib.dtype_code(s.dtype, what), t.data_ptr(),
                                       _lib.dtype_code(t.dtype, what), B, Q, N, mode, _lib.ptr(m8), ms[0], ms[1],
                                       ms[2], temperature, g32.data_ptr(), n_rows.data_ptr(), ds.data_ptr(),
                                       _lib.stream_handle(dev))
    _lib.check(st, what)
    return ds


class _DistillKLFn(torch.autograd.Function):
    """fsi_distill_kl_fwd with fsi_distill_kl_bwd as the gradient in the scores."""

    @staticmethod
    def forward(ctx, s: Tensor, t: Tensor, mode: int, m8: Optional[Tensor], temperature: float) -> Tensor:
        loss, n_rows = _distill_kl_op(s, t, mode, m8, temperature)
        ctx.save_for_backward(s, t, m8, n_rows)
        ctx.mode, ctx.temperature = mode, temperature
        return loss

    @staticmethod
    def backward(ctx, g: Tensor):
        s, t, m8, n_rows = ctx.saved_tensors
        return _distill_kl_bwd_op(s, t, ctx.mode, m8, ctx.temperature, g, n_rows), None, None, None, None


@_lib.fsi_op("index_rms_norm", lambda xc, what: torch.empty_like(xc))
def _rms_norm_op(xc: Tensor, what: str) -> Tensor:
    dev = xc.device
    code = _lib.dtype_code(xc.dtype, what)
    d = xc.shape[-1]
    out = torch.empty_like(xc)
    st = _lib.lib().fsi_index_rms_norm(xc.data_ptr(), code, xc.numel() // max(d, 1), d, out.data_ptr(),
                                       _lib.stream_handle(dev))
    _lib.check(st, what)
    return out


@_lib.fsi_op("index_rms_norm_bwd", lambda xc, g, what: torch.empty_like(xc))
def _rms_norm_bwd_op(xc: Tensor, g: Tensor, what: str) -> Tensor:
    dev = _lib.require_gpu(g, xc, what=what)
    gc = g.to(xc.dtype).contiguous()
    dx = torch.empty_like(xc)
    d = xc.shape[-1]
    st = _lib.lib().fsi_index_rms_norm_bwd(xc.data_ptr(), gc.data_ptr(), _lib.dtype_code(xc.dtype, what),
                                           xc.numel() // max(d, 1), d, dx.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return dx


class _IndexRmsNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, xc: Tensor, what: str) -> Tensor:
        ctx.save_for_backward(xc)
        ctx.what = what
        return _rms_norm_op(xc, what)

    @staticmethod
    def backward(ctx, g: Tensor):
        (xc,) = ctx.saved_tensors
        return _rms_norm_bwd_op(xc, g, ctx.what + " backward"), None


def index_rms_norm(x: Tensor, what: str = "index_rms_norm") -> Tensor:
    """F.rms_norm over the last (16-wide) dimension, eps = FLT_EPSILON; differentiable."""
    _lib.require_gpu(x, what=what)
    _lib.dtype_code(x.dtype, what)
    return _IndexRmsNormFn.apply(x.contiguous(), what)


def _pool_fake(k_lin, v_lin, block_size):
    batch, n_elements, d = k_lin.shape
    kb = k_lin.new_empty((batch, n_elements // block_size, d))
    return kb, torch.empty_like(kb)


@_lib.fsi_op("pool_kv", _pool_fake)
def _pool_kv_op(k_lin: Tensor, v_lin: Tensor, block_size: int) -> Tuple[Tensor, Tensor]:
    what = "compute_kv_blocks_16d"
    dev = k_lin.device
    code = _lib.dtype_code(k_lin.dtype, what)
    batch, n_elements, d = k_lin.shape
    nb = n_elements // block_size
    k_blocks = torch.empty((batch, nb, d), dtype=k_lin.dtype, device=dev)
    v_blocks = torch.empty_like(k_blocks)
    st = _lib.lib().fsi_index_pool_kv(k_lin.data_ptr(), v_lin.data_ptr(), code, batch, n_elements, d, block_size,
                                      k_blocks.data_ptr(), v_blocks.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return k_blocks, v_blocks


@_lib.fsi_op("pool_kv_bwd", lambda k_lin, gk, gv, block_size: (torch.empty_like(k_lin), torch.empty_like(k_lin)))
def _pool_kv_bwd_op(k_lin: Tensor, gk: Tensor, gv: Tensor, block_size: int) -> Tuple[Tensor, Tensor]:
    what = "compute_kv_blocks_16d backward"
    dev = _lib.require_gpu(k_lin, what=what)
    batch, n_elements, d = k_lin.shape
    gk = gk.to(k_lin.dtype).contiguous()
    gv = gv.to(k_lin.dtype).contiguous()
    dk, dv = torch.empty_like(k_lin), torch.empty_like(k_lin)
    st = _lib.lib().fsi_index_pool_kv_bwd(k_lin.data_ptr(), gk.data_ptr(), gv.data_ptr(),
                                          _lib.dtype_code(k_lin.dtype, what), batch, n_elements, d, block_size,
                                          dk.data_ptr(), dv.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return dk, dv


class _PoolKVFn(torch.autograd.Function):
    """fsi_index_pool_kv with fsi_index_pool_kv_bwd as its gradient (B, N, 16) inputs."""

    @staticmethod
    def forward(ctx, k_lin: Tensor, v_lin: Tensor, block_size: int):
        ctx.save_for_backward(k_lin)
        ctx.block_size = block_size
        return _pool_kv_op(k_lin, v_lin, block_size)

    @staticmethod
    def backward(ctx, gk: Optional[Tensor], gv: Optional[Tensor]):
        (k_lin,) = ctx.saved_tensors
        batch, n_elements, d = k_lin.shape
        nb = n_elements // ctx.block_size
        zeros = lambda: k_lin.new_zeros((batch, nb, d))  # noqa: E731
        gk = zeros() if gk is None else gk
        gv = zeros() if gv is None else gv
        dk, dv = _pool_kv_bwd_op(k_lin, gk, gv, ctx.block_size)
        return dk, dv, None


@_lib.fsi_op("block_scores", lambda q, k: q.new_empty((q.shape[0], q.shape[1], k.shape[1])))
def _block_scores_op(q: Tensor, k: Tensor) -> Tensor:
    what = "compute_block_scores"
    dev = q.device
    B, Q, d = q.shape
    N = k.shape[1]
    out = torch.empty((B, Q, N), dtype=q.dtype, device=dev)
    st = _lib.lib().fsi_block_scores(q.data_ptr(), k.data_ptr(), _lib.dtype_code(q.dtype, what), B, Q, N, d,
                                     out.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return out


@_lib.fsi_op("block_scores_bwd", lambda q, k, g: (torch.empty_like(q), torch.empty_like(k)))
def _block_scores_bwd_op(q: Tensor, k: Tensor, g: Tensor) -> Tuple[Tensor, Tensor]:
    what = "compute_block_scores backward"
    dev = _lib.require_gpu(g, q, k, what=what)
    gc = g.to(q.dtype).contiguous()
    B, Q, d = q.shape
    N = k.shape[1]
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    st = _lib.lib().fsi_block_scores_bwd(q.data_ptr(), k.data_ptr(), gc.data_ptr(), _lib.dtype_code(q.dtype, what),
                                         B, Q, N, d, dq.data_ptr(), dk.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return dq, dk


class _BlockScoresFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q: Tensor, k: Tensor) -> Tensor:
        ctx.save_for_backward(q, k)
        return _block_scores_op(q, k)

    @staticmethod
    def backward(ctx, g: Tensor):
        q, k = ctx.saved_tensors
        return _block_scores_bwd_op(q, k, g)


@_lib.fsi_op("additive_context", lambda s, v, causal: v.new_empty((s.shape[0], s.shape[1], v.shape[-1])))
def _additive_context_op(s: Tensor, v: Tensor, causal: bool) -> Tensor:
    what = "additive_stream"
    dev = s.device
    B, Qb, Nb = s.shape
    d = v.shape[-1]
    context = torch.empty((B, Qb, d), dtype=v.dtype, device=dev)
    st = _lib.lib().fsi_additive_context(s.data_ptr(), v.data_ptr(), _lib.dtype_code(v.dtype, what), B, Qb, Nb, d,
                                         int(causal), context.data_ptr(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return context


@_lib.fsi_op("additive_context_bwd", lambda s, v, g, causal: (torch.empty_like(s), torch.empty_like(v)))
def _additive_context_bwd_op(s: Tensor, v: Tensor, g: Tensor, causal: bool) -> Tuple[Tensor, Tensor]:
    what = "additive_stream backward"
    dev = _lib.require_gpu(g, s, v, what=what)
    gc = g.to(v.dtype).contiguous()
    B, Qb, Nb = s.shape
    d = v.shape[-1]
    ds, dv = torch.empty_like(s), torch.empty_like(v)
    lib = _lib.lib()
    ws = torch.empty(max(1, lib.fsi_additive_context_bwd_workspace_size(B, Qb)), dtype=torch.uint8, device=dev)
    st = lib.fsi_additive_context_bwd(s.data_ptr(), v.data_ptr(), gc.data_ptr(), _lib.dtype_code(v.dtype, what),
                                      B, Qb, Nb, d, int(causal), ds.data_ptr(), dv.data_ptr(), ws.data_ptr(),
                                      ws.numel(), _lib.stream_handle(dev))
    _lib.check(st, what)
    return ds, dv


class _AdditiveContextFn(torch.autograd.Function):
    """context = masked_softmax(scores, causal ? p < q : all).to(v) @ v (core.py:296-309)."""

    @staticmethod
    def forward(ctx, s: Tensor, v: Tensor, causal: bool) -> Tensor:
        ctx.save_for_backward(s, v)
        ctx.causal = bool(causal)
        return _additive_context_op(s, v, bool(causal))

    @staticmethod
    def backward(ctx, g: Tensor):
        s, v = ctx.saved_tensors
        ds, dv = _additive_context_bwd_op(s, v, g, ctx.causal)
        return ds, dv, None


def block_scores(q_blocks: Tensor, k_blocks: Tensor) -> Tensor:
    """normalize(q) . normalize(k)^T / sqrt(d) with the reference's rounding
    points (core.py:254-266); differentiable.  q: (B, Q, 16); k: (B, N, 16)."""
    what = "compute_block_scores"
    _lib.require_gpu(q_blocks, k_blocks, what=what)
    if q_blocks.dtype != k_blocks.dtype:
        raise TypeError(f"{what}: q {q_blocks.dtype} and k {k_blocks.dtype} differ")
    _lib.dtype_code(q_blocks.dtype, what)
    q = q_blocks.contiguous()
    k = k_blocks.contiguous()
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError(f"{what}: q {tuple(q.shape)} and k {tuple(k.shape)} do not match")
    return _BlockScoresFn.apply(q, k)
