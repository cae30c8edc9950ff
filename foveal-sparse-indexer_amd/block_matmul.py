"""Block-sparse linear layers on MI355X: drop-in for foveal_indexer/block_matmul.py
and triton_block_sparse_linear (foveal_indexer/triton_ops.py:316-370).

The GEMMs run on the HIP block-sparse MFMA engine (csrc/bsgemm.hip): active
column blocks (BlockSparseLinear) or active 2-D tiles (BlockwiseMatMul2D) are
read straight from the full weight, no gathered copies.  BlockSparseLinear's
routing (16-D scores, per-token top-p, union of blocks) runs in the HIP routing
kernels; BlockwiseMatMul2D's tile routing (per-token top-p over all tiles, union
mask) runs in the HIP tile router (csrc/tile_route.hip).
"""
from __future__ import annotations

import math
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _lib
from .core import FovealIndexer, Route, _AdditiveContextFn, _PoolKVFn, masked_softmax, select_blocks


def _linear_launch(x2d: Tensor, weight: Tensor, bias: Optional[Tensor], idx: Tensor, block_size: int,
                   out: Tensor) -> Tensor:
    what = "block_sparse_linear"
    dev = x2d.device
    M, K = x2d.shape
    N = weight.shape[0]
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    ws = _lib.workspace(dev, L.fsi_block_sparse_linear_workspace_size(N, block_size), stream)
    err = _lib.error_word(dev)
    st = L.fsi_block_sparse_linear(x2d.data_ptr(), x2d.stride(0), weight.data_ptr(), weight.stride(0),
                                   _lib.ptr(bias), idx.data_ptr() if idx.numel() else None, idx.numel(), block_size,
                                   M, N, K, _lib.dtype_code(x2d.dtype, what), out.data_ptr(), out.stride(0),
                                   ws.data_ptr(), ws.numel(), err.data_ptr(), stream)
    _lib.check(st, what)
    if _lib.checks_enabled():
        _lib.raise_device_errors(dev, what)
    return out


@_lib.fsi_op("block_sparse_linear", lambda x2d, weight, bias, idx, block_size:
             x2d.new_empty((x2d.shape[0], weight.shape[0])))
def _linear_op(x2d: Tensor, weight: Tensor, bias: Optional[Tensor], idx: Tensor, block_size: int) -> Tensor:
    """fsi_block_sparse_linear into a new (M, N) tensor."""
    out = torch.empty((x2d.shape[0], weight.shape[0]), dtype=x2d.dtype, device=x2d.device)
    return _linear_launch(x2d, weight, bias, idx, block_size, out)


def _column_mask(idx: Tensor, n_blocks: int, block_size: int) -> Tensor:
    """(N,) float mask of the active column blocks' output columns."""
    m = torch.zeros(n_blocks, dtype=torch.float32, device=idx.device)
    if idx.numel():
        m[idx.long()] = 1.0
    return m.repeat_interleave(block_size)


class _BlockSparseLinearFn(torch.autograd.Function):
    """Column-block sparse linear on the HIP kernels with the gradients of the
    reference's gather -> F.linear -> scatter (block_matmul.py:215-232):
    dy restricted to the active columns, dx = dy_S W_S, dW_S = dy_S^T x,
    dbias_S = sum(dy_S) — library GEMMs on the restricted dy."""

    @staticmethod
    def forward(ctx, x2d, weight, bias, idx, block_size):
        out = _linear_op(x2d, weight, bias, idx, block_size)
        ctx.save_for_backward(x2d, weight, idx)
        ctx.block_size, ctx.has_bias = block_size, bias is not None
        return out

    @staticmethod
    def backward(ctx, dy):
        x2d, weight, idx = ctx.saved_tensors
        cm = _column_mask(idx, weight.shape[0] // ctx.block_size, ctx.block_size).to(dy.dtype)
        dys = dy * cm
        dx = dys @ weight
        dw = dys.t() @ x2d
        db = dys.sum(0) if ctx.has_bias else None
        return dx, dw, db, None, None


def block_sparse_linear(x2d: Tensor, weight: Tensor, bias: Optional[Tensor], active_blocks: Tensor,
                        block_size: int, out: Optional[Tensor] = None) -> Tensor:
    """out = zeros; out[:, blk] = x w[blk]^T (+ bias[blk]) for the active column
    blocks.  fp32 or bf16 (fp32 accumulation); differentiable in x, weight and
    bias."""
    what = "block_sparse_linear"
    dev = _lib.require_gpu(x2d, weight, bias, what=what)
    if x2d.dtype != weight.dtype or (bias is not None and bias.dtype != x2d.dtype):
        raise TypeError(f"{what}: x {x2d.dtype}, weight {weight.dtype} and bias dtypes differ")
    _lib.dtype_code(x2d.dtype, what)
    x2d = x2d.contiguous()
    weight = weight.contiguous()
    bias = bias.contiguous() if bias is not None else None
    M, K = x2d.shape
    N, K2 = weight.shape
    if K2 != K:
        raise ValueError(f"{what}: K mismatch {K} vs {K2}")
    idx = torch.as_tensor(active_blocks).reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x2d, weight, bias)):
        res = _BlockSparseLinearFn.apply(x2d, weight, bias, idx, int(block_size))
        if out is not None:
            out.copy_(res.detach())
        return res
    if out is None:
        return _linear_op(x2d, weight, bias, idx, int(block_size))
    return _linear_launch(x2d, weight, bias, idx, int(block_size), out)


def triton_block_sparse_linear(x: Tensor, weight: Tensor, bias: Optional[Tensor], active_block_indices: Tensor,
                               block_size: int = 32) -> Tensor:
    """Block-sparse linear Y = X W_active^T (+ bias) (triton_ops.py:316-370); the
    `triton_` name is kept for compatibility, the kernel is HIP."""
    if not x.is_cuda:
        raise RuntimeError("Block-Sparse Linear requires a ROCm GPU (no CPU path).")
    M, K = x.shape
    N, K_w = weight.shape
    assert K == K_w, f"K mismatch: {K} vs {K_w}"
    return block_sparse_linear(x, weight, bias, active_block_indices, block_size)


def blockwise_matmul(x2d: Tensor, weight: Tensor, tile_mask: Tensor, block_k: int, block_n: int,
                     rows_per_group: Optional[int] = None, out: Optional[Tensor] = None) -> Tensor:
    """out = x (weight o expand(tile_mask))^T.  tile_mask: bool (T,) or (groups, T)
    with tile id k_b * (N / block_n) + n_b (block_matmul.py:384-385); with
    groups > 1, row group g covers rows [g rows_per_group, (g+1) rows_per_group)
    and the groups must cover every row (ValueError otherwise); one group
    applies to every row whatever rows_per_group says."""
    what = "blockwise_matmul"
    dev = _lib.require_gpu(x2d, weight, tile_mask, what=what)
    if x2d.dtype != weight.dtype:
        raise TypeError(f"{what}: x {x2d.dtype} and weight {weight.dtype} differ")
    _lib.dtype_code(x2d.dtype, what)
    x2d = x2d.contiguous()
    weight = weight.contiguous()
    M, K = x2d.shape
    mask = tile_mask.to(device=dev)
    if mask.dim() == 1:
        mask = mask[None]
    rpg = rows_per_group if rows_per_group is not None else max(M, 1)
    if mask.shape[0] == 1:
        rpg = max(M, 1)
    elif int(rpg) <= 0 or mask.shape[0] * int(rpg) < M:
        raise ValueError(f"{what}: {mask.shape[0]} row groups of {rpg} rows do not cover {M} rows")
    # bool and uint8 masks are read in place as bytes (any nonzero byte is active)
    if mask.dtype == torch.bool:
        m8 = mask.contiguous().view(torch.uint8)
    elif mask.dtype == torch.uint8:
        m8 = mask.contiguous()
    else:
        m8 = (mask != 0).to(torch.uint8).contiguous()
    if torch.is_grad_enabled() and (x2d.requires_grad or weight.requires_grad):
        res = _BlockwiseMatmulFn.apply(x2d, weight, m8, int(block_k), int(block_n), int(rpg))
        if out is not None:
            out.copy_(res.detach())
        return res
    if out is None:
        return _blockwise_op(x2d, weight, m8, int(block_k), int(block_n), int(rpg))
    return _blockwise_launch(x2d, weight, m8, int(block_k), int(block_n), int(rpg), out)


def _blockwise_launch(x2d: Tensor, weight: Tensor, m8: Tensor, block_k: int, block_n: int, rpg: int,
                      out: Tensor) -> Tensor:
    what = "blockwise_matmul"
    dev = x2d.device
    M, K = x2d.shape
    N = weight.shape[0]
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    ws = _lib.workspace(dev, L.fsi_blockwise_matmul_workspace_size(M, N, K, block_k), stream)
    st = L.fsi_blockwise_matmul(x2d.data_ptr(), x2d.stride(0), weight.data_ptr(), weight.stride(0), m8.data_ptr(),
                                m8.shape[0], rpg, block_k, block_n, M, N, K, _lib.dtype_code(x2d.dtype, what),
                                out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, what)
    return out


@_lib.fsi_op("blockwise_matmul", lambda x2d, weight, m8, block_k, block_n, rpg:
             x2d.new_empty((x2d.shape[0], weight.shape[0])))
def _blockwise_op(x2d: Tensor, weight: Tensor, m8: Tensor, block_k: int, block_n: int, rpg: int) -> Tensor:
    """fsi_blockwise_matmul into a new (M, N) tensor."""
    out = torch.empty((x2d.shape[0], weight.shape[0]), dtype=x2d.dtype, device=x2d.device)
    return _blockwise_launch(x2d, weight, m8, block_k, block_n, rpg, out)


def _expand_tiles(m: Tensor, N: int, K: int, block_k: int, block_n: int) -> Tensor:
    """(nkb * nnb,) k-major tile mask -> (N, K) element mask of the weight."""
    nkb, nnb = K // block_k, N // block_n
    return m.view(nkb, nnb).t().repeat_interleave(block_n, 0).repeat_interleave(block_k, 1)


class _BlockwiseMatmulFn(torch.autograd.Function):
    """2-D tile-sparse matmul on the HIP kernels with the gradients of the
    reference's per-tile F.linear sum (block_matmul.py:381-392), i.e. of
    x (W o M)^T: dx = dy (W o M), dW = (dy^T x) o M, row group by row group —
    library GEMMs in the backward."""

    @staticmethod
    def forward(ctx, x2d, weight, m8, block_k, block_n, rpg):
        out = _blockwise_op(x2d, weight, m8, block_k, block_n, rpg)
        ctx.save_for_backward(x2d, weight, m8)
        ctx.meta = (block_k, block_n, rpg)
        return out

    @staticmethod
    def backward(ctx, dy):
        x2d, weight, m8 = ctx.saved_tensors
        block_k, block_n, rpg = ctx.meta
        N, K = weight.shape
        M = x2d.shape[0]
        dx = torch.zeros_like(x2d)
        dw = torch.zeros_like(weight)
        for g in range(m8.shape[0]):  # the groups cover every row (checked in blockwise_matmul)
            rows = slice(min(g * rpg, M), min((g + 1) * rpg, M))
            em = _expand_tiles(m8[g].bool(), N, K, block_k, block_n).to(weight.dtype)
            dx[rows] = dy[rows] @ (weight * em)
            dw += (dy[rows].t() @ x2d[rows]) * em
        return dx, dw, None, None, None, None


def tile_route(scores: Tensor, top_p: float, base_tiles: int, rows_per_group: Optional[int] = None):
    """BlockwiseMatMul2D's tile selection (block_matmul.py:364-377) on the HIP
    router (fsi_tile_route): per token row, softmax over all tiles, the tiles
    whose sorted running mass stays below top_p plus the one that crosses it
    (no K_min, no K_max), and the union over rows with tiles [0, base_tiles).

    scores: (rows, T) fp32 or bf16.  rows_per_group: one union per group of that
    many consecutive rows (None: one union over all rows, as the reference).
    Returns (mask (groups, T) bool, probs (rows, T) in the scores' dtype,
    needed (rows,) int32)."""
    what = "tile_route"
    dev = _lib.require_gpu(scores, what=what)
    code = _lib.dtype_code(scores.dtype, what)
    if scores.dim() != 2:
        raise ValueError(f"{what}: scores must be (rows, tiles), got {tuple(scores.shape)}")
    if scores.stride(1) != 1:
        scores = scores.contiguous()
    rows = scores.shape[0]
    rpg = max(rows, 1) if rows_per_group is None else int(rows_per_group)
    mask, probs, needed = _tile_route_op(scores, float(top_p), int(base_tiles), rpg)
    return mask.view(torch.bool), probs, needed


def _tile_route_fake(scores, top_p, base_tiles, rpg):
    rows, T = scores.shape
    groups = max(1, -(-rows // rpg)) if rows else 1
    return (scores.new_empty((groups, T), dtype=torch.uint8), scores.new_empty((rows, T)),
            scores.new_empty((rows,), dtype=torch.int32))


@_lib.fsi_op("tile_route", _tile_route_fake)
def _tile_route_op(scores: Tensor, top_p: float, base_tiles: int, rpg: int) -> Tuple[Tensor, Tensor, Tensor]:
    """fsi_tile_route: (mask (groups, T) uint8, probs (rows, T), needed (rows,) int32)."""
    what = "tile_route"
    dev = scores.device
    rows, T = scores.shape
    groups = max(1, -(-rows // rpg)) if rows else 1
    mask = torch.empty((groups, T), dtype=torch.uint8, device=dev)
    probs = torch.empty((rows, T), dtype=scores.dtype, device=dev)
    needed = torch.empty((rows,), dtype=torch.int32, device=dev)
    st = _lib.lib().fsi_tile_route(scores.data_ptr() if rows else None, _lib.dtype_code(scores.dtype, what), rows, T,
                                   max(scores.stride(0), T), rpg, base_tiles, top_p, mask.data_ptr(),
                                   needed.data_ptr() if rows else None, probs.data_ptr() if rows else None,
                                   _lib.stream_handle(dev))
    _lib.check(st, what)
    return mask, probs, needed


def _eval_active_blocks(block_scores: Tensor, base_blocks: int, top_p: float, max_remote: int, num_blocks: int):
    """BlockSparseLinear's inference selection (block_matmul.py:168-185): per token,
    softmax over the remote blocks, needed = clamp(#(cum < top_p) + 1, 0, K_max)
    top blocks; the active set is the base blocks plus the union over tokens.
    Returns (sorted active block ids int32, mean needed)."""
    dev = block_scores.device
    B, T, nb = block_scores.shape
    mask = torch.zeros(num_blocks, dtype=torch.bool, device=dev)
    mask[:base_blocks] = True
    remote = block_scores[..., base_blocks:]
    mean_needed = 0.0
    if remote.shape[-1] > 0:
        r = select_blocks(remote.contiguous(), causal=False, local_window_blocks=0, top_p=top_p,
                          min_remote_blocks=0, max_remote_blocks=max_remote, remote_capacity=max(max_remote, 1))
        cap = r.remote_indices.shape[-1]
        valid = torch.arange(cap, device=dev).view(1, 1, cap) < r.remote_counts[..., None]
        sel = r.remote_indices[valid].long() + base_blocks
        if sel.numel():
            mask[sel] = True
        mean_needed = float(r.remote_counts.float().mean())
    return torch.where(mask)[0].to(torch.int32), mean_needed


class BlockSparseLinear(nn.Module):
    """Linear projection with blockwise dynamic sparsity (block_matmul.py:26-282)."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        block_size: int = 64,
        base_blocks: int = 2,
        index_dim: int = 16,
        top_p: float = 0.95,
        min_remote_blocks: int = 0,
        max_remote_blocks: int = 8,
        remote_capacity: int = 8,
        use_additive_stream: bool = True,
        bias: bool = False,
        dtype: Optional[torch.dtype] = None,
    ):
        super().__init__()
        if out_features % block_size != 0:
            raise ValueError(f"out_features ({out_features}) must be divisible by block_size ({block_size})")
        self.in_features = in_features
        self.out_features = out_features
        self.block_size = block_size
        self.num_blocks = out_features // block_size
        self.base_blocks = min(base_blocks, self.num_blocks)
        self.use_additive_stream = use_additive_stream
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=dtype))
        if bias:
            self.bias = nn.Parameter(torch.empty(out_features, dtype=dtype))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()
        self.indexer = FovealIndexer(
            hidden_size=in_features, index_dim=index_dim, block_size=block_size,
            local_window_blocks=self.base_blocks, top_p=top_p, min_remote_blocks=min_remote_blocks,
            max_remote_blocks=max_remote_blocks, remote_capacity=remote_capacity, causal=False,
            use_additive_stream=use_additive_stream,
        ).to(dtype if dtype is not None else torch.get_default_dtype())
        self.weight_to_k = nn.Linear(in_features, index_dim, bias=False, dtype=dtype)
        self.weight_to_v = nn.Linear(in_features, index_dim, bias=False, dtype=dtype)
        self.indexer.out_proj = nn.Linear(index_dim, out_features, bias=False, dtype=dtype)
        nn.init.normal_(self.weight_to_k.weight, std=in_features ** -0.5)
        nn.init.normal_(self.weight_to_v.weight, std=in_features ** -0.5)
        nn.init.normal_(self.indexer.out_proj.weight, std=1e-3)
        self._cached_kp: Optional[Tensor] = None
        self._cached_vp: Optional[Tensor] = None

    def reset_parameters(self) -> None:
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        if self.bias is not None:
            fan_in = self.weight.shape[1]
            bound = 1 / math.sqrt(fan_in) if fan_in > 0 else 0
            nn.init.uniform_(self.bias, -bound, bound)

    def refresh_block_cache(self) -> None:
        with torch.no_grad():
            self._cached_kp, self._cached_vp = self.get_block_keys_and_values()

    def get_block_keys_and_values(self) -> Tuple[Tensor, Tensor]:
        """Pooled 16-D key and value per weight block (block_matmul.py:109-128);
        differentiable in the weight and the two 16-D projections."""
        what = "get_block_keys_and_values"
        k_lin = self.weight_to_k(self.weight).contiguous()
        v_lin = self.weight_to_v(self.weight).contiguous()
        _lib.require_gpu(k_lin, v_lin, what=what)
        _lib.dtype_code(k_lin.dtype, what)
        return _PoolKVFn.apply(k_lin.unsqueeze(0), v_lin.unsqueeze(0), self.block_size)

    def forward(self, x: Tensor, compute_teacher_loss: bool = False) -> Tuple[Tensor, Dict[str, Any]]:
        orig_ndim = x.ndim
        if orig_ndim == 2:
            x = x.unsqueeze(1)
        batch, seq_len, in_feat = x.shape
        device = x.device
        q_16d = self.indexer.compute_query_16d(x.detach())
        if not self.training and self._cached_kp is not None:
            kp_16d, vp_16d = self._cached_kp, self._cached_vp
        else:
            kp_16d, vp_16d = self.get_block_keys_and_values()
            if not self.training:
                self._cached_kp, self._cached_vp = kp_16d, vp_16d
        kp_16d = kp_16d.expand(batch, -1, -1)
        vp_16d = vp_16d.expand(batch, -1, -1)
        block_scores = self.indexer.compute_block_scores(q_16d, kp_16d)

        route: Optional[Route] = None
        if not self.training and not torch.is_grad_enabled():
            active, mean_remote = _eval_active_blocks(block_scores, self.base_blocks, self.indexer.top_p,
                                                      self.indexer.max_remote_blocks, self.num_blocks)
        else:
            route = self.indexer.route(block_scores)
            mask = torch.zeros(self.num_blocks, dtype=torch.bool, device=device)
            mask[: self.base_blocks] = True
            cap = route.remote_indices.shape[-1]
            valid = torch.arange(cap, device=device).view(1, 1, cap) < route.remote_counts[..., None]
            sel = route.remote_indices[valid]
            sel = sel[sel >= self.base_blocks]
            if sel.numel() > 0:
                mask[sel.long()] = True
            active = torch.where(mask)[0].to(torch.int32)
            mean_remote = float(route.mean_remote_blocks)
        num_active = int(active.numel())

        out = block_sparse_linear(x.reshape(batch * seq_len, in_feat), self.weight, self.bias, active,
                                  self.block_size).view(batch, seq_len, self.out_features)
        additive_out = None
        if self.use_additive_stream:
            ctx = _additive_context(block_scores, vp_16d)
            additive_out = self.indexer.out_proj(ctx).to(out.dtype)
            out = out + additive_out
        if orig_ndim == 2:
            out = out.squeeze(1)
        mean_active = self.base_blocks + mean_remote
        aux: Dict[str, Any] = {
            "route": route,
            "additive_out": additive_out,
            "active_blocks_union": num_active,
            "mean_active_blocks": mean_active,
            "total_blocks": self.num_blocks,
            "sparsity": 1.0 - (mean_active / self.num_blocks),
            "distill_loss": torch.tensor(0.0, device=device),
        }
        if compute_teacher_loss:
            with torch.no_grad():
                dense_out = F.linear(x, self.weight, self.bias)
                energy = torch.norm(dense_out.view(batch, seq_len, self.num_blocks, self.block_size), p=2, dim=-1)
                teacher = F.softmax(energy, dim=-1)
            aux["distill_loss"] = self.indexer.distillation_loss(block_scores, teacher)
        return out, aux


def _additive_context(scores: Tensor, v_blocks: Tensor) -> Tensor:
    """softmax over every block (probabilities in the values' dtype) times the
    block values (block_matmul.py:257-260)."""
    what = "additive_stream"
    _lib.require_gpu(scores, v_blocks, what=what)
    s = scores.to(v_blocks.dtype).contiguous() if scores.dtype != v_blocks.dtype else scores.contiguous()
    # differentiable in the scores and the block values (HIP backward kernels)
    return _AdditiveContextFn.apply(s, v_blocks.contiguous(), False)


class BlockwiseMatMul2D(nn.Module):
    """2-D tile-sparse matmul (block_matmul.py:285-419)."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        block_k: int = 64,
        block_n: int = 64,
        base_tiles_ratio: float = 0.25,
        index_dim: int = 16,
        top_p: float = 0.95,
        dtype: Optional[torch.dtype] = None,
    ):
        super().__init__()
        if in_features % block_k != 0 or out_features % block_n != 0:
            raise ValueError(f"Shapes ({in_features}, {out_features}) must be divisible by "
                             f"tile sizes ({block_k}, {block_n})")
        self.in_features = in_features
        self.out_features = out_features
        self.block_k = block_k
        self.block_n = block_n
        self.num_k_blocks = in_features // block_k
        self.num_n_blocks = out_features // block_n
        self.total_tiles = self.num_k_blocks * self.num_n_blocks
        self.base_tiles = max(1, int(self.total_tiles * base_tiles_ratio))
        self.weight = nn.Parameter(torch.empty(out_features, in_features, dtype=dtype))
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        self.tile_q = nn.Linear(block_k, index_dim, bias=False, dtype=dtype)
        self.tile_k = nn.Linear(block_k * block_n, index_dim, bias=False, dtype=dtype)
        self.tile_v = nn.Linear(block_k * block_n, index_dim, bias=False, dtype=dtype)
        self.out_proj = nn.Linear(index_dim, out_features, bias=False, dtype=dtype)
        nn.init.normal_(self.tile_q.weight, std=block_k ** -0.5)
        nn.init.normal_(self.tile_k.weight, std=(block_k * block_n) ** -0.5)
        nn.init.normal_(self.tile_v.weight, std=(block_k * block_n) ** -0.5)
        nn.init.normal_(self.out_proj.weight, std=1e-3)
        self.top_p = top_p
        self.index_dim = index_dim

    def tile_keys_and_values(self) -> Tuple[Tensor, Tensor]:
        """16-D key (normalised) and value of every tile (block_matmul.py:341-353)."""
        w_tiles = (self.weight.view(self.num_n_blocks, self.block_n, self.num_k_blocks, self.block_k)
                   .permute(2, 0, 1, 3).contiguous().view(self.total_tiles, self.block_n * self.block_k))
        tile_k = F.normalize(F.rms_norm(self.tile_k(w_tiles), (self.index_dim,)), dim=-1)
        tile_v = self.tile_v(w_tiles)
        return tile_k, tile_v

    def route_tiles(self, x: Tensor):
        """Per-token top-p over all tiles, union with the base tiles
        (block_matmul.py:355-379).  Returns (tile mask, probs, scores)."""
        batch, seq_len, _ = x.shape
        tile_k, tile_v = self.tile_keys_and_values()
        x_k = x.view(batch, seq_len, self.num_k_blocks, self.block_k).mean(dim=2)
        q_16d = F.normalize(F.rms_norm(self.tile_q(x_k), (self.index_dim,)), dim=-1)
        # plain 2-D products with contiguous operands (no batched bf16 product on a transposed view)
        scores = (q_16d.reshape(-1, self.index_dim) @ tile_k.t().contiguous()).view(batch, seq_len, -1)
        scores = scores / math.sqrt(self.index_dim)
        mask, probs, _ = tile_route(scores.detach().reshape(-1, self.total_tiles), self.top_p, self.base_tiles)
        return mask[0], probs.view(batch, seq_len, -1), scores, tile_v

    def forward(self, x: Tensor, compute_teacher_loss: bool = False) -> Tuple[Tensor, Dict[str, Any]]:
        batch, seq_len, _ = x.shape
        device = x.device
        mask, probs, scores, tile_v = self.route_tiles(x)
        n_active = int(mask.sum())
        out = blockwise_matmul(x.reshape(batch * seq_len, self.in_features), self.weight, mask, self.block_k,
                               self.block_n).view(batch, seq_len, self.out_features)
        if torch.is_grad_enabled() and scores.requires_grad:
            # the additive stream trains tile_q / tile_k through the softmax (block_matmul.py:395)
            probs = masked_softmax(scores, torch.ones((), dtype=torch.bool, device=device))
        context = (probs.to(tile_v.dtype).reshape(-1, self.total_tiles) @ tile_v.contiguous()).view(
            batch, seq_len, self.index_dim)
        out = out + self.out_proj(context)
        aux: Dict[str, Any] = {
            "active_tiles": n_active,
            "total_tiles": self.total_tiles,
            "tile_sparsity": 1.0 - (n_active / self.total_tiles),
            "distill_loss": torch.tensor(0.0, device=device),
        }
        if compute_teacher_loss:
            with torch.no_grad():
                dense_out = F.linear(x, self.weight)
                energy = torch.norm(dense_out.view(batch, seq_len, self.num_n_blocks, self.block_n), p=2, dim=-1)
                # tile (k_b, n_b) takes the energy of its output block n_b (block_matmul.py:404-410)
                tile_energy = energy.repeat(1, 1, self.num_k_blocks)
                teacher = F.softmax(tile_energy, dim=-1)
            aux["distill_loss"] = -(teacher * F.log_softmax(scores, dim=-1)).sum(dim=-1).mean()
        return out, aux
