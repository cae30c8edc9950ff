"""Oracle for the block-sparse GEMMs — TEST INFRASTRUCTURE ONLY.

  * block_sparse_linear_f64   triton_block_sparse_linear / BlockSparseLinear GEMM
                              (foveal_indexer/triton_ops.py:316-370,
                              foveal_indexer/block_matmul.py:217-232): zeros, then
                              x w[blk]^T + bias[blk] on the active column blocks
  * blockwise_matmul_f64      BlockwiseMatMul2D (foveal_indexer/block_matmul.py:381-392):
                              x (w o M)^T with the tile mask expanded to elements,
                              one mask per row group
  * eval_active_blocks        BlockSparseLinear inference selection
                              (foveal_indexer/block_matmul.py:168-185)
  * block_sparse_forward      BlockSparseLinear.forward in eval mode under no_grad
                              (foveal_indexer/block_matmul.py:131-262), torch CPU ops
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

from . import indexer as IX


def block_sparse_linear_f64(x: Tensor, w: Tensor, bias, active, block_size: int) -> Tensor:
    M = x.shape[0]
    N = w.shape[0]
    out = torch.zeros(M, N, dtype=torch.float64)
    for b in sorted(set(int(i) for i in active)):
        cols = slice(b * block_size, (b + 1) * block_size)
        out[:, cols] = x.double() @ w[cols].double().t()
        if bias is not None:
            out[:, cols] += bias[cols].double()
    return out


def expand_tile_mask(mask: Tensor, N: int, K: int, block_k: int, block_n: int) -> Tensor:
    """(T,) k-major tile mask -> (N, K) element mask of w."""
    nkb, nnb = K // block_k, N // block_n
    m = mask.view(nkb, nnb).t()  # (n_b, k_b)
    return m.repeat_interleave(block_n, 0).repeat_interleave(block_k, 1)


def blockwise_matmul_f64(x: Tensor, w: Tensor, masks: Tensor, block_k: int, block_n: int,
                         rows_per_group: int) -> Tensor:
    M, K = x.shape
    N = w.shape[0]
    if masks.dim() == 1:
        masks = masks[None]
    out = torch.zeros(M, N, dtype=torch.float64)
    for g in range(masks.shape[0]):
        rows = slice(g * rows_per_group, min(M, (g + 1) * rows_per_group))
        em = expand_tile_mask(masks[g], N, K, block_k, block_n)
        out[rows] = x[rows].double() @ (w.double() * em).t()
    return out


def eval_active_blocks(block_scores: Tensor, base_blocks: int, top_p: float, max_remote: int, num_blocks: int):
    remote = block_scores[..., base_blocks:]
    mask = torch.zeros(num_blocks, dtype=torch.bool)
    mask[:base_blocks] = True
    if remote.shape[-1] > 0:
        probs = F.softmax(remote, dim=-1)
        sp, si = probs.sort(dim=-1, descending=True)
        cum = sp.cumsum(dim=-1)
        needed = torch.clamp((cum < top_p).sum(dim=-1) + 1, 0, max_remote)
        slot = torch.arange(si.shape[-1]).view(1, 1, -1)
        sel = si[slot < needed.unsqueeze(-1)] + base_blocks
        if sel.numel():
            mask[sel.long()] = True
    return torch.where(mask)[0]


@torch.no_grad()
def block_sparse_forward(m, x: Tensor) -> Tensor:
    """BlockSparseLinear eval forward with module m's (CPU) weights."""
    orig = x.ndim
    if orig == 2:
        x = x.unsqueeze(1)
    B, T, D = x.shape
    q = IX.rms_norm16(m.indexer.q_proj(x))
    kb, vb = IX.pool_kv(m.weight_to_k(m.weight)[None], m.weight_to_v(m.weight)[None], m.block_size)
    scores = IX.block_scores(q, kb.expand(B, -1, -1).contiguous())
    active = eval_active_blocks(scores, m.base_blocks, m.indexer.top_p, m.indexer.max_remote_blocks, m.num_blocks)
    off = torch.arange(m.block_size)
    chan = (active.view(-1, 1) * m.block_size + off).flatten()
    out = torch.zeros(B, T, m.out_features, dtype=x.dtype)
    out[:, :, chan] = F.linear(x, m.weight[chan])
    if m.bias is not None:
        out[:, :, chan] = out[:, :, chan] + m.bias[chan].to(out.dtype)
    if m.use_additive_stream:
        probs = F.softmax(scores, dim=-1).to(vb.dtype)
        ctx = torch.bmm(probs, vb.expand(B, -1, -1).contiguous())
        out = out + m.indexer.out_proj(ctx).to(out.dtype)
    if orig == 2:
        out = out.squeeze(1)
    return out, active
