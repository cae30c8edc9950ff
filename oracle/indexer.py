"""Oracle for the FovealIndexer representations — TEST INFRASTRUCTURE ONLY.

Restates with torch CPU ops, in the reference's order and dtypes:
  * compute_query_16d norm     foveal_indexer/core.py:214-222 (F.rms_norm after q_proj)
  * compute_kv_blocks_16d      foveal_indexer/core.py:224-250
  * compute_block_scores       foveal_indexer/core.py:254-266
  * additive_stream context    foveal_indexer/core.py:288-310 (up to out_proj)
  * distillation_loss          foveal_indexer/core.py:315-353
The projections themselves (nn.Linear) are inputs here: the HIP path runs them
as library GEMMs and these functions start from their outputs.
Backward passes: torch autograd of these functions, as in the reference's
training (tests/test_indexer.py:63-101); with fp64 inputs and acc=float64 they
are exact fp64 gradients, pinned by finite differences (gradcheck).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor

from .routing import masked_probs


def rms_norm16(x_lin: Tensor) -> Tensor:
    """F.rms_norm over the last dimension, default eps (core.py:222)."""
    return F.rms_norm(x_lin, (x_lin.shape[-1],))


def pool_kv(k_lin: Tensor, v_lin: Tensor, block_size: int, acc: torch.dtype = torch.float32):
    """(k_blocks, v_blocks) from the k/v projections (core.py:241-250)."""
    B, N, d = k_lin.shape
    nb = N // block_size
    k_elem = F.rms_norm(k_lin, (d,))
    k_blocks = k_elem.view(B, nb, block_size, d).mean(dim=2)
    v_blocks = v_lin.view(B, nb, block_size, d).mean(dim=2)
    k_blocks = F.normalize(k_blocks.to(acc), dim=-1).to(k_lin.dtype)
    return k_blocks, v_blocks


def block_scores(q_blocks: Tensor, k_blocks: Tensor, acc: torch.dtype = torch.float32) -> Tensor:
    """cosine / sqrt(d) with the operands cast back to their dtype (core.py:263-265)."""
    qn = F.normalize(q_blocks.to(acc), dim=-1).to(q_blocks.dtype)
    kn = F.normalize(k_blocks.to(acc), dim=-1).to(k_blocks.dtype)
    return torch.bmm(qn, kn.transpose(-2, -1).contiguous()) / math.sqrt(q_blocks.shape[-1])


def additive_context(block_scores: Tensor, v_blocks: Tensor, causal: bool, acc: torch.dtype = torch.float32) -> Tensor:
    """masked_softmax(scores, valid).to(v dtype) @ v_blocks (core.py:296-310)."""
    B, Qb, Nb = block_scores.shape
    if causal:
        valid = torch.arange(Nb).view(1, Nb) < torch.arange(Qb).view(Qb, 1)
    else:
        valid = torch.ones(Qb, Nb, dtype=torch.bool)
    probs = masked_probs(block_scores, valid[None].expand(B, -1, -1), acc).to(v_blocks.dtype)
    return torch.bmm(probs, v_blocks)


def distillation_loss(student: Tensor, teacher: Tensor, valid_mask: Tensor | None = None, causal: bool = True,
                      temperature: float = 1.0, acc: torch.dtype = torch.float32) -> Tensor:
    """FovealIndexer.distillation_loss (core.py:315-353): cross-entropy of the
    teacher block mass (clamped at 0, zeroed outside the valid set, renormalised,
    uniform over the valid set when its mass is <= 1e-12) against
    log_softmax(student / T) over the valid set, averaged over query rows that
    have a valid block.  valid_mask defaults to key block < query block (causal)
    or everything.  Autograd of this restatement is the oracle gradient."""
    B, Q, N = student.shape
    if valid_mask is None:
        if causal:
            valid = torch.arange(N).view(1, N) < torch.arange(Q).view(Q, 1)
        else:
            valid = torch.ones(Q, N, dtype=torch.bool)
        valid = valid[None].expand(B, Q, N)
    else:
        valid = torch.broadcast_to(valid_mask.bool(), (B, Q, N))
    z = (student.to(acc) / temperature).masked_fill(~valid, float("-inf"))
    logp = torch.where(valid, torch.log_softmax(z, dim=-1), torch.zeros((), dtype=acc))
    t = torch.where(valid, teacher.to(acc).clamp(min=0.0), torch.zeros((), dtype=acc))
    mass = t.sum(dim=-1, keepdim=True)
    n_valid = valid.to(acc).sum(dim=-1, keepdim=True)
    target = torch.where(mass > 1e-12, t / mass.clamp(min=1e-12), valid.to(acc) / n_valid.clamp(min=1.0))
    per_row = -(target.detach() * logp).sum(dim=-1)
    rows = valid.any(dim=-1)
    if bool(rows.any()):
        return per_row[rows].mean()
    return student.sum() * 0.0
