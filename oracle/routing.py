"""Oracle for 16-D indexer routing — TEST INFRASTRUCTURE ONLY.

Restates with torch CPU ops, in the reference's order (ATen CPU exp, sums,
sort and cumsum decide every bit of the result):
  * masked_softmax                     foveal_indexer/core.py:36-43
  * select_blocks                      foveal_indexer/core.py:46-160
  * FovealIndexer scoring              foveal_indexer/core.py:214-266
  * FovealPattentionMLP pooled router  foveal_indexer/foveal_pattention.py:310-321
  * decode_step page routing           foveal_indexer/attention.py:313-337
  * BlockSparseLinear eval routing     foveal_indexer/block_matmul.py:167-185
  * BlockwiseMatMul2D tile routing     foveal_indexer/block_matmul.py:344-379

Beyond the reference outputs, select_route also returns the fp32 probabilities
and sorted cumulative mass so tests can tell real mismatches from near-ties.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import Tensor


def masked_probs(scores: Tensor, mask: Tensor, acc: torch.dtype = torch.float32) -> Tensor:
    """fp32 softmax over `mask`, masked entries exactly 0, all-masked rows 0,
    returned in the scores' dtype (core.py:36-43).  `acc` = float64 gives the
    exact (fp64) value and gradient for fp64 scores."""
    s = scores.to(acc).masked_fill(~mask, float("-inf"))
    mx = s.amax(dim=-1, keepdim=True)
    mx = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
    e = torch.exp(s - mx) * mask
    z = e.sum(dim=-1, keepdim=True).clamp_min(1e-20)
    return (e / z).to(scores.dtype)


def route_masks(query_blocks: int, total_blocks: int, causal: bool, local_window_blocks: int):
    """(complete, local, remote) boolean masks of shape (Qb, Nb) (core.py:79-99)."""
    qb = torch.arange(query_blocks).view(-1, 1)
    pb = torch.arange(total_blocks).view(1, -1)
    if causal:
        complete = pb < qb
        if local_window_blocks > 0:
            first_local = (qb - local_window_blocks).clamp_min(0)
            local = complete & (pb >= first_local)
            remote = complete & (pb < first_local)
        else:
            local = torch.zeros_like(complete)
            remote = complete
    else:
        complete = torch.ones(query_blocks, total_blocks, dtype=torch.bool)
        if local_window_blocks > 0:
            local = (pb < local_window_blocks).expand(query_blocks, -1)
            remote = (pb >= local_window_blocks).expand(query_blocks, -1)
        else:
            local = torch.zeros_like(complete)
            remote = complete
    return complete, local, remote


def select_route(
    block_scores: Tensor,
    *,
    causal: bool = True,
    block_size: int = 64,
    local_window_blocks: int = 0,
    top_p=0.95,
    min_remote_blocks=0,
    max_remote_blocks=16,
    remote_capacity: int = 16,
) -> dict:
    """Adaptive top-p routing with base mass (core.py:46-160).  Returns the
    Route fields plus 'probs', 'sorted_probs', 'cumulative', 'target', 'local_mass'."""
    B, Qb, Nb = block_scores.shape
    p_t = torch.as_tensor(top_p, dtype=torch.float32)
    kmin_t = torch.as_tensor(min_remote_blocks, dtype=torch.int64)
    kmax_t = torch.as_tensor(max_remote_blocks, dtype=torch.int64)
    complete, local, remote = route_masks(Qb, Nb, causal, local_window_blocks)

    probs = masked_probs(block_scores, complete[None].expand(B, -1, -1))
    local_mass = (probs * local[None]).sum(dim=-1)
    ranked = probs.masked_fill(~remote[None], -1.0)
    sp, order = ranked.sort(dim=-1, descending=True)
    sp = sp.clamp_min(0.0)
    cum = sp.cumsum(dim=-1)

    target = (p_t - local_mass).clamp_min(0.0)
    available = remote.sum(dim=-1).view(1, Qb).expand(B, -1)
    need = (cum < target[..., None]).sum(dim=-1) + (target > 0).long()
    need = torch.where(available > 0, need, torch.zeros_like(need))
    need = torch.where(available > 0, torch.maximum(need, kmin_t), need)
    counts = torch.minimum(torch.minimum(need, available), kmax_t)

    idx = order[..., :remote_capacity].to(torch.int32)
    if idx.shape[-1] < remote_capacity:
        idx = F.pad(idx, (0, remote_capacity - idx.shape[-1]))

    if local_window_blocks > 0:
        if causal:
            width = local_window_blocks + 1
            offs = torch.arange(width)
            qb = torch.arange(Qb)
            start = (qb - local_window_blocks).clamp_min(0)
            n_local = qb - start + 1
            base = torch.where(offs[None] < n_local[:, None], start[:, None] + offs[None], torch.zeros(1, dtype=torch.long))
            base_indices = base[None].expand(B, -1, -1).to(torch.int32)
            base_counts = n_local[None].expand(B, -1).to(torch.int32)
        else:
            base_indices = torch.arange(local_window_blocks, dtype=torch.int32)[None, None].expand(B, Qb, -1)
            base_counts = torch.full((B, Qb), local_window_blocks, dtype=torch.int32)
    else:
        base_indices = base_counts = None

    cap_rate = torch.where(kmax_t > 0, (counts >= kmax_t).float().mean(), torch.zeros((), dtype=torch.float32))
    return {
        "remote_indices": idx,
        "remote_counts": counts.to(torch.int32),
        "base_indices": base_indices,
        "base_counts": base_counts,
        "cap_rate": cap_rate,
        "mean_remote_blocks": counts.float().mean(),
        "base_only_rate": (counts == 0).float().mean(),
        "probs": probs.float(),
        "sorted_probs": sp.float(),
        "cumulative": cum.float(),
        "target": target.float(),
        "local_mass": local_mass.float(),
    }


def cosine_scores_f32(q: Tensor, k: Tensor) -> Tensor:
    """fp32 cosine / sqrt(d) scores (the fp32 form of core.py:263-265: inputs
    upcast, F.normalize, bmm, divide by sqrt(index_dim)); q (B,Q,d), k (B,N,d)."""
    qn = F.normalize(q.float(), dim=-1)
    kn = F.normalize(k.float(), dim=-1)
    return torch.bmm(qn, kn.transpose(-2, -1)) / math.sqrt(q.shape[-1])


def mlp_router_scores(x2d: Tensor, q_proj_weight: Tensor, block_keys: Tensor) -> Tensor:
    """Pooled eval scores rms_norm(q_proj(mean(x))) @ K^T, no 1/sqrt(d)
    (foveal_pattention.py:312-313); dtype of the inputs."""
    d = q_proj_weight.shape[0]
    q16 = F.rms_norm(F.linear(x2d.mean(dim=0, keepdim=True), q_proj_weight), (d,))
    return torch.matmul(q16, block_keys.t()).squeeze(0)


def mlp_pooled_route(x2d: Tensor, q_proj_weight: Tensor, block_keys: Tensor, base_blocks: int,
                     remote_blocks: int) -> Tensor:
    """Active blocks [0..base) ++ topk(s[base:]) + base (foveal_pattention.py:314-321),
    with ties among equal scores ordered by lower block index."""
    s = mlp_router_scores(x2d, q_proj_weight, block_keys).float()
    rem = s[base_blocks:]
    # stable descending order = topk's values with ties broken by index
    order = torch.sort(rem, descending=True, stable=True).indices[:remote_blocks]
    top = order.to(torch.int32) + base_blocks
    return torch.cat([torch.arange(base_blocks, dtype=torch.int32), top])


def decode_route(qi: Tensor, kp_cache: Tensor, pos: int, page_size: int, local_window: int,
                 completed_pages: int, top_p: float, min_remote: int, max_remote: int) -> dict:
    """Remote pages of one decode step (attention.py:313-337), per sequence.
    qi: (B, 1, d) 16-D query; kp_cache: (B, P, d) fp32 page keys."""
    B = qi.shape[0]
    local_start = max(0, pos + 1 - local_window)
    flp = local_start // page_size
    out = {"local_start": local_start, "first_local_page": flp, "pages": [[] for _ in range(B)],
           "probs": None, "sorted_probs": None, "cumulative": None}
    if not (completed_pages > flp and flp > 0):
        return out
    qn = F.normalize(qi.float(), dim=-1)
    kr = kp_cache[:, :flp]
    scores = torch.einsum("btr,bpr->btp", qn, kr).squeeze(1) / math.sqrt(qi.shape[-1])
    probs = F.softmax(scores, dim=-1)
    sp, order = probs.sort(dim=-1, descending=True)
    cum = sp.cumsum(dim=-1)
    kmax = min(max_remote, flp)
    for b in range(B):
        need = int((cum[b] < top_p).sum().item()) + 1
        need = max(min_remote, min(need, kmax))
        out["pages"][b] = order[b, :need].tolist()
    out.update(probs=probs, sorted_probs=sp, cumulative=cum, scores=scores)
    return out


def tile_route(scores: Tensor, top_p: float, base_tiles: int, rows_per_group: int | None = None) -> dict:
    """BlockwiseMatMul2D tile selection (block_matmul.py:364-377) over token rows.

    scores: (rows, T) in the module dtype.  probs = softmax (in that dtype), tiles
    sorted by probability descending (stable: equal probabilities keep tile
    order), cumulative mass with ATen's CPU cumsum, needed = #(cum < top_p) + 1
    capped at T (no K_min / K_max), and the union of every row's first `needed`
    tiles with tiles [0, base_tiles).  With rows_per_group, one union per group
    of consecutive rows (the reference has a single group).
    Returns mask (groups, T) bool, needed (rows,), probs, sorted_probs,
    cumulative and order."""
    R, T = scores.shape
    probs = F.softmax(scores, dim=-1)
    sp, order = probs.sort(dim=-1, descending=True, stable=True)
    cum = sp.cumsum(dim=-1)
    needed = ((cum < top_p).sum(dim=-1) + 1).clamp_max(T)
    rpg = R if rows_per_group is None else rows_per_group
    groups = max(1, -(-R // max(rpg, 1)))
    mask = torch.zeros(groups, T, dtype=torch.bool)
    mask[:, :base_tiles] = True
    for r in range(R):
        mask[r // max(rpg, 1), order[r, : int(needed[r])]] = True
    return {"mask": mask, "needed": needed, "probs": probs, "sorted_probs": sp, "cumulative": cum, "order": order}
