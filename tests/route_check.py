"""Tie-tolerant comparison of routing results with the CPU oracle.

Bit-exact except where the reference itself is not determined:
  * slots may hold different blocks only where the oracle's ranked values
    (probability for remote blocks, -1 otherwise) are equal or within `rtol`
    relative -- torch.sort leaves equal keys in unspecified order, and ulp-level
    exp/sum differences can swap near-equal probabilities;
  * counts may differ only where the oracle's cumulative mass at the boundary
    lies within `ctol` of the target.
Everything else (distinctness of the ranked slots, padding, counts) must match.
"""
from __future__ import annotations

import torch

F32_RTOL, F32_CTOL = 1e-6, 1e-5
BF16_RTOL, BF16_CTOL = 2.0 ** -7, 8e-3


def tolerances(dtype: torch.dtype):
    return (BF16_RTOL, BF16_CTOL) if dtype == torch.bfloat16 else (F32_RTOL, F32_CTOL)


def ranked_values(ora: dict, remote: torch.Tensor) -> torch.Tensor:
    """(B, Qb, Nb) value each block is ranked by in the reference."""
    return ora["probs"].float().masked_fill(~remote[None], -1.0)


def check_rows(gpu_idx, gpu_cnt, ora: dict, remote: torch.Tensor, rtol: float, ctol: float, max_report: int = 5):
    """Return a list of mismatch descriptions (empty = parity)."""
    gi = gpu_idx.cpu().long()
    gc = gpu_cnt.cpu().long()
    oi = ora["remote_indices"].long()
    oc = ora["remote_counts"].long()
    vals = ranked_values(ora, remote)
    cum = ora["cumulative"].float()
    target = ora["target"].float()
    B, Qb, cap = oi.shape
    Nb = vals.shape[-1]
    n_ranked = min(cap, Nb)
    bad = []
    for b in range(B):
        for q in range(Qb):
            g, o = gi[b, q], oi[b, q]
            if n_ranked:
                if not bool(((g[:n_ranked] >= 0) & (g[:n_ranked] < Nb)).all()):
                    bad.append(f"({b},{q}) index out of range: {g[:n_ranked].tolist()}")
                    continue
                if len(set(g[:n_ranked].tolist())) != n_ranked:
                    bad.append(f"({b},{q}) repeated blocks {g[:n_ranked].tolist()}")
                vg = vals[b, q, g[:n_ranked]]
                vo = vals[b, q, o[:n_ranked]]
                diff = (vg - vo).abs()
                lim = rtol * torch.maximum(vg.abs(), vo.abs())
                if bool((diff > lim).any()):
                    k = int(torch.nonzero(diff > lim)[0])
                    bad.append(f"({b},{q}) slot {k}: gpu block {int(g[k])} ({float(vg[k]):.9g}) vs "
                               f"oracle block {int(o[k])} ({float(vo[k]):.9g})")
            if cap > Nb and not bool((g[Nb:] == 0).all()):
                bad.append(f"({b},{q}) padding past {Nb} not zero: {g[Nb:].tolist()}")
            if int(gc[b, q]) != int(oc[b, q]):
                k = min(int(gc[b, q]), int(oc[b, q])) - 1
                boundary = float(cum[b, q, k]) if 0 <= k < Nb else 0.0  # no selected block: zero mass
                near = k < Nb and abs(boundary - float(target[b, q])) <= ctol
                if not near:
                    bad.append(f"({b},{q}) count gpu {int(gc[b, q])} vs oracle {int(oc[b, q])} "
                               f"(target {float(target[b, q]):.9g})")
            if len(bad) >= max_report:
                return bad
    return bad
