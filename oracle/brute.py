"""Pure-Python brute-force selection on tiny rows — TEST INFRASTRUCTURE ONLY.

Written independently of oracle/routing.py (no torch): fp64 softmax, an
explicit ranking by (probability desc, index asc), a running fp64 sum, and the
count rule of foveal_indexer/core.py:111-119 spelled out step by step.  Used to
pin oracle.routing.select_route on inputs whose margins are far above fp32
rounding, so both must agree exactly on counts and selected sets.
"""
from __future__ import annotations

import math


def select_row(scores, complete, local, remote, top_p, k_min, k_max, capacity):
    """One (batch, query-block) row.  scores: floats; complete/local/remote: bools.
    Returns (indices[:capacity] in rank order, count)."""
    n = len(scores)
    valid = [i for i in range(n) if complete[i]]
    probs = [0.0] * n
    if valid:
        m = max(scores[i] for i in valid)
        z = sum(math.exp(scores[i] - m) for i in valid)
        for i in valid:
            probs[i] = math.exp(scores[i] - m) / z
    local_mass = sum(probs[i] for i in range(n) if local[i])
    remote_ids = [i for i in range(n) if remote[i]]
    ranked = sorted(remote_ids, key=lambda i: (-probs[i], i))
    rest = [i for i in range(n) if not remote[i]]
    order = ranked + rest

    target = max(top_p - local_mass, 0.0)
    running, below = 0.0, 0
    for pos, i in enumerate(order):
        if remote[i]:
            running += probs[i]
        if running < target:
            below += 1
    needed = below + (1 if target > 0 else 0)
    available = len(remote_ids)
    if available > 0:
        needed = max(needed, k_min)
    else:
        needed = 0
    count = min(needed, available, k_max)
    idx = order[:capacity] + [0] * max(0, capacity - n)
    return idx, count


def masks(qb, nb, causal, local_window_blocks):
    """Row masks for query block qb (core.py:79-99)."""
    complete, local, remote = [], [], []
    for p in range(nb):
        if causal:
            c = p < qb
            first = max(qb - local_window_blocks, 0)
            if local_window_blocks > 0:
                loc, rem = c and p >= first, c and p < first
            else:
                loc, rem = False, c
        else:
            c = True
            if local_window_blocks > 0:
                loc, rem = p < local_window_blocks, p >= local_window_blocks
            else:
                loc, rem = False, True
        complete.append(c)
        local.append(loc)
        remote.append(rem)
    return complete, local, remote


def topk_desc(values, k):
    """Indices of the k largest values, ties to the lower index."""
    return sorted(range(len(values)), key=lambda i: (-values[i], i))[:k]


def distill_loss_rows(student, teacher, valid, temperature):
    """Brute-force block KL loss (foveal_indexer/core.py:315-353) on nested
    lists [row][block]: fp64 log-softmax of student / T over the valid blocks,
    target = clamped teacher mass renormalised over them (uniform if it sums to
    <= 1e-12), loss = mean over rows with a valid block of -sum target * logp.
    Returns (loss, per-row losses or None for rows without a valid block)."""
    rows = []
    for s_row, t_row, v_row in zip(student, teacher, valid):
        ids = [i for i, ok in enumerate(v_row) if ok]
        if not ids:
            rows.append(None)
            continue
        z = [s_row[i] / temperature for i in ids]
        m = max(z)
        lse = m + math.log(sum(math.exp(v - m) for v in z))
        t = [max(t_row[i], 0.0) for i in ids]
        mass = sum(t)
        if mass > 1e-12:
            tgt = [v / mass for v in t]
        else:
            tgt = [1.0 / len(ids)] * len(ids)
        rows.append(-sum(w * (v - lse) for w, v in zip(tgt, z)))
    kept = [r for r in rows if r is not None]
    loss = sum(kept) / len(kept) if kept else 0.0
    return loss, rows


def tile_route_row(scores, top_p):
    """Tiles one token row of BlockwiseMatMul2D selects (foveal_indexer/block_matmul.py:364-377),
    spelled out: fp64 softmax, tiles ranked by (probability desc, tile asc), running
    fp64 mass, count = #(running mass < top_p) + 1, capped at the tile count.
    Returns the selected tile ids in rank order."""
    m = max(scores)
    e = [math.exp(s - m) for s in scores]
    z = sum(e)
    probs = [v / z for v in e]
    ranked = sorted(range(len(scores)), key=lambda i: (-probs[i], i))
    running, below = 0.0, 0
    for i in ranked:
        running += probs[i]
        if running < top_p:
            below += 1
    return ranked[: min(below + 1, len(scores))]


def sram_pick_row(scores, m, top_p, max_remote):
    """Greedy picks of one query block m from its raw 16-D scores (already / 4):
    fp64 softmax over the blocks other than m with the 1e-6 pad, then per round
    the largest remaining probability (first index on ties), attended iff the
    mass of all earlier rounds is < top_p and it is > 1e-4; retired either way.
    Returns the picks, -1 where not attended."""
    n = len(scores)
    others = [j for j in range(n) if j != m]
    probs = [0.0] * n
    if others:
        top = max(scores[j] for j in others)
        top = max(top, -1.0e4)
        z = sum(math.exp(scores[j] - top) for j in others) + 1e-6
        for j in others:
            probs[j] = math.exp(scores[j] - top) / z
    out, mass = [], 0.0
    for _ in range(max_remote):
        best = 0
        for j in range(1, n):
            if probs[j] > probs[best]:
                best = j
        p = probs[best]
        out.append(best if (mass < top_p and p > 1e-4) else -1)
        mass += p
        probs[best] = -1.0
    return out
