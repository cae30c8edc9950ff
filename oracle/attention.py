"""Oracle for foveal decode attention — TEST INFRASTRUCTURE ONLY.

  * decode_attention_f64   textbook softmax attention in fp64 over the support
                           of foveal_indexer/attention.py:339-365 (tokens
                           [max(0, pos + 1 - W), pos] then the selected pages),
                           GQA head h -> KV head h // groups
  * DecodeStepOracle       FovealSparseAttention.decode_step restated with torch
                           CPU ops in the reference's order (attention.py:284-379),
                           fed by the same module weights; per-sequence pages by
                           default, the reference's sequence-0 pages with batch0=True
  * sparse_mask            _build_sparse_mask (attention.py:148-178): causal local
                           window OR the query block's listed remote pages
  * block_list_weights     the key multiplicities of triton_foveal_sparse_attention
                           (triton_ops.py:26-93): query block m counts each key of
                           every listed block once per listing
  * weighted_attention_f64 softmax attention in fp64 with per-key weights
                           (0 / 1 for a boolean mask: the SDPA of attention.py:211-216;
                           counts for the Triton kernel); a row with no weight gives 0
                           (the Triton kernel's clamp of l at 1e-6)
  * prefill_forward        FovealSparseAttention.forward (attention.py:180-269) with
                           a given route, and its teacher page mass (:243-265)
  * sram_select            the in-kernel routing of triton_fused_sram_indexer_attention
                           (triton_ops.py:164-182,219-245) in fp32: 16-D scores / 4,
                           softmax over the other blocks (+1e-6), greedy picks gated by
                           mass < top_p and p > 1e-4
  * sram_attention_f64     that kernel's attention (triton_ops.py:186-248) as fp64
                           softmax attention over the self block plus the attended picks
"""
from __future__ import annotations

import math
from typing import List

import torch
import torch.nn.functional as F
from torch import Tensor

from .routing import decode_route


def support_tokens(pos: int, window: int, pages: List[int], page_size: int) -> List[int]:
    ls = max(0, pos + 1 - window)
    toks = list(range(ls, pos + 1))
    for p in pages:
        toks.extend(range(p * page_size, (p + 1) * page_size))
    return toks


def decode_attention_f64(q: Tensor, k: Tensor, v: Tensor, pos, window: int, pages, page_size: int,
                         scale: float) -> Tensor:
    """q: (B, Hq, hd); k, v: (B, Hkv, S, hd) dense; pos: int or list per sequence;
    pages: per-sequence lists of logical pages.  Returns (B, Hq, hd) fp64."""
    B, Hq, hd = q.shape
    Hkv = k.shape[1]
    groups = Hq // Hkv
    out = torch.zeros(B, Hq, hd, dtype=torch.float64)
    for b in range(B):
        pb = pos[b] if isinstance(pos, (list, tuple)) else int(pos)
        toks = torch.tensor(support_tokens(pb, window, pages[b], page_size), dtype=torch.long)
        for h in range(Hq):
            g = h // groups
            kk = k[b, g, toks].double()
            vv = v[b, g, toks].double()
            s = (kk @ q[b, h].double()) * scale
            w = torch.softmax(s, dim=0)
            out[b, h] = w @ vv
    return out


class DecodeStepOracle:
    """CPU restatement of FovealSparseAttention.decode_step with a contiguous
    reference-layout cache (attention.py:22-94, 284-379)."""

    def __init__(self, module, batch: int, max_seq_len: int, batch0: bool = False):
        self.m = module
        self.batch0 = batch0
        dt = module.q_proj.weight.dtype
        P = math.ceil(max_seq_len / module.page_size)
        self.k = torch.zeros(batch, module.num_kv_heads, max_seq_len, module.head_dim, dtype=dt)
        self.v = torch.zeros_like(self.k)
        self.kp = torch.zeros(batch, P, module.indexer.index_dim, dtype=torch.float32)
        self.vp = torch.zeros(batch, P, module.indexer.index_dim, dtype=dt)
        self.pk = torch.zeros(batch, module.page_size, module.indexer.index_dim, dtype=dt)
        self.pv = torch.zeros_like(self.pk)
        self.seq_len = 0
        self.completed = 0

    @torch.no_grad()
    def step(self, x: Tensor, attend=None):
        """One decode step.  attend: per-sequence page lists to attend instead of
        this step's own selection (a checker's hook for comparing outputs over
        the same support where a near-tie made two selections differ); the
        returned pages and route are always this step's own."""
        m = self.m
        B = x.shape[0]
        pos = self.seq_len
        q = m.q_proj(x).view(B, m.num_heads, 1, m.head_dim)
        k = m.k_proj(x).view(B, m.num_kv_heads, 1, m.head_dim)
        v = m.v_proj(x).view(B, m.num_kv_heads, 1, m.head_dim)
        qi = F.rms_norm(m.indexer.q_proj(x), (m.indexer.index_dim,))
        ki = F.rms_norm(m.indexer.k_proj(x), (m.indexer.index_dim,))
        vi = m.indexer.v_proj(x)
        self.k[:, :, pos:pos + 1] = k
        self.v[:, :, pos:pos + 1] = v
        off, page = pos % m.page_size, pos // m.page_size
        self.pk[:, off] = ki.squeeze(1)
        self.pv[:, off] = vi.squeeze(1)
        if off == m.page_size - 1:
            self.kp[:, page] = F.normalize(self.pk.mean(dim=1).float(), dim=-1)
            self.vp[:, page] = self.pv.mean(dim=1)
            self.completed += 1
        self.seq_len += 1
        r = decode_route(qi, self.kp, pos, m.page_size, m.local_window, self.completed, m.indexer.top_p,
                         m.indexer.min_remote_blocks, m.indexer.max_remote_blocks)
        pages = r["pages"]
        att_pages = [pages[0]] * B if self.batch0 else pages
        if attend is not None:
            att_pages = attend
        attn = decode_attention_f64(q[:, :, 0].float(), self.k, self.v, pos, m.local_window, att_pages, m.page_size,
                                    m.scale).to(x.dtype)
        out = m.out_proj(attn.reshape(B, 1, m.num_heads * m.head_dim))
        if m.use_additive_stream and self.completed > 0:
            qn = F.normalize(qi.float(), dim=-1)
            sc = torch.einsum("btr,bpr->btp", qn, self.kp[:, :self.completed]) / math.sqrt(m.indexer.index_dim)
            pr = F.softmax(sc, dim=-1).to(self.vp.dtype)
            ctx = torch.einsum("btp,bpr->btr", pr, self.vp[:, :self.completed])
            out = out + m.indexer.out_proj(ctx)
        return out, pages, r


def sparse_mask(batch: int, seq_len: int, window: int, page_size: int, remote_indices: Tensor,
                remote_counts: Tensor) -> Tensor:
    """(B, T, T) bool: key s visible to query t (attention.py:148-178)."""
    q = torch.arange(seq_len)
    k = torch.arange(seq_len)
    allowed = (k[None, :] <= q[:, None]) & (k[None, :] > q[:, None] - window)
    allowed = allowed[None].expand(batch, -1, -1).clone()
    for b in range(batch):
        for qb in range(remote_counts.shape[1]):
            q0, q1 = qb * page_size, min((qb + 1) * page_size, seq_len)
            for slot in range(int(remote_counts[b, qb])):
                page = int(remote_indices[b, qb, slot])
                allowed[b, q0:q1, page * page_size:min((page + 1) * page_size, seq_len)] = True
    return allowed


def block_list_weights(batch: int, seq_len: int, block: int, block_indices: Tensor, counts: Tensor) -> Tensor:
    """(B, T, T) float64: how many times key s is listed for query t's block
    (triton_ops.py:67-88: one pass over the block per listing)."""
    w = torch.zeros(batch, seq_len, seq_len, dtype=torch.float64)
    for b in range(batch):
        for m in range(counts.shape[1]):
            q0, q1 = m * block, min((m + 1) * block, seq_len)
            for j in range(int(counts[b, m])):
                kb = int(block_indices[b, m, j])
                w[b, q0:q1, kb * block:min((kb + 1) * block, seq_len)] += 1.0
    return w


def weighted_attention_f64(q: Tensor, k: Tensor, v: Tensor, weights: Tensor, scale: float) -> Tensor:
    """out[b, h, t] = sum_s w[b, t, s] exp(scale q.k_s) v_s / sum_s w[b, t, s] exp(scale q.k_s)
    in fp64, KV head h // (Hq / Hkv); q: (B, Hq, T, hd), k, v: (B, Hkv, T, hd),
    weights: (B, T, T) bool or float.  Rows with no weight give 0."""
    B, Hq, T, hd = q.shape
    Hkv = k.shape[1]
    groups = Hq // Hkv
    w = weights.double()
    kk = k.double().repeat_interleave(groups, dim=1)
    vv = v.double().repeat_interleave(groups, dim=1)
    s = torch.matmul(q.double(), kk.transpose(-2, -1)) * scale
    s = s.masked_fill(w[:, None] == 0, float("-inf"))
    mx = s.amax(dim=-1, keepdim=True)
    mx = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
    e = torch.exp(s - mx) * w[:, None]
    z = e.sum(dim=-1, keepdim=True)
    p = torch.where(z > 0, e / z.clamp_min(1e-300), torch.zeros_like(e))
    return torch.matmul(p, vv)


@torch.no_grad()
def prefill_forward(m, x: Tensor, remote_indices: Tensor, remote_counts: Tensor):
    """FovealSparseAttention.forward (attention.py:180-269) on the CPU with the
    module's weights and a given route: projections in the module dtype, the
    masked SDPA (attention.py:211-216) as fp64 attention under sparse_mask,
    out_proj, additive stream.  Also returns the teacher page mass of
    attention.py:243-265 (dense causal softmax over all T keys, anchor rows,
    summed per page, averaged over heads), computed in fp32 as written there.
    Returns (out (B, T, D), teacher_mass (B, Qb, pages))."""
    B, T, _ = x.shape
    ps = m.page_size
    pages = T // ps
    q = m.q_proj(x).view(B, T, m.num_heads, m.head_dim).transpose(1, 2)
    k = m.k_proj(x).view(B, T, m.num_kv_heads, m.head_dim).transpose(1, 2)
    v = m.v_proj(x).view(B, T, m.num_kv_heads, m.head_dim).transpose(1, 2)
    mask = sparse_mask(B, T, m.local_window, ps, remote_indices, remote_counts)
    attn = weighted_attention_f64(q, k, v, mask, m.scale).to(x.dtype)
    out = m.out_proj(attn.transpose(1, 2).reshape(B, T, m.num_heads * m.head_dim))
    if m.use_additive_stream:
        from . import indexer as IX

        qi = IX.rms_norm16(m.indexer.q_proj(x))
        kb, vb = IX.pool_kv(m.indexer.k_proj(x), m.indexer.v_proj(x), ps)
        scores = IX.block_scores(qi[:, ::ps], kb)
        ctx = IX.additive_context(scores, vb, True)
        out = out + m.indexer.out_proj(ctx).repeat_interleave(ps, dim=1)
    groups = m.num_heads // m.num_kv_heads
    kf = k.float().repeat_interleave(groups, dim=1)
    s = torch.matmul(q.float(), kf.transpose(-2, -1)) * m.scale
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
    s = s.masked_fill(~causal[None, None], -float("inf"))
    probs = torch.softmax(s, dim=-1)[:, :, ::ps]
    teacher = probs.view(B, m.num_heads, pages, pages, ps).sum(dim=-1).mean(dim=1)
    return out, teacher


def sram_select(q16: Tensor, k16: Tensor, top_p: float, max_remote: int):
    """Greedy block picks of triton_ops.py:164-182,219-245 in fp32.  q16, k16:
    (B, M, 16).  Returns (picks (B, M, max_remote) int64 with -1 where a pick is
    not attended, probs (B, M, M) float32 before any pick is retired)."""
    B, M, _ = q16.shape
    s = torch.matmul(q16.float(), k16.float().transpose(1, 2)) * 0.25
    remote = ~torch.eye(M, dtype=torch.bool)[None].expand(B, -1, -1)
    s = torch.where(remote, s, torch.full_like(s, -1.0e4))
    mx = s.amax(dim=-1, keepdim=True)
    e = torch.where(remote, torch.exp(s - mx), torch.zeros_like(s))
    probs = e / (e.sum(dim=-1, keepdim=True) + 1e-6)
    picks = torch.full((B, M, max_remote), -1, dtype=torch.int64)
    left = probs.clone()
    for b in range(B):
        for m in range(M):
            mass = torch.zeros((), dtype=torch.float32)
            row = left[b, m]
            for r in range(max_remote):
                best = int(torch.argmax(row))  # first index of the maximum
                bp = row[best].clone()
                if bool(mass < top_p) and bool(bp > 1e-4):
                    picks[b, m, r] = best
                mass = mass + bp
                row[best] = -1.0
    return picks, probs


def sram_attention_f64(q: Tensor, k: Tensor, v: Tensor, picks: Tensor, block: int, scale: float) -> Tensor:
    """Attention of every query of block m over the keys of block m and of each
    attended pick (triton_ops.py:186-248), fp64.  q, k, v: (B, H, N, D); picks:
    (B, N / block, R) with -1 for a pick that is not attended."""
    B, H, N, D = q.shape
    w = torch.zeros(B, N, N, dtype=torch.float64)
    for b in range(B):
        for m in range(N // block):
            rows = slice(m * block, (m + 1) * block)
            w[b, rows, m * block:(m + 1) * block] = 1.0
            for kb in picks[b, m].tolist():
                if kb >= 0:
                    w[b, rows, kb * block:(kb + 1) * block] = 1.0
    return weighted_attention_f64(q, k, v, w, scale)
