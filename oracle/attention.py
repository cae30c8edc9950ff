"""Oracle for foveal decode attention — TEST INFRASTRUCTURE ONLY.

  * decode_attention_f64   textbook softmax attention in fp64 over the support
                           of foveal_indexer/attention.py:339-365 (tokens
                           [max(0, pos + 1 - W), pos] then the selected pages),
                           GQA head h -> KV head h // groups
  * DecodeStepOracle       FovealSparseAttention.decode_step restated with torch
                           CPU ops in the reference's order (attention.py:284-379),
                           fed by the same module weights; per-sequence pages by
                           default, the reference's sequence-0 pages with batch0=True
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
    def step(self, x: Tensor):
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
