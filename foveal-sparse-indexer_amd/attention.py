"""Foveal sparse attention on MI355X: drop-in pieces of
foveal_indexer/attention.py and of triton_foveal_sparse_attention
(foveal_indexer/triton_ops.py:256-313).

decode_route: the per-step remote-page routing and additive-stream context of
FovealSparseAttention.decode_step (attention.py:313-337,369-376) as one HIP
launch over the whole batch (the reference loops over sequences in Python with
a host sync per sequence).

sparse_attention: block-sparse prefill attention (the local window plus routed
pages of FovealSparseAttention.forward, attention.py:148-227, or the block lists
of the Triton kernel) in one HIP launch that never forms the (T, T) mask.
"""
from __future__ import annotations

import math
from typing import Any, Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _lib
from .core import FovealIndexer, index_rms_norm


def decode_route(
    qi: Tensor,
    kp: Tensor,
    vp: Optional[Tensor],
    *,
    pos: int | Tensor,
    page_size: int,
    local_window: int,
    completed_pages: int,
    top_p: float,
    min_remote_blocks: int,
    max_remote_blocks: int,
    return_context: bool = False,
):
    """Remote pages of one decode step for every sequence.

    qi: (B, 16) or (B, 1, 16) 16-D index query (model dtype); kp: (B, P, 16)
    fp32 page keys; vp: (B, P, 16) page values (model dtype; needed for the
    context).  pos: current position (int, or (B,) int tensor).
    Returns (pages (B, cap) int32 in rank order with -1 past the count,
    counts (B,) int32[, context (B, 16) in vp's dtype]), cap = max(K_max, K_min, 1)."""
    what = "decode_route"
    dev = _lib.require_gpu(qi, kp, vp, what=what)
    q2 = qi.reshape(qi.shape[0], -1).contiguous()
    code = _lib.dtype_code(q2.dtype, what)
    if kp.dtype != torch.float32:
        raise TypeError(f"{what}: page keys must be float32 (FovealKVCache.kp_cache), got {kp.dtype}")
    kpc = kp.contiguous()
    B, P, d = kpc.shape
    if q2.shape != (B, d):
        raise ValueError(f"{what}: query {tuple(qi.shape)} does not match page keys {tuple(kp.shape)}")
    vpc = None
    if return_context:
        if vp is None:
            raise ValueError(f"{what}: return_context needs page values")
        if vp.dtype != q2.dtype:
            raise TypeError(f"{what}: page values {vp.dtype} and query {q2.dtype} differ")
        vpc = vp.contiguous()
        if tuple(vpc.shape) != (B, P, d):
            raise ValueError(f"{what}: page values {tuple(vp.shape)} != {(B, P, d)}")
    pos_rows = None
    pos_val = 0
    if isinstance(pos, Tensor):
        pos_rows = pos.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
        if pos_rows.numel() != B:
            raise ValueError(f"{what}: {pos_rows.numel()} positions for {B} sequences")
    else:
        pos_val = int(pos)
    cap = max(int(max_remote_blocks), int(min_remote_blocks), 1)
    pages, counts, ctx = _decode_route_op(q2, kpc, vpc, pos_rows, pos_val, int(page_size), int(local_window),
                                          int(completed_pages), float(top_p), int(min_remote_blocks),
                                          int(max_remote_blocks), cap, bool(return_context))
    if return_context:
        return pages, counts, ctx
    return pages, counts


def _decode_route_fake(q2, kp, vp, pos_rows, pos_val, page_size, local_window, completed, top_p, k_min, k_max, cap,
                       want_ctx):
    B, d = q2.shape
    return (q2.new_empty((B, cap), dtype=torch.int32), q2.new_empty((B,), dtype=torch.int32),
            q2.new_empty((B, d) if want_ctx else (0,)))


@_lib.fsi_op("decode_route", _decode_route_fake)
def _decode_route_op(q2: Tensor, kp: Tensor, vp: Optional[Tensor], pos_rows: Optional[Tensor], pos_val: int,
                     page_size: int, local_window: int, completed: int, top_p: float, k_min: int, k_max: int,
                     cap: int, want_ctx: bool) -> Tuple[Tensor, Tensor, Tensor]:
    """fsi_decode_route: (pages (B, cap) int32, counts (B,) int32, context (B, 16) or empty)."""
    what = "decode_route"
    dev = q2.device
    B, d = q2.shape
    P = kp.shape[1]
    pages = torch.empty((B, cap), dtype=torch.int32, device=dev)
    counts = torch.empty((B,), dtype=torch.int32, device=dev)
    ctx = torch.empty((B, d) if want_ctx else (0,), dtype=q2.dtype, device=dev)
    st = _lib.lib().fsi_decode_route(
        q2.data_ptr(), kp.data_ptr(), _lib.ptr(vp), _lib.dtype_code(q2.dtype, what), B, P, d, _lib.ptr(pos_rows),
        pos_val, page_size, local_window, completed, top_p, k_min, k_max, cap, pages.data_ptr(), counts.data_ptr(),
        ctx.data_ptr() if want_ctx else None, _lib.stream_handle(dev))
    _lib.check(st, what)
    return pages, counts, ctx


PAGE_SIZE = 64


class FovealKVCache:
    """KV cache for foveal decoding (drop-in for attention.py:22-94).

    Same constructor, `update` and public state (`k_cache`, `v_cache`,
    `kp_cache`, `vp_cache`, `partial_kp`, `partial_vp`, `seq_len`,
    `completed_pages`) as the reference, including its default dtype (fp32).
    Two layouts of the full-rank K/V:
      * paged (bf16, page_size 64, head_dim 64 or 128, unless paged=False):
        `k_cache` / `v_cache` are physical page pools in the MFMA-tile layouts
        of include/fsi.h, and `page_table` (B, max_pages) maps each sequence's
        logical pages to them (sequence b owns pages [b * max_pages,
        (b + 1) * max_pages) unless a caller-built table is installed);
        `to_dense()` / `load_dense()` convert to and from the reference layout;
      * contiguous (every other dtype / page size / head_dim, or paged=False):
        `k_cache` / `v_cache` are (B, Hkv, max_seq_len, head_dim) exactly as in
        the reference, so callers may read and write them directly.
    """

    def __init__(
        self,
        batch_size: int,
        max_seq_len: int,
        num_kv_heads: int,
        head_dim: int,
        index_dim: int,
        page_size: int,
        device: torch.device,
        dtype: torch.dtype = torch.float32,
        n_phys_pages: Optional[int] = None,
        page_table: Optional[Tensor] = None,
        paged: Optional[bool] = None,
    ):
        if dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"FovealKVCache: dtype {dtype} unsupported (float32 or bfloat16)")
        if page_size <= 0 or head_dim <= 0 or head_dim > 256:
            raise ValueError(f"FovealKVCache: page_size {page_size} / head_dim {head_dim} unsupported")
        pageable = dtype == torch.bfloat16 and page_size == PAGE_SIZE and head_dim in (64, 128)
        if paged and not pageable:
            raise ValueError("FovealKVCache: the paged layout needs bfloat16, page_size 64 and head_dim 64 or 128")
        self.paged = pageable if paged is None else bool(paged)
        if not self.paged and (page_table is not None or n_phys_pages is not None):
            raise ValueError("FovealKVCache: page_table / n_phys_pages apply to the paged layout only")
        self.batch_size = batch_size
        self.max_seq_len = max_seq_len
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.index_dim = index_dim
        self.page_size = page_size
        self.device = torch.device(device)
        self.dtype = dtype
        self.max_pages = -(-max_seq_len // page_size)
        if self.paged:
            if page_table is None:
                page_table = torch.arange(batch_size * self.max_pages, dtype=torch.int32).view(batch_size,
                                                                                               self.max_pages)
            self.page_table = page_table.to(device=self.device, dtype=torch.int32).contiguous()
            if tuple(self.page_table.shape) != (batch_size, self.max_pages):
                raise ValueError(f"FovealKVCache: page table {tuple(self.page_table.shape)} != "
                                 f"{(batch_size, self.max_pages)}")
            self.n_phys_pages = int(n_phys_pages) if n_phys_pages is not None else batch_size * self.max_pages
            per_page = num_kv_heads * page_size * head_dim
            self.k_cache = torch.zeros(self.n_phys_pages, per_page, device=self.device, dtype=dtype)
            self.v_cache = torch.zeros(self.n_phys_pages, per_page, device=self.device, dtype=dtype)
        else:
            self.page_table = None
            self.n_phys_pages = 0
            shape = (batch_size, num_kv_heads, max_seq_len, head_dim)
            self.k_cache = torch.zeros(shape, device=self.device, dtype=dtype)
            self.v_cache = torch.zeros(shape, device=self.device, dtype=dtype)
        self.kp_cache = torch.zeros(batch_size, self.max_pages, index_dim, device=self.device, dtype=torch.float32)
        self.vp_cache = torch.zeros(batch_size, self.max_pages, index_dim, device=self.device, dtype=dtype)
        self.partial_kp = torch.zeros(batch_size, page_size, index_dim, device=self.device, dtype=dtype)
        self.partial_vp = torch.zeros(batch_size, page_size, index_dim, device=self.device, dtype=dtype)
        self.seq_len = 0
        self.completed_pages = 0

    def _write(self, k: Tensor, v: Tensor, start: int) -> None:
        what = "FovealKVCache"
        B, H, n, hd = k.shape
        if (B, H, hd) != (self.batch_size, self.num_kv_heads, self.head_dim) or v.shape != k.shape:
            raise ValueError(f"{what}: K {tuple(k.shape)} / V {tuple(v.shape)} do not match the cache")
        if start < 0 or start + n > self.max_seq_len:
            raise RuntimeError(f"KV cache capacity {self.max_seq_len} exceeded.")
        if not self.paged:
            # the reference layout: a slice copy (attention.py:72-73), cast to the cache dtype
            with torch.no_grad():
                self.k_cache[:, :, start:start + n] = k
                self.v_cache[:, :, start:start + n] = v
            return
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise TypeError(f"{what}: K/V dtype {k.dtype}/{v.dtype} != {self.dtype}")
        if k.stride(-1) != 1:
            k = k.contiguous()
        if v.stride(-1) != 1:
            v = v.contiguous()
        _lib.require_gpu(k, v, self.k_cache, what=what)
        _kv_write_op(k, v, int(start), self.page_table, self.max_pages, self.n_phys_pages, self.k_cache, self.v_cache)

    def update(self, k_step: Tensor, v_step: Tensor, ki_step: Tensor, vi_step: Tensor) -> int:
        """Append one token's KV and 16-D index representation (attention.py:62-94)."""
        pos = self.seq_len
        if pos >= self.max_seq_len:
            raise RuntimeError(f"KV cache capacity {self.max_seq_len} exceeded.")
        self._write(k_step, v_step, pos)
        offset = pos % self.page_size
        page = pos // self.page_size
        with torch.no_grad():  # cache state, as the kernels read it: no autograd history
            self.partial_kp[:, offset] = ki_step.reshape(self.batch_size, self.index_dim)
            self.partial_vp[:, offset] = vi_step.reshape(self.batch_size, self.index_dim)
        if offset == self.page_size - 1:
            _kv_page_pool_op(self.partial_kp, self.partial_vp, self.kp_cache, self.vp_cache, page)
            self.completed_pages += 1
        self.seq_len += 1
        return pos

    def load_dense(self, k: Tensor, v: Tensor, start: int = 0) -> None:
        """Write (B, Hkv, n, hd) K/V at positions start .. start + n - 1 (the
        reference layout) without touching the 16-D page state."""
        self._write(k, v, start)

    def to_dense(self, n_tok: Optional[int] = None, batch: Optional[slice] = None):
        """(K, V) of positions [0, n_tok) in the reference layout (b, Hkv, n, hd)
        for the sequences in `batch` (a slice; all by default)."""
        n = self.seq_len if n_tok is None else int(n_tok)
        if not self.paged:
            sel = batch if batch is not None else slice(None)
            return self.k_cache[sel, :, :n].clone(), self.v_cache[sel, :, :n].clone()
        rows = self.page_table[batch] if batch is not None else self.page_table
        return _kv_read_op(self.k_cache, self.v_cache, rows.contiguous(), self.num_kv_heads, n, self.head_dim,
                           self.max_pages, self.n_phys_pages)


@_lib.fsi_op("kv_write", lambda k, v, start, page_table, max_pages, n_phys, k_cache, v_cache: None,
             mutates_args=("k_cache", "v_cache"))
def _kv_write_op(k: Tensor, v: Tensor, start: int, page_table: Tensor, max_pages: int, n_phys: int, k_cache: Tensor,
                 v_cache: Tensor) -> None:
    """fsi_kv_write: (B, H, n, hd) K/V at positions start .. start + n - 1 into the paged pool."""
    what = "FovealKVCache"
    dev = k.device
    B, H, n, hd = k.shape
    err = _lib.error_word(dev)
    st = _lib.lib().fsi_kv_write(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2), v.stride(0),
                                 v.stride(1), v.stride(2), B, H, n, hd, None, start, page_table.data_ptr(), max_pages,
                                 n_phys, k_cache.data_ptr(), v_cache.data_ptr(), err.data_ptr(),
                                 _lib.stream_handle(dev))
    _lib.check(st, what)
    if _lib.checks_enabled():
        _lib.raise_device_errors(dev, what)


@_lib.fsi_op("kv_page_pool", lambda partial_kp, partial_vp, kp_cache, vp_cache, page: None,
             mutates_args=("kp_cache", "vp_cache"))
def _kv_page_pool_op(partial_kp: Tensor, partial_vp: Tensor, kp_cache: Tensor, vp_cache: Tensor, page: int) -> None:
    """fsi_kv_page_pool: mean of the page's 16-D rows into kp_cache[:, page] / vp_cache[:, page]."""
    B, page_size, d = partial_kp.shape
    st = _lib.lib().fsi_kv_page_pool(
        partial_kp.data_ptr(), partial_vp.data_ptr(), _lib.dtype_code(partial_kp.dtype, "kv_page_pool"), B,
        page_size, d, kp_cache[:, page].data_ptr(), vp_cache[:, page].data_ptr(), kp_cache.shape[1] * d,
        _lib.stream_handle(kp_cache.device))
    _lib.check(st, "FovealKVCache.update")


def _kv_read_fake(k_cache, v_cache, rows, heads, n, hd, max_pages, n_phys):
    k = k_cache.new_empty((rows.shape[0], heads, n, hd))
    return k, torch.empty_like(k)


@_lib.fsi_op("kv_read", _kv_read_fake)
def _kv_read_op(k_cache: Tensor, v_cache: Tensor, rows: Tensor, heads: int, n: int, hd: int, max_pages: int,
                n_phys: int) -> Tuple[Tensor, Tensor]:
    """fsi_kv_read: positions [0, n) of the sequences whose page-table rows are given, (b, H, n, hd)."""
    k = torch.empty((rows.shape[0], heads, n, hd), dtype=k_cache.dtype, device=k_cache.device)
    v = torch.empty_like(k)
    st = _lib.lib().fsi_kv_read(k_cache.data_ptr(), v_cache.data_ptr(), rows.shape[0], heads, n, hd, rows.data_ptr(),
                                max_pages, n_phys, k.data_ptr(), v.data_ptr(), _lib.stream_handle(k_cache.device))
    _lib.check(st, "FovealKVCache.to_dense")
    return k, v


def _decode_launch(q3: Tensor, k_cache: Tensor, v_cache: Tensor, page_table: Optional[Tensor], max_pages: int,
                   n_phys: int, max_seq_len: int, page_size: int, n_kv_heads: int, pos_rows: Optional[Tensor],
                   pos_val: int, window: int, remote_pages: Optional[Tensor], remote_counts: Optional[Tensor],
                   cap: int, scale: float, out: Tensor) -> Tensor:
    """Paged pool (page_table given): fsi_decode_attn; contiguous cache: fsi_decode_attn_dense."""
    what = "decode_attention"
    dev = q3.device
    B, Hq, hd = q3.shape
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    err = _lib.error_word(dev)
    rp = _lib.ptr(remote_pages) if cap else None
    rc = _lib.ptr(remote_counts) if cap else None
    if page_table is not None:
        ws = _lib.workspace(dev, L.fsi_decode_attn_workspace_size(B, Hq, n_kv_heads, hd, window, cap, max_pages),
                            stream)
        st = L.fsi_decode_attn(q3.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), page_table.data_ptr(),
                               max_pages, n_phys, _lib.ptr(pos_rows), pos_val, window, rp, rc, cap, B, Hq, n_kv_heads,
                               hd, scale, out.data_ptr(), ws.data_ptr(), ws.numel(), err.data_ptr(), stream)
    else:
        k, v = k_cache, v_cache
        ws = _lib.workspace(dev, L.fsi_decode_attn_dense_workspace_size(B, Hq, hd, window, cap, page_size,
                                                                        max_seq_len), stream)
        st = L.fsi_decode_attn_dense(q3.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                                     k.stride(2), v.stride(0), v.stride(1), v.stride(2), max_seq_len,
                                     _lib.ptr(pos_rows), pos_val, window, page_size, rp, rc, cap, B, Hq, n_kv_heads,
                                     hd, scale, _lib.dtype_code(q3.dtype, what), out.data_ptr(), ws.data_ptr(),
                                     ws.numel(), err.data_ptr(), stream)
    _lib.check(st, what)
    if _lib.checks_enabled():
        _lib.raise_device_errors(dev, what)
    return out


@_lib.fsi_op("decode_attention", lambda q3, *rest: torch.empty_like(q3))
def _decode_op(q3: Tensor, k_cache: Tensor, v_cache: Tensor, page_table: Optional[Tensor], max_pages: int,
               n_phys: int, max_seq_len: int, page_size: int, n_kv_heads: int, pos_rows: Optional[Tensor],
               pos_val: int, window: int, remote_pages: Optional[Tensor], remote_counts: Optional[Tensor], cap: int,
               scale: float) -> Tensor:
    """Decode attention into a new (B, Hq, hd) tensor."""
    return _decode_launch(q3, k_cache, v_cache, page_table, max_pages, n_phys, max_seq_len, page_size, n_kv_heads,
                          pos_rows, pos_val, window, remote_pages, remote_counts, cap, scale, torch.empty_like(q3))


def _decode_step_fake(qi, kp, vp, completed, top_p, k_min, k_max, cap, want_ctx, q3, k_cache, v_cache, page_table,
                      max_pages, n_phys, pos_rows, pos_val, window, n_kv_heads, scale, batch0):
    B = q3.shape[0]
    return (torch.empty_like(q3), q3.new_empty((B, cap), dtype=torch.int32), q3.new_empty((B,), dtype=torch.int32),
            qi.new_empty((B, qi.shape[-1]) if want_ctx else (0,)))


@_lib.fsi_op("decode_step_attention", _decode_step_fake)
def _decode_step_op(qi: Tensor, kp: Tensor, vp: Optional[Tensor], completed: int, top_p: float, k_min: int,
                    k_max: int, cap: int, want_ctx: bool, q3: Tensor, k_cache: Tensor, v_cache: Tensor,
                    page_table: Tensor, max_pages: int, n_phys: int, pos_rows: Optional[Tensor], pos_val: int,
                    window: int, n_kv_heads: int, scale: float, batch0: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """fsi_decode_step_attn: (attention (B, Hq, hd), pages (B, cap), counts (B,), context (B, 16) or empty)."""
    what = "decode_step"
    dev = q3.device
    B, Hq, hd = q3.shape
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    out = torch.empty_like(q3)
    pages = torch.empty((B, cap), dtype=torch.int32, device=dev)
    counts = torch.empty((B,), dtype=torch.int32, device=dev)
    ctx = torch.empty((B, qi.shape[-1]) if want_ctx else (0,), dtype=qi.dtype, device=dev)
    ws = _lib.workspace(dev, L.fsi_decode_attn_workspace_size(B, Hq, n_kv_heads, hd, window, cap, max_pages), stream)
    err = _lib.error_word(dev)
    st = L.fsi_decode_step_attn(
        qi.data_ptr(), kp.data_ptr(), _lib.ptr(vp), kp.shape[1], completed, top_p, k_min, k_max, cap,
        pages.data_ptr(), counts.data_ptr(), ctx.data_ptr() if want_ctx else None, q3.data_ptr(),
        k_cache.data_ptr(), v_cache.data_ptr(), page_table.data_ptr(), max_pages, n_phys, _lib.ptr(pos_rows), pos_val,
        window, B, Hq, n_kv_heads, hd, scale, int(batch0), out.data_ptr(), ws.data_ptr(), ws.numel(), err.data_ptr(),
        stream)
    _lib.check(st, what)
    if _lib.checks_enabled():
        _lib.raise_device_errors(dev, what)
    return out, pages, counts, ctx


def decode_step_attention(q: Tensor, qi: Tensor, cache: FovealKVCache, *, pos: int | Tensor, window: int,
                          completed_pages: int, top_p: float, min_remote_blocks: int, max_remote_blocks: int,
                          scale: float, return_context: bool = False, batch0: bool = False):
    """Page routing and decode attention of one step (decode_route + decode_attention)
    through fsi_decode_step_attn: one launch when there is at least one (sequence, KV
    head) pair per compute unit (four waves of each pair's workgroup route the sequence
    while four stream the local window, then all stream the selected pages), otherwise
    two (routing beside the local window, then the selected pages and the merge).  Needs the paged bf16 cache and a bf16 index query.
    batch0: every sequence attends sequence 0's pages (attention.py:348).
    Returns (attention (B, Hq, hd), pages (B, cap), counts (B,)[, context (B, 16)]),
    cap = max(K_max, K_min, 1); no autograd (use decode_route + decode_attention)."""
    what = "decode_step"
    dev = _lib.require_gpu(q, qi, cache.kp_cache, what=what)
    if not cache.paged:
        raise ValueError(f"{what}: the fused step needs the paged cache layout")
    B = q.shape[0]
    Hq, hd = q.shape[1], q.shape[-1]
    q3 = q.detach().reshape(B, Hq, hd).contiguous()
    q2 = qi.detach().reshape(B, -1).contiguous()
    if q3.dtype != torch.bfloat16 or q2.dtype != torch.bfloat16 or q2.shape[1] != 16:
        raise TypeError(f"{what}: bf16 q and (B, 16) bf16 index query required")
    if B != cache.batch_size or hd != cache.head_dim:
        raise ValueError(f"{what}: q {tuple(q.shape)} does not match the cache")
    pos_rows, pos_val = None, 0
    if isinstance(pos, Tensor):
        pos_rows = pos.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
    else:
        pos_val = int(pos)
    cap = max(int(max_remote_blocks), int(min_remote_blocks), 1)
    vp = cache.vp_cache if return_context else None
    out, pages, counts, ctx = _decode_step_op(
        q2, cache.kp_cache, vp, int(completed_pages), float(top_p), int(min_remote_blocks), int(max_remote_blocks),
        cap, bool(return_context), q3, cache.k_cache, cache.v_cache, cache.page_table, cache.max_pages,
        cache.n_phys_pages, pos_rows, pos_val, int(window), cache.num_kv_heads, float(scale), bool(batch0))
    if return_context:
        return out, pages, counts, ctx
    return out, pages, counts


def _cache_args(cache: FovealKVCache):
    return (cache.k_cache, cache.v_cache, cache.page_table if cache.paged else None, cache.max_pages,
            cache.n_phys_pages if cache.paged else 0, cache.max_seq_len, cache.page_size, cache.num_kv_heads)


def _decode_attention_launch(q3: Tensor, cache: FovealKVCache, pos_rows: Optional[Tensor], pos_val: int,
                             window: int, remote_pages: Optional[Tensor], remote_counts: Optional[Tensor], cap: int,
                             scale: float, out: Optional[Tensor] = None) -> Tensor:
    args = (*_cache_args(cache), pos_rows, int(pos_val), int(window), remote_pages, remote_counts, int(cap),
            float(scale))
    if out is None:
        return _decode_op(q3, *args)
    return _decode_launch(q3, *args, out)


class _DecodeAttnFn(torch.autograd.Function):
    """Decode attention with a gradient for the query.  The cached keys and values
    are inference state (the kernels read them in place), so they are constants
    here; the backward (fsi_decode_attn_bwd_q) recomputes each sequence's softmax
    over its support on the device in fp32, one wave per (sequence, query head):
    dq = scale * sum_t p_t (dO . v_t - dO . o) k_t."""

    @staticmethod
    def forward(ctx, q3, cache, pos_rows, pos_val, window, remote_pages, remote_counts, cap, scale):
        out = _decode_attention_launch(q3, cache, pos_rows, pos_val, window, remote_pages, remote_counts, cap, scale)
        ctx.cache, ctx.meta = cache, (pos_val, window, cap, scale)
        ctx.save_for_backward(q3, pos_rows, remote_pages, remote_counts)
        return out

    @staticmethod
    def backward(ctx, dout):
        q3, pos_rows, remote_pages, remote_counts = ctx.saved_tensors
        cache = ctx.cache
        pos_val, window, cap, scale = ctx.meta
        what = "decode_attention backward"
        dev = q3.device
        B, Hq, hd = q3.shape
        dq = torch.empty((B, Hq, hd), dtype=torch.float32, device=dev)
        g = dout.reshape(B, Hq, hd).to(q3.dtype).contiguous()
        q = q3.contiguous()
        k, v = cache.k_cache, cache.v_cache
        paged = cache.paged
        ks = (0, 0, 0) if paged else (k.stride(0), k.stride(1), k.stride(2))
        vs = (0, 0, 0) if paged else (v.stride(0), v.stride(1), v.stride(2))
        L = _lib.lib()
        err = _lib.error_word(dev)
        st = L.fsi_decode_attn_bwd_q(
            q.data_ptr(), g.data_ptr(), k.data_ptr(), v.data_ptr(), *ks, *vs, cache.max_seq_len,
            cache.page_table.data_ptr() if paged else None, cache.max_pages, cache.n_phys_pages if paged else 0,
            _lib.ptr(pos_rows), int(pos_val), int(window), cache.page_size,
            _lib.ptr(remote_pages) if cap else None, _lib.ptr(remote_counts) if cap else None, int(cap), B, Hq,
            cache.num_kv_heads, hd, float(scale), _lib.dtype_code(q3.dtype, what), dq.data_ptr(), err.data_ptr(),
            _lib.stream_handle(dev))
        _lib.check(st, what)
        if _lib.checks_enabled():
            _lib.raise_device_errors(dev, what)
        return dq.to(q3.dtype), None, None, None, None, None, None, None, None


def decode_attention(
    q: Tensor,
    cache: FovealKVCache,
    *,
    pos: int | Tensor,
    window: int,
    remote_pages: Optional[Tensor],
    remote_counts: Optional[Tensor],
    scale: float,
    out: Optional[Tensor] = None,
) -> Tensor:
    """softmax(scale q K^T) V over [max(0, pos + 1 - window), pos] plus the
    selected remote pages, for every sequence and query head (attention.py:339-365).
    q: (B, Hq, hd) or (B, Hq, 1, hd) in the cache's dtype.  Returns (B, Hq, hd).
    Paged caches run the split-K MFMA kernels, contiguous ones the generic
    kernel.  Differentiable in q (the cached keys and values are constants)."""
    what = "decode_attention"
    dev = _lib.require_gpu(q, cache.k_cache, what=what)
    B = q.shape[0]
    Hq, hd = q.shape[1], q.shape[-1]
    q3 = q.reshape(B, Hq, hd)
    if q3.dtype != cache.dtype:
        raise TypeError(f"{what}: q dtype {q3.dtype} != cache dtype {cache.dtype}")
    if B != cache.batch_size or hd != cache.head_dim:
        raise ValueError(f"{what}: q {tuple(q.shape)} does not match the cache")
    pos_rows, pos_val = None, 0
    if isinstance(pos, Tensor):
        pos_rows = pos.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
    else:
        pos_val = int(pos)
    cap = 0
    if remote_pages is not None and remote_pages.numel():
        remote_pages = remote_pages.to(device=dev, dtype=torch.int32).contiguous()
        remote_counts = remote_counts.to(device=dev, dtype=torch.int32).contiguous()
        cap = remote_pages.shape[-1]
    else:
        remote_pages = remote_counts = None
    if torch.is_grad_enabled() and q3.requires_grad:
        res = _DecodeAttnFn.apply(q3.contiguous(), cache, pos_rows, pos_val, int(window), remote_pages,
                                  remote_counts, cap, float(scale))
        if out is not None:
            out.copy_(res.detach())
        return res
    return _decode_attention_launch(q3.detach().contiguous(), cache, pos_rows, pos_val, int(window), remote_pages,
                                    remote_counts, cap, float(scale), out)


SATTN_LOCAL_REMOTE = 0  # FSI_SATTN_LOCAL_REMOTE
SATTN_BLOCK_LIST = 1  # FSI_SATTN_BLOCK_LIST


def _attn_operand(t: Tensor, what: str, name: str) -> Tensor:
    if t.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{what}: {name} dtype {t.dtype} unsupported (bfloat16 or float32)")
    if t.dim() != 4:
        raise ValueError(f"{what}: {name} must be (B, H, T, head_dim), got {tuple(t.shape)}")
    if t.stride(3) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _sparse_attention_launch(q, k, v, lists, counts, cap, block, mode, window, scale, out):
    what = "sparse_attention"
    dev = q.device
    B, Hq, T, hd = q.shape
    Hkv = k.shape[1]
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    ws = _lib.workspace(dev, L.fsi_sparse_attn_workspace_size(B, Hkv, T, hd), stream)
    err = _lib.error_word(dev)
    st = L.fsi_sparse_attn(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), B, Hq, Hkv, T, hd, int(block), int(mode), int(window),
        _lib.ptr(lists), lists.stride(0) if cap else 0, lists.stride(1) if cap else 0, cap, counts.data_ptr(),
        counts.stride(0), counts.stride(1), float(scale), _lib.dtype_code(q.dtype, what), out.data_ptr(),
        out.stride(0), out.stride(1), out.stride(2), ws.data_ptr(), ws.numel(), err.data_ptr(), stream)
    _lib.check(st, what)
    if _lib.checks_enabled():
        _lib.raise_device_errors(dev, what)
    return out


def _sparse_out(q: Tensor) -> Tensor:
    B, Hq, T, hd = q.shape
    return q.new_empty((B, T, Hq, hd)).transpose(1, 2)


@_lib.fsi_op("sparse_attention", lambda q, k, v, lists, counts, cap, block, mode, window, scale: _sparse_out(q))
def _sparse_attn_op(q: Tensor, k: Tensor, v: Tensor, lists: Optional[Tensor], counts: Tensor, cap: int, block: int,
                    mode: int, window: int, scale: float) -> Tensor:
    """fsi_sparse_attn into a new (B, Hq, T, hd) tensor laid out as (B, T, Hq, hd)."""
    return _sparse_attention_launch(q, k, v, lists, counts, cap, block, mode, window, scale, _sparse_out(q))


def _sparse_attention_bwd(q, k, v, out, dout, lists, counts, cap, block, mode, window, scale):
    """fsi_sparse_attn_bwd: fp32 (dq, dk, dv) of sparse_attention over the same
    pattern, from the saved operands and output, without any (T, T) tensor."""
    what = "sparse_attention backward"
    dev = q.device
    B, Hq, T, hd = q.shape
    Hkv = k.shape[1]
    dout = _attn_operand(dout.to(q.dtype), what, "grad")
    dq = torch.empty((B, Hq, T, hd), dtype=torch.float32, device=dev)
    dk = torch.empty((B, Hkv, T, hd), dtype=torch.float32, device=dev)
    dv = torch.empty_like(dk)
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    ws = _lib.workspace(dev, L.fsi_sparse_attn_bwd_workspace_size(B, Hq, T, int(block)), stream)
    err = _lib.error_word(dev)
    st = L.fsi_sparse_attn_bwd(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), out.data_ptr(), out.stride(0), out.stride(1),
        out.stride(2), dout.data_ptr(), dout.stride(0), dout.stride(1), dout.stride(2), B, Hq, Hkv, T, hd,
        int(block), int(mode), int(window), _lib.ptr(lists), lists.stride(0) if cap else 0,
        lists.stride(1) if cap else 0, cap, counts.data_ptr(), counts.stride(0), counts.stride(1), float(scale),
        _lib.dtype_code(q.dtype, what), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws.numel(),
        err.data_ptr(), stream)
    _lib.check(st, what)
    if _lib.checks_enabled():
        _lib.raise_device_errors(dev, what)
    return dq, dk, dv


class _SparseAttnFn(torch.autograd.Function):
    """sparse_attention with gradients for q, k and v.  The forward is the HIP
    kernel; the backward is the HIP backward (fsi_sparse_attn_bwd): the block
    map of the pattern, then per 64-query tile the row statistics and dQ, and
    per 64-key tile dK and dV accumulated over the query tiles that reach it, in
    fp32 on LDS tiles; memory O(T hd) plus (T / block)^2 block entries, never
    the (T, T) scores the reference's masked SDPA materialises."""

    @staticmethod
    def forward(ctx, q, k, v, lists, counts, cap, block, mode, window, scale):
        out = _sparse_attn_op(q, k, v, lists, counts, cap, block, mode, window, scale)
        ctx.save_for_backward(q, k, v, lists, counts, out)
        ctx.meta = (cap, block, mode, window, scale)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, lists, counts, out = ctx.saved_tensors
        cap, block, mode, window, scale = ctx.meta
        if q.shape[-1] <= 128:
            dq, dk, dv = _sparse_attention_bwd(q, k, v, out, dout, lists, counts, cap, block, mode, window, scale)
        else:  # head_dim 129..256: the LDS tiles do not fit; dense fp32 recompute over the pattern
            dq, dk, dv = _sparse_attention_bwd_dense(q, k, v, dout, lists, counts, cap, block, mode, window, scale)
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None, None, None, None)


def _sparse_logit_bias(lists, counts, cap, B, T, block, mode, window, dev):
    """(B, 1, T, T) additive logit bias of a sparse pattern: 0 for an allowed key
    (log of its multiplicity for block lists), -inf elsewhere (the reference
    builds the same boolean mask, attention.py:148-176)."""
    nb = -(-T // block)
    mult = torch.zeros(B, nb, nb + 1, dtype=torch.float32, device=dev)  # last column: ids out of range
    if cap:
        slot = torch.arange(cap, device=dev)
        valid = slot[None, None] < counts.clamp(0, cap)[..., None]
        ids = lists.long().clamp(-1, nb)
        ids = torch.where(valid & (ids >= 0) & (ids < nb), ids, torch.full_like(ids, nb))
        mult.scatter_add_(2, ids, valid.float())
    mult = mult[..., :nb]
    tb = torch.arange(T, device=dev) // block
    page = mult[:, tb][:, :, tb]  # (B, T, T): multiplicity of key s's block for query t's block
    if mode == SATTN_LOCAL_REMOTE:
        t = torch.arange(T, device=dev)
        win = (t[None, :] <= t[:, None]) & (t[None, :] > t[:, None] - window)
        allowed = win[None] | (page > 0)
        bias = torch.zeros(B, T, T, device=dev).masked_fill_(~allowed, float("-inf"))
    else:
        bias = torch.where(page > 0, page.log(), torch.full_like(page, float("-inf")))
    return bias[:, None]


def _sparse_attention_bwd_dense(q, k, v, dout, lists, counts, cap, block, mode, window, scale):
    """Gradients of sparse_attention by a dense fp32 recompute over the pattern
    (B x Hq x T x T memory) with library matmuls; only for head_dim > 128."""
    B, Hq, T, hd = q.shape
    G = Hq // k.shape[1]
    bias = _sparse_logit_bias(lists, counts, cap, B, T, block, mode, window, q.device)
    with torch.enable_grad():
        qf = q.detach().float().requires_grad_()
        kf = k.detach().float().requires_grad_()
        vf = v.detach().float().requires_grad_()
        ke = kf.repeat_interleave(G, dim=1)
        ve = vf.repeat_interleave(G, dim=1)
        s = torch.matmul(qf, ke.transpose(-1, -2).contiguous()) * scale + bias
        empty = torch.isneginf(s).all(dim=-1, keepdim=True)  # rows with no key give 0
        p = torch.softmax(s.masked_fill(empty, 0.0), dim=-1).masked_fill(empty, 0.0)
        o = torch.matmul(p, ve)
        return torch.autograd.grad(o, (qf, kf, vf), dout.float())


def sparse_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    lists: Optional[Tensor],
    counts: Tensor,
    *,
    block: int,
    mode: int = SATTN_LOCAL_REMOTE,
    window: int = 0,
    scale: Optional[float] = None,
    out: Optional[Tensor] = None,
) -> Tensor:
    """Block-sparse attention of q (B, Hq, T, hd) over k, v (B, Hkv, T, hd), bf16
    or fp32 (fp32 softmax and accumulation either way).

    mode SATTN_LOCAL_REMOTE (attention.py:148-218): query t sees keys s with
    t - window < s <= t plus every key of the pages lists[b, t // block, :counts]
    (a union).  mode SATTN_BLOCK_LIST (triton_ops.py:26-93): query block qb sees
    every key of the listed key blocks.  lists: (B, ceil(T / block), capacity)
    int32; counts: (B, ceil(T / block)).  Views with unit stride over head_dim
    (such as proj(x).view(B, T, H, hd).transpose(1, 2)) are read in place; `out`
    may be such a view too.  Differentiable in q, k and v.  Returns (B, Hq, T, hd)."""
    what = "sparse_attention"
    dev = _lib.require_gpu(q, k, v, counts, lists, what=what)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError(f"{what}: q, k, v dtypes {q.dtype}, {k.dtype}, {v.dtype} differ")
    qa, ka, va = (_attn_operand(t, what, n) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    B, Hq, T, hd = qa.shape
    Hkv = ka.shape[1]
    if tuple(ka.shape) != (B, Hkv, T, hd) or tuple(va.shape) != (B, Hkv, T, hd) or Hq % Hkv:
        raise ValueError(f"{what}: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)} do not match")
    Qb = -(-T // block)
    counts = counts.to(device=dev, dtype=torch.int32)
    if tuple(counts.shape) != (B, Qb):
        raise ValueError(f"{what}: counts {tuple(counts.shape)} != {(B, Qb)}")
    cap = 0
    if lists is not None and lists.numel():
        lists = lists.to(device=dev, dtype=torch.int32)
        if lists.dim() != 3 or tuple(lists.shape[:2]) != (B, Qb) or lists.stride(2) != 1:
            lists = lists.contiguous()
        if lists.dim() != 3 or tuple(lists.shape[:2]) != (B, Qb):
            raise ValueError(f"{what}: lists {tuple(lists.shape)} != {(B, Qb)} + (capacity,)")
        cap = lists.shape[2]
    else:
        lists = None
    if scale is None:
        scale = 1.0 / math.sqrt(hd)
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        res = _SparseAttnFn.apply(qa, ka, va, lists, counts, cap, int(block), int(mode), int(window), float(scale))
        if out is not None:
            out.copy_(res.detach())
        return res
    if out is None:
        return _sparse_attn_op(qa.detach(), ka.detach(), va.detach(), lists, counts, cap, int(block), int(mode),
                               int(window), float(scale))
    if tuple(out.shape) != (B, Hq, T, hd) or out.dtype != qa.dtype or out.stride(3) != 1:
        raise ValueError(f"{what}: out must be a (B, Hq, T, hd) {qa.dtype} tensor with unit stride over hd")
    return _sparse_attention_launch(qa.detach(), ka.detach(), va.detach(), lists, counts, cap, block, mode, window,
                                    scale, out)


def triton_foveal_sparse_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    block_indices: Tensor,
    active_counts: Tensor,
    scale: Optional[float] = None,
    block_size: int = 16,
) -> Tensor:
    """Block-sparse attention (triton_ops.py:256-313): query block m of
    block_size queries attends every key of block_indices[b, m, :active_counts[b, m]],
    with no causal mask; a query block with no active block gets 0.  q, k, v:
    (B, H, N, D) bf16 or fp32 with N % block_size == 0.  The `triton_` name is
    kept for compatibility; the kernels are HIP (MFMA for bf16 with block_size a
    multiple of 16 and D 16, 32, 64 or 128; the generic kernel otherwise)."""
    B, H, N, D = q.shape
    if N % block_size != 0:
        raise ValueError(f"N ({N}) must be divisible by block_size ({block_size})")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    res = sparse_attention(q, k, v, block_indices, active_counts, block=block_size, mode=SATTN_BLOCK_LIST,
                           scale=scale)
    return res.contiguous()


_SRAM_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}


def sram_indexer_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    q16: Tensor,
    k16: Tensor,
    scale: Optional[float] = None,
    top_p: float = 0.8,
    max_remote_blocks: int = 2,
    block_size: int = 16,
    return_selection: bool = False,
):
    """Fused 16-D block indexer, greedy block selection and block attention in
    one HIP launch (fsi_sram_indexer_attention).  q, k, v: (B, H, N, D) fp32,
    bf16 or fp16; q16, k16: (B, N / block_size, 16) in q's dtype or fp32.  With
    return_selection, also returns the (B, N / block_size, max_remote_blocks)
    int32 picks (-1 where a pick is not attended).  No autograd, as the
    reference kernel."""
    what = "triton_fused_sram_indexer_attention"
    if not q.is_cuda:
        raise RuntimeError(f"{what} requires a GPU tensor (the HIP library)")
    B, H, N, D = q.shape
    if N % block_size != 0:
        raise AssertionError(f"N ({N}) must be divisible by block_size ({block_size})")
    M = N // block_size
    if q.dtype not in _SRAM_DTYPES:
        raise TypeError(f"{what}: dtype {q.dtype} unsupported (float32, bfloat16 or float16)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"{what}: q, k and v must share one dtype")
    if tuple(k.shape) != (B, H, N, D) or tuple(v.shape) != (B, H, N, D):
        raise ValueError(f"{what}: k and v must be {(B, H, N, D)}")
    if tuple(q16.shape) != (B, M, 16) or tuple(k16.shape) != (B, M, 16):
        raise ValueError(f"{what}: q16 and k16 must be {(B, M, 16)}")
    idx_dtype = q.dtype if q16.dtype == q.dtype and k16.dtype == q.dtype else torch.float32
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    q, k, v = (t.detach().contiguous() for t in (q, k, v))
    q16 = q16.detach().to(idx_dtype).contiguous()
    k16 = k16.detach().to(idx_dtype).contiguous()
    out, sel = _sram_op(q, k, v, q16, k16, float(scale), float(top_p), int(max_remote_blocks), int(block_size),
                        bool(return_selection))
    return (out, sel) if return_selection else out


def _sram_fake(q, k, v, q16, k16, scale, top_p, max_remote, block_size, want_sel):
    B, M = q16.shape[0], q16.shape[1]
    return torch.empty_like(q), q.new_empty((B, M, max_remote) if want_sel else (0,), dtype=torch.int32)


@_lib.fsi_op("sram_indexer_attention", _sram_fake)
def _sram_op(q: Tensor, k: Tensor, v: Tensor, q16: Tensor, k16: Tensor, scale: float, top_p: float, max_remote: int,
             block_size: int, want_sel: bool) -> Tuple[Tensor, Tensor]:
    """fsi_sram_indexer_attention: (out (B, H, N, D), picks (B, M, max_remote) int32 or empty)."""
    B, H, N, D = q.shape
    M = q16.shape[1]
    out = torch.empty_like(q)
    sel = torch.empty((B, M, max_remote) if want_sel else (0,), dtype=torch.int32, device=q.device)
    st = _lib.lib().fsi_sram_indexer_attention(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _SRAM_DTYPES[q.dtype], q16.data_ptr(), k16.data_ptr(),
        _SRAM_DTYPES[q16.dtype], B, H, N, D, block_size, max_remote, scale, top_p, out.data_ptr(),
        sel.data_ptr() if want_sel else None, _lib.stream_handle(q.device))
    _lib.check(st, "triton_fused_sram_indexer_attention")
    return out, sel


def triton_fused_sram_indexer_attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    q16: Tensor,
    k16: Tensor,
    scale: Optional[float] = None,
    top_p: float = 0.8,
    max_remote_blocks: int = 2,
    block_size: int = 16,
) -> Tensor:
    """Foveal sparse attention with the 16-D indexing and routing fused into the
    attention launch (triton_ops.py:373-435, kernel :142-249): query block m
    scores all blocks with q16 . k16 / 4, softmaxes over the other blocks, takes
    up to max_remote_blocks greedy picks while the picked mass stays below top_p
    (each pick > 1e-4), and attends its own block plus the picks (no causal
    mask).  q, k, v: (B, H, N, D); q16, k16: (B, N / block_size, 16).  The
    `triton_` name is kept for compatibility; the kernel is HIP."""
    return sram_indexer_attention(q, k, v, q16, k16, scale=scale, top_p=top_p, max_remote_blocks=max_remote_blocks,
                                  block_size=block_size)


class FovealSparseAttention(nn.Module):
    """Causal foveal sparse attention (attention.py:97-379): same constructor,
    parameters (state_dict compatible), `init_kv_cache` and `decode_step`.

    decode_step runs on the MI355X path: 16-D index projections + norm, paged
    cache append, page routing + additive-stream context in one launch, and
    split-K paged attention over the local window plus the selected pages.
    Every sequence attends its own selected pages; the reference attends
    sequence 0's pages for all sequences (attention.py:348) and
    `reference_batch0_pages = True` reproduces that.  `selected_remote_pages`
    reports each sequence's own selection in both modes, as the reference does.
    The prefill `forward` routes with the HIP indexer ops and runs one
    block-sparse attention launch (`sparse_attention`).  Both paths take the
    reference's dtypes (fp32 by default, bf16) and are differentiable: the
    attention backward recomputes the sparse pattern densely (as the reference's
    forward does), decode's gradient reaches q (the cache is inference state).
    """

    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        num_kv_heads: Optional[int] = None,
        head_dim: Optional[int] = None,
        page_size: int = 64,
        local_window_blocks: int = 4,
        index_dim: int = 16,
        top_p: float = 0.95,
        min_remote_pages: int = 0,
        max_remote_pages: int = 8,
        remote_capacity: int = 8,
        use_additive_stream: bool = True,
    ):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads if num_kv_heads is not None else num_heads
        self.head_dim = head_dim if head_dim is not None else hidden_size // num_heads
        self.page_size = page_size
        self.local_window_blocks = local_window_blocks
        self.local_window = local_window_blocks * page_size
        self.use_additive_stream = use_additive_stream
        self.groups = self.num_heads // self.num_kv_heads
        self.scale = 1.0 / math.sqrt(self.head_dim)
        self.reference_batch0_pages = False

        self.q_proj = nn.Linear(hidden_size, self.num_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.num_kv_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.num_kv_heads * self.head_dim, bias=False)
        self.out_proj = nn.Linear(self.num_heads * self.head_dim, hidden_size, bias=False)
        self.indexer = FovealIndexer(
            hidden_size=hidden_size,
            index_dim=index_dim,
            block_size=page_size,
            local_window_blocks=local_window_blocks,
            top_p=top_p,
            min_remote_blocks=min_remote_pages,
            max_remote_blocks=max_remote_pages,
            remote_capacity=remote_capacity,
            causal=True,
            use_additive_stream=use_additive_stream,
        )

    def forward(self, x: Tensor, compute_teacher_loss: bool = False) -> Tuple[Tensor, Dict[str, Any]]:
        """Prefill forward pass (attention.py:180-269).  x: (B, T, D), T a
        multiple of page_size.  Returns (out (B, T, D), aux with 'route',
        'additive_out', 'distill_loss').

        The attention runs as one block-sparse HIP launch over the local window
        plus each query block's routed pages (the reference builds a (B, T, T)
        boolean mask and calls dense SDPA).  The teacher for the distillation loss
        (attention.py:243-267) needs only the softmax rows of the query-block
        anchors, which are computed in fp32 for those rows alone."""
        batch, seq_len, _ = x.shape
        if seq_len % self.page_size != 0:
            raise ValueError(f"Sequence length {seq_len} must be multiple of page_size {self.page_size}")
        num_pages = seq_len // self.page_size

        x_detach = x.detach()
        q_16d = self.indexer.compute_query_16d(x_detach)
        kp_16d, vp_16d = self.indexer.compute_kv_blocks_16d(x_detach)
        q_block_16d = q_16d[:, :: self.page_size]
        block_scores = self.indexer.compute_block_scores(q_block_16d, kp_16d)
        route = self.indexer.route(block_scores)

        q = self.q_proj(x).view(batch, seq_len, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(x).view(batch, seq_len, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(x).view(batch, seq_len, self.num_kv_heads, self.head_dim).transpose(1, 2)

        # (B, Hq, T, hd) view of a (B, T, Hq, hd) buffer: the heads merge without a copy
        attn = sparse_attention(q, k, v, route.remote_indices, route.remote_counts, block=self.page_size,
                                mode=SATTN_LOCAL_REMOTE, window=self.local_window, scale=self.scale)
        out = self.out_proj(attn.transpose(1, 2).reshape(batch, seq_len, self.num_heads * self.head_dim))

        additive_out = None
        if self.use_additive_stream:
            additive_out = self.indexer.additive_stream(block_scores, vp_16d)
            out = out + additive_out

        aux: Dict[str, Any] = {
            "route": route,
            "additive_out": additive_out,
            "distill_loss": torch.tensor(0.0, device=x.device),
        }
        if compute_teacher_loss:
            with torch.no_grad():
                teacher_mass = self._teacher_page_mass(q, k, num_pages)
            aux["distill_loss"] = self.indexer.distillation_loss(block_scores, teacher_mass)
        return out, aux

    def _teacher_page_mass(self, q: Tensor, k: Tensor, num_pages: int) -> Tensor:
        """Dense causal attention mass per key page for the first query of each
        query block, averaged over heads (attention.py:243-265): (B, Q_blocks, pages)."""
        batch, _, seq_len, hd = q.shape
        qa = q[:, :, :: self.page_size].float().reshape(batch, self.num_kv_heads, self.groups * num_pages, hd)
        s = torch.matmul(qa.contiguous(), k.float().transpose(-2, -1).contiguous()) * self.scale
        s = s.view(batch, self.num_heads, num_pages, seq_len)
        anchors = torch.arange(0, seq_len, self.page_size, device=q.device)
        keys = torch.arange(seq_len, device=q.device)
        s = s.masked_fill(keys[None, :] > anchors[:, None], -float("inf"))
        probs = torch.softmax(s, dim=-1)
        page_mass = probs.view(batch, self.num_heads, num_pages, num_pages, self.page_size).sum(dim=-1)
        return page_mass.mean(dim=1)

    def init_kv_cache(self, batch_size: int, max_seq_len: int, device: torch.device) -> FovealKVCache:
        """A paged cache for decoding (attention.py:271-282)."""
        return FovealKVCache(
            batch_size=batch_size,
            max_seq_len=max_seq_len,
            num_kv_heads=self.num_kv_heads,
            head_dim=self.head_dim,
            index_dim=self.indexer.index_dim,
            page_size=self.page_size,
            device=device,
            dtype=self.q_proj.weight.dtype,
        )

    def decode_step(self, x_step: Tensor, kv_cache: FovealKVCache) -> Tuple[Tensor, Dict[str, Any]]:
        """One autoregressive step for every sequence (attention.py:284-379)."""
        batch, seq_one, _ = x_step.shape
        if seq_one != 1:
            raise ValueError("decode_step processes one token at a time")
        pos = kv_cache.seq_len
        q = self.q_proj(x_step).view(batch, self.num_heads, self.head_dim)
        k = self.k_proj(x_step).view(batch, self.num_kv_heads, 1, self.head_dim)
        v = self.v_proj(x_step).view(batch, self.num_kv_heads, 1, self.head_dim)
        x_detach = x_step.detach()
        qi = self.indexer.compute_query_16d(x_detach)
        ki = index_rms_norm(self.indexer.k_proj(x_detach), "decode_step")
        vi = self.indexer.v_proj(x_detach)
        kv_cache.update(k, v, ki, vi)

        completed = kv_cache.completed_pages
        want_ctx = self.use_additive_stream and completed > 0
        fused = (kv_cache.paged and qi.dtype == torch.bfloat16
                 and not (torch.is_grad_enabled() and q.requires_grad))
        if fused:  # routing beside the local-window attention, one stream
            res = decode_step_attention(
                q, qi, kv_cache, pos=pos, window=self.local_window, completed_pages=completed,
                top_p=self.indexer.top_p, min_remote_blocks=self.indexer.min_remote_blocks,
                max_remote_blocks=self.indexer.max_remote_blocks, scale=self.scale, return_context=want_ctx,
                batch0=self.reference_batch0_pages)
            attn, pages, counts = res[0], res[1], res[2]
            return self._decode_finish(attn, pages, counts, res[3] if want_ctx else None, batch)
        routed = decode_route(
            qi, kv_cache.kp_cache, kv_cache.vp_cache, pos=pos, page_size=self.page_size,
            local_window=self.local_window, completed_pages=completed, top_p=self.indexer.top_p,
            min_remote_blocks=self.indexer.min_remote_blocks, max_remote_blocks=self.indexer.max_remote_blocks,
            return_context=want_ctx)
        pages, counts = routed[0], routed[1]
        att_pages, att_counts = pages, counts
        if self.reference_batch0_pages:
            att_pages = pages[:1].expand(batch, -1).contiguous()
            att_counts = counts[:1].expand(batch).contiguous()
        attn = decode_attention(q, kv_cache, pos=pos, window=self.local_window, remote_pages=att_pages,
                                remote_counts=att_counts, scale=self.scale)
        return self._decode_finish(attn, pages, counts, routed[2] if want_ctx else None, batch)

    def _decode_finish(self, attn: Tensor, pages: Tensor, counts: Tensor, ctx: Optional[Tensor], batch: int):
        out = self.out_proj(attn.reshape(batch, 1, self.num_heads * self.head_dim))
        if ctx is not None:
            out = out + self.indexer.out_proj(ctx.view(batch, 1, -1))
        cnt = counts.tolist()
        rows = pages.tolist()
        selected: List[List[int]] = [rows[b][:cnt[b]] for b in range(batch)]
        return out, {"selected_remote_pages": selected}
