"""Foveal sparse attention decode path on MI355X: drop-in pieces of
foveal_indexer/attention.py.

decode_route: the per-step remote-page routing and additive-stream context of
FovealSparseAttention.decode_step (attention.py:313-337,369-376) as one HIP
launch over the whole batch (the reference loops over sequences in Python with
a host sync per sequence).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _lib


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
    pages = torch.empty((B, cap), dtype=torch.int32, device=dev)
    counts = torch.empty((B,), dtype=torch.int32, device=dev)
    ctx = torch.empty((B, d), dtype=q2.dtype, device=dev) if return_context else None
    st = _lib.lib().fsi_decode_route(
        q2.data_ptr(), kpc.data_ptr(), _lib.ptr(vpc), code, B, P, d, _lib.ptr(pos_rows), pos_val, int(page_size),
        int(local_window), int(completed_pages), float(top_p), int(min_remote_blocks), int(max_remote_blocks), cap,
        pages.data_ptr(), counts.data_ptr(), _lib.ptr(ctx), _lib.stream_handle(dev))
    _lib.check(st, what)
    if return_context:
        return pages, counts, ctx
    return pages, counts
