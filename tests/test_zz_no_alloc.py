"""fsi_decode_attn_noalloc (partials in the library's static device scratch)
against fsi_decode_attn (partials in a caller workspace), both called through
the C ABI: two calls in a row, the second on a smaller input, each output equal
to the workspace entry point's bit for bit (the same kernels on the same inputs)
and within the bf16 tolerance of the fp64 oracle."""
import math

import pytest
import torch

from oracle import attention as A
from oracle import pattention as Pt

pytestmark = pytest.mark.gpu


def _case(fsi, dev, B, Hq, Hkv, hd, max_seq, seed):
    g = torch.Generator().manual_seed(seed)
    P = -(-max_seq // 64)
    n_phys = B * P + 5
    table = torch.randperm(n_phys, generator=g)[:B * P].view(B, P).to(torch.int32)
    c = fsi.FovealKVCache(B, max_seq, Hkv, hd, 16, 64, dev, torch.bfloat16, n_phys_pages=n_phys, page_table=table)
    k = torch.randn(B, Hkv, max_seq, hd, generator=g).bfloat16()
    v = torch.randn(B, Hkv, max_seq, hd, generator=g).bfloat16()
    c.load_dense(k.to(dev), v.to(dev))
    q = torch.randn(B, Hq, hd, generator=g).bfloat16()
    return c, k, v, q


def _call(L, _lib, fn, c, q, pos, W, rp, cnt, scale, out, ws=None):
    args = [q.data_ptr(), c.k_cache.data_ptr(), c.v_cache.data_ptr(), c.page_table.data_ptr(), c.max_pages,
            c.n_phys_pages, None, pos, W, rp.data_ptr(), cnt.data_ptr(), rp.shape[1], q.shape[0], q.shape[1],
            c.num_kv_heads, q.shape[2], scale, out.data_ptr()]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    args += [None, torch.cuda.current_stream().cuda_stream]
    st = getattr(L, fn)(*args)
    assert st == 0, (fn, _lib.lib().fsi_last_error())


def test_decode_attn_noalloc_matches_workspace_entry_point(fsi, dev):
    from foveal_sparse_indexer_amd import _lib

    L = _lib.lib()
    cases = [  # the second call is smaller than the first
        (8, 32, 8, 128, 4096, 4000, 1024, [[0, 3, 7, 11, 20], [1], [2, 5], [], [9, 8], [4], [30, 31], [6]]),
        (2, 8, 2, 64, 1024, 700, 128, [[0, 5, 3], [2]]),
    ]
    for i, (B, Hq, Hkv, hd, max_seq, pos, W, pages) in enumerate(cases):
        print(f"[case] noalloc call {i}: B={B} Hq={Hq} hd={hd} pos={pos}", flush=True)
        c, k, v, q = _case(fsi, dev, B, Hq, Hkv, hd, max_seq, seed=10 + i)
        cap = max(1, max(len(p) for p in pages))
        rp = torch.full((B, cap), -1, dtype=torch.int32)
        for b, p in enumerate(pages):
            rp[b, :len(p)] = torch.tensor(p, dtype=torch.int32)
        cnt = torch.tensor([len(p) for p in pages], dtype=torch.int32)
        qd, rpd, cntd = q.to(dev), rp.to(dev), cnt.to(dev)
        scale = 1.0 / math.sqrt(hd)
        need = L.fsi_decode_attn_workspace_size(B, Hq, Hkv, hd, W, cap, c.max_pages)
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        ref_out = torch.empty(B, Hq, hd, dtype=torch.bfloat16, device=dev)
        got = torch.full((B, Hq, hd), float("nan"), dtype=torch.bfloat16, device=dev)
        _call(L, _lib, "fsi_decode_attn", c, qd, pos, W, rpd, cntd, scale, ref_out, ws)
        _call(L, _lib, "fsi_decode_attn_noalloc", c, qd, pos, W, rpd, cntd, scale, got)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref_out.cpu())
        exact = A.decode_attention_f64(q.float(), k, v, pos, W, pages, 64, scale)
        assert Pt.rel_l2(got.cpu().float(), exact.float()) <= 2e-3


def test_decode_attn_noalloc_rejects_oversized(fsi, dev):
    """Partials beyond the static scratch are refused before any launch."""
    from foveal_sparse_indexer_amd import _lib

    L = _lib.lib()
    B, Hq, Hkv, hd, W, cap, max_pages = 4096, 64, 4, 128, 8192, 64, 4096
    need = L.fsi_decode_attn_workspace_size(B, Hq, Hkv, hd, W, cap, max_pages)
    assert need > (16 << 20)
    x = torch.empty(64, dtype=torch.bfloat16, device=dev)
    st = L.fsi_decode_attn_noalloc(x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), max_pages, 8, None, 0, W,
                                   x.data_ptr(), x.data_ptr(), cap, B, Hq, Hkv, hd, 0.1, x.data_ptr(), None, None)
    assert st == _lib.FSI_ERR_CAPACITY
    assert b"scratch" in L.fsi_last_error()
