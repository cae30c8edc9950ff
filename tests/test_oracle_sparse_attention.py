"""Pins of the prefill sparse-attention oracle (CPU only).

sparse_mask is checked against a per-element set-membership restatement of
_build_sparse_mask (attention.py:148-178); weighted_attention_f64 with a boolean
mask against torch's SDPA with the same mask and repeat_interleave'd KV heads
(the call of attention.py:199-216); block_list_weights' multiplicities against
attention over explicitly concatenated key blocks (what the Triton kernel's loop
of triton_ops.py:67-88 computes when a block is listed twice)."""
import math

import torch
import torch.nn.functional as F

from oracle import attention as A


def _brute_mask(B, T, W, ps, idx, cnt):
    out = torch.zeros(B, T, T, dtype=torch.bool)
    for b in range(B):
        for t in range(T):
            listed = set(int(p) for p in idx[b, t // ps, :int(cnt[b, t // ps])])
            for s in range(T):
                out[b, t, s] = (t - W < s <= t) or (s // ps in listed)
    return out


def test_sparse_mask_matches_membership_rule():
    g = torch.Generator().manual_seed(0)
    B, T, W, ps = 2, 96, 20, 16
    Qb = T // ps
    idx = torch.randint(0, Qb, (B, Qb, 3), generator=g, dtype=torch.int32)
    cnt = torch.randint(0, 4, (B, Qb), generator=g, dtype=torch.int32)
    idx[0, 3] = torch.tensor([1, 1, 5])  # a duplicate and a future page
    cnt[0, 3] = 3
    got = A.sparse_mask(B, T, W, ps, idx, cnt)
    assert torch.equal(got, _brute_mask(B, T, W, ps, idx, cnt))
    # no pages: exactly the causal band
    band = A.sparse_mask(1, 40, 7, 8, torch.zeros(1, 5, 0, dtype=torch.int32), torch.zeros(1, 5, dtype=torch.int32))
    t = torch.arange(40)
    assert torch.equal(band[0], (t[None] <= t[:, None]) & (t[None] > t[:, None] - 7))


def test_weighted_attention_matches_sdpa_with_bool_mask():
    g = torch.Generator().manual_seed(1)
    B, Hq, Hkv, T, hd = 2, 6, 2, 48, 16
    q = torch.randn(B, Hq, T, hd, generator=g)
    k = torch.randn(B, Hkv, T, hd, generator=g)
    v = torch.randn(B, Hkv, T, hd, generator=g)
    idx = torch.randint(0, 6, (B, 6, 2), generator=g, dtype=torch.int32)
    cnt = torch.randint(0, 3, (B, 6), generator=g, dtype=torch.int32)
    mask = A.sparse_mask(B, T, 10, 8, idx, cnt)
    got = A.weighted_attention_f64(q, k, v, mask, 0.3)
    ref = F.scaled_dot_product_attention(q.double(), k.double().repeat_interleave(3, dim=1),
                                         v.double().repeat_interleave(3, dim=1), attn_mask=mask[:, None], scale=0.3)
    assert torch.allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_block_list_weights_equal_concatenated_keys():
    g = torch.Generator().manual_seed(2)
    B, H, T, hd, blk = 1, 2, 32, 8, 8
    q = torch.randn(B, H, T, hd, generator=g)
    k = torch.randn(B, H, T, hd, generator=g)
    v = torch.randn(B, H, T, hd, generator=g)
    idx = torch.tensor([[[2, 0, 2], [1, 3, 3], [0, 0, 0], [3, 1, 2]]], dtype=torch.int32)
    cnt = torch.tensor([[3, 1, 0, 2]], dtype=torch.int32)
    w = A.block_list_weights(B, T, blk, idx, cnt)
    got = A.weighted_attention_f64(q, k, v, w, 0.5)
    for m in range(4):
        rows = slice(m * blk, (m + 1) * blk)
        blocks = [int(x) for x in idx[0, m, :int(cnt[0, m])]]
        if not blocks:
            assert torch.equal(got[0, :, rows], torch.zeros(H, blk, hd, dtype=torch.float64))
            continue
        keys = torch.cat([torch.arange(j * blk, (j + 1) * blk) for j in blocks])
        s = q[0, :, rows].double() @ k[0][:, keys].double().transpose(-2, -1) * 0.5
        ref = torch.softmax(s, dim=-1) @ v[0][:, keys].double()
        assert torch.allclose(got[0, :, rows], ref, rtol=1e-10, atol=1e-12)


def test_prefill_forward_dense_window_is_causal_attention():
    """With a window covering the whole sequence the sparse mask is the causal
    mask, so the oracle's attention equals SDPA(is_causal=True)."""
    import __graft_entry__

    fsi = __graft_entry__.load_package()
    torch.manual_seed(0)
    m = fsi.FovealSparseAttention(hidden_size=64, num_heads=4, num_kv_heads=2, head_dim=16, page_size=8,
                                  local_window_blocks=8, use_additive_stream=False)
    x = torch.randn(2, 64, 64)
    idx = torch.zeros(2, 8, 8, dtype=torch.int32)
    cnt = torch.zeros(2, 8, dtype=torch.int32)
    out, teacher = A.prefill_forward(m, x, idx, cnt)
    with torch.no_grad():
        q = m.q_proj(x).view(2, 64, 4, 16).transpose(1, 2)
        k = m.k_proj(x).view(2, 64, 2, 16).transpose(1, 2).repeat_interleave(2, dim=1)
        v = m.v_proj(x).view(2, 64, 2, 16).transpose(1, 2).repeat_interleave(2, dim=1)
        att = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=1 / math.sqrt(16))
        ref = m.out_proj(att.transpose(1, 2).reshape(2, 64, 64))
    assert torch.allclose(out, ref, rtol=1e-4, atol=1e-5)
    # teacher mass: each anchor row is a distribution over the pages up to its own
    assert torch.allclose(teacher.sum(-1), torch.ones(2, 8), atol=1e-5)
    assert torch.all(teacher.triu(1) == 0)
    # anchor 0 sees only key 0, which lies in page 0
    assert torch.allclose(teacher[:, 0, 0], torch.ones(2))
