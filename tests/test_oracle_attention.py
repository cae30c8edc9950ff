"""Pins of the decode-attention oracle (CPU only): closed forms and agreement
with torch's SDPA in fp64 on an explicitly gathered support."""
import torch
import torch.nn.functional as F

from oracle import attention as A


def test_support_tokens_layout():
    # local window first, then each selected page; page 2's tokens before the window start are excluded
    toks = A.support_tokens(pos=200, window=64, pages=[0, 1], page_size=64)
    assert toks[:64] == list(range(137, 201))
    assert toks[64:] == list(range(0, 128))
    assert A.support_tokens(pos=5, window=64, pages=[], page_size=64) == list(range(0, 6))


def test_single_token_support_returns_its_value():
    q = torch.randn(1, 2, 8)
    k = torch.randn(1, 1, 4, 8)
    v = torch.randn(1, 1, 4, 8)
    out = A.decode_attention_f64(q, k, v, pos=0, window=1, pages=[[]], page_size=64, scale=0.3)
    assert torch.allclose(out[0, 0], v[0, 0, 0].double()) and torch.allclose(out[0, 1], v[0, 0, 0].double())


def test_equal_scores_average_the_support():
    q = torch.randn(1, 1, 8)
    k = torch.zeros(1, 1, 130, 8)
    v = torch.randn(1, 1, 130, 8)
    out = A.decode_attention_f64(q, k, v, pos=129, window=2, pages=[[0]], page_size=64, scale=1.0)
    toks = [128, 129] + list(range(64))
    assert torch.allclose(out[0, 0], v[0, 0, toks].double().mean(0))


def test_matches_sdpa_with_gqa():
    g = torch.Generator().manual_seed(0)
    B, Hq, Hkv, S, hd = 2, 4, 2, 256, 16
    q = torch.randn(B, Hq, hd, generator=g)
    k = torch.randn(B, Hkv, S, hd, generator=g)
    v = torch.randn(B, Hkv, S, hd, generator=g)
    pages = [[0, 2], [1]]
    out = A.decode_attention_f64(q, k, v, pos=[230, 250], window=40, pages=pages, page_size=64, scale=0.25)
    for b, pos in enumerate([230, 250]):
        toks = A.support_tokens(pos, 40, pages[b], 64)
        kk = k[b][:, toks].double().repeat_interleave(2, dim=0)
        vv = v[b][:, toks].double().repeat_interleave(2, dim=0)
        ref = F.scaled_dot_product_attention(q[b][:, None].double(), kk, vv, scale=0.25)[:, 0]
        assert torch.allclose(out[b], ref, atol=1e-12)


def test_decode_step_oracle_page_pooling_brute_force():
    """After a full page the oracle's page key is normalize(mean of the page's
    rms-normed index keys) in fp32 and its page value the mean of the index
    values (attention.py:84-91), checked against a plain fp64 recomputation."""
    import math

    import __graft_entry__

    fsi = __graft_entry__.load_package()  # module classes only; no GPU work
    torch.manual_seed(0)
    m = fsi.FovealSparseAttention(hidden_size=32, num_heads=2, num_kv_heads=1, head_dim=64, page_size=64,
                                  local_window_blocks=1, max_remote_pages=1, remote_capacity=1)
    ora = A.DecodeStepOracle(m, batch=1, max_seq_len=128)
    xs = torch.randn(64, 1, 1, 32)
    kis, vis = [], []
    for t in range(64):
        ora.step(xs[t])
        with torch.no_grad():
            kis.append(F.rms_norm(m.indexer.k_proj(xs[t]), (16,))[0, 0].double())
            vis.append(m.indexer.v_proj(xs[t])[0, 0].double())
    km = sum(kis) / 64
    assert ora.completed == 1
    assert torch.allclose(ora.kp[0, 0].double(), km / km.norm(), atol=1e-6)
    assert torch.allclose(ora.vp[0, 0].double(), sum(vis) / 64, atol=1e-6)
    assert math.isclose(float(ora.kp[0, 0].norm()), 1.0, rel_tol=1e-6)
