"""Parity at the exact configurations the benchmark times (BASELINE.json configs
C1-C5, built by the same constructors bench.py uses), against the CPU oracle:

  C1  fp32 FovealPattentionMLP, D 512, 2048 parameter tokens, base 2, K_max 8,
      x 4 x 128 (foveal_pattention.py:264-352): routing bit-exact, output vs
      fp64 within 1e-6 rel-L2 (the fp32 kernels sum each 16-wide K tile into a
      fresh partial, ~2.4e-7 from the exact value; CPU fp32 GEMMs sit at ~5e-7);
  C3b 8B prefill, 4096 tokens x 4096, 64 of 224 blocks, packed weights
      (foveal_pattention.py:278-288) vs the oracle eval forward, bf16 rel-L2 <= 2e-3;
  C4  32 sequences x 131072 context, 32 routed pages each, 16 GiB paged pool
      (attention.py:339-367): routing vs the oracle, attention of 3 sequences vs
      fp64 over supports gathered on the device;
  C5  4096 x 8192 x 8192, 128 x 128 tiles, per-row-group masks at 10/25/50%
      (block_matmul.py:381-392): 2 row groups per density vs fp64.
"""
import math

import pytest
import torch

import bench
from oracle import attention as A
from oracle import pattention as P
from oracle import routing as R
from route_check import check_rows, tolerances

pytestmark = pytest.mark.gpu


def test_c1_fp32_module_exact_config(fsi, dev):
    print("[case] C1 fp32 module", flush=True)
    g = torch.Generator().manual_seed(0)
    D, N_p, base, kmax, kmin, top_p = 512, 2048, 2, 8, 2, 0.9
    kg = torch.randn(N_p, D, generator=g) * 0.02
    ku = torch.randn(N_p, D, generator=g) * 0.02
    v = torch.randn(N_p, D, generator=g) * 0.02
    qmat = torch.linalg.qr(torch.randn(D, 16, generator=g))[0]
    keys = torch.randn(N_p // 64, 16, generator=g) * 0.25
    x = torch.randn(4, 128, D, generator=g)
    m = fsi.FovealPattentionMLP(hidden_dim=D, intermediate_dim=N_p, block_size=64, base_blocks=base,
                                remote_blocks=kmax, temperature=1.0, dtype=torch.float32)
    with torch.no_grad():
        m.k_gate.copy_(kg)
        m.k_up.copy_(ku)
        m.v.copy_(v)
        m.q_proj_16d.weight.copy_(qmat.t())
        m.block_keys_16d.copy_(keys)
    m = m.to(dev).eval()
    with torch.no_grad():
        out = m(x.to(dev)).cpu()
    active = m._cached_active_blocks.cpu()
    x2 = x.reshape(-1, D)
    ref_active = R.mlp_pooled_route(x2, qmat.t().contiguous(), keys, base, kmax)
    assert torch.equal(active, ref_active), (active.tolist(), ref_active.tolist())
    # The top-p form of the same routing (select_blocks on the pooled row, local = base blocks):
    s = R.mlp_router_scores(x2, qmat.t().contiguous(), keys).float()[None, None]
    kw = dict(causal=False, local_window_blocks=base, top_p=top_p, min_remote_blocks=kmin, max_remote_blocks=kmax,
              remote_capacity=kmax)
    got = fsi.select_blocks(s.to(dev), **kw)
    ref = R.select_route(s, **kw)
    remote = R.route_masks(1, N_p // 64, False, base)[2]
    assert check_rows(got.remote_indices, got.remote_counts, ref, remote, *tolerances(torch.float32)) == []
    assert int(got.remote_counts[0, 0]) == kmax  # K_max binds at this config (flat cosine-free scores)
    assert sorted(got.remote_indices[0, 0].tolist()) == sorted((ref_active[base:]).tolist())
    mask = torch.zeros(N_p, dtype=torch.bool)
    mask[P.channel_index(active, 64)] = True
    exact = P.dense_swiglu_f64(x2, kg, ku, v, mask)
    err = P.rel_l2(out.reshape(-1, D), exact)
    print(f"C1 fp32 rel-L2 vs fp64: {err:.3e}", flush=True)
    assert err <= 1e-6


def test_c2_routing_full_launch(fsi, dev):
    """The timed C2 launch exactly (bench.c2_inputs, 8192 queries x 4096 keys,
    top-p 0.9, K_min 4, K_max 64, capacity 64) against the oracle's
    select_blocks on fp32 cosine scores (core.py:46-160, 254-266): every slot and
    count, tie-tolerant only where the reference order is itself undetermined,
    and the selected mass."""
    print("[case] C2 full launch 8192 x 4096", flush=True)
    Q, N, KMIN, KMAX, CAP, TOP_P = 8192, 4096, 4, 64, 64, 0.9
    q, k = bench.c2_inputs(Q, N, dev)
    with torch.no_grad():
        idx, cnt, mass = fsi.score_and_route(q, k, causal=False, top_p=TOP_P, min_remote_blocks=KMIN,
                                             max_remote_blocks=KMAX, remote_capacity=CAP, return_mass=True)
    s = R.cosine_scores_f32(q.cpu()[None], k.cpu()[None])
    ora = R.select_route(s, causal=False, top_p=TOP_P, min_remote_blocks=KMIN, max_remote_blocks=KMAX,
                         remote_capacity=CAP)
    del s
    remote = torch.ones(Q, N, dtype=torch.bool)
    bad = check_rows(idx, cnt, ora, remote, *tolerances(torch.float32), max_report=10)
    assert not bad, bad
    oc = ora["remote_counts"][0].long()
    same = cnt.cpu()[0].long() == oc
    print(f"C2: {int(same.sum())} of {Q} counts identical, mean count {float(oc.float().mean()):.2f}", flush=True)
    assert int(same.sum()) >= Q - 8  # count differences only at boundary near-ties (checked above)
    cm = ora["cumulative"][0]
    ref_mass = torch.where(oc > 0, cm.gather(1, (oc - 1).clamp_min(0)[:, None])[:, 0], torch.zeros(Q))
    assert torch.allclose(mass.cpu()[0][same], ref_mass[same].float(), atol=2e-6)


def test_c3b_prefill_full_size(fsi, dev):
    print("[case] C3b prefill 4096 tokens", flush=True)
    layers = bench.make_layers(fsi, 1, dev)
    m = layers[0]
    gx = torch.Generator(device=dev).manual_seed(1)
    torch.randn(bench.DECODE_BATCH, 1, bench.D_MODEL, device=dev, generator=gx)  # bench draws x_dec first
    x_pre = torch.randn(1, bench.PREFILL_TOKENS, bench.D_MODEL, device=dev, generator=gx).bfloat16()
    with torch.no_grad():
        out = m(x_pre)
    active = m._cached_active_blocks.cpu()
    assert active.numel() == bench.BASE + bench.REMOTE and m._packed is not None  # packed prefill path
    x2 = x_pre.reshape(-1, bench.D_MODEL).cpu()
    ref = P.mlp_eval_forward(x2, m.k_gate.detach().cpu(), m.k_up.detach().cpu(), m.v.detach().cpu(), active, 64,
                             fused=True)
    err = P.rel_l2(out.reshape(-1, bench.D_MODEL).cpu(), ref)
    print(f"C3b rel-L2: {err:.3e}", flush=True)
    assert err <= 2e-3


def test_c4_decode_attention_full_size(fsi, dev):
    print("[case] C4 decode attention 32 x 131072", flush=True)
    c = bench.C4
    cache, q, qi = bench.c4_inputs(fsi, dev)
    B, CTX, PAGE, W = c["B"], c["CTX"], c["PAGE"], c["W"]
    pos = CTX - 1
    scale = 1.0 / math.sqrt(c["HD"])
    with torch.no_grad():
        pages, counts = fsi.decode_route(qi, cache.kp_cache, None, pos=pos, page_size=PAGE, local_window=W,
                                         completed_pages=CTX // PAGE, top_p=c["TOP_P"], min_remote_blocks=0,
                                         max_remote_blocks=c["KMAX"])
        out = fsi.decode_attention(q, cache, pos=pos, window=W, remote_pages=pages, remote_counts=counts,
                                   scale=scale).cpu()
    ref_r = R.decode_route(qi.cpu()[:, None], cache.kp_cache.cpu(), pos, PAGE, W, CTX // PAGE, c["TOP_P"], 0,
                           c["KMAX"])
    cnt = counts.cpu().tolist()
    assert cnt == [len(p) for p in ref_r["pages"]] and min(cnt) == c["KMAX"]  # K_max binds: 32 pages each
    for b in range(B):
        assert sorted(pages[b, :cnt[b]].tolist()) == sorted(ref_r["pages"][b])
    for b in (0, 13, B - 1):
        sel = pages[b, :cnt[b]].tolist()
        toks = torch.tensor(A.support_tokens(pos, W, sel, PAGE), device=dev)
        kd, vd = cache.to_dense(CTX, batch=slice(b, b + 1))
        ks, vs = kd[:, :, toks].cpu(), vd[:, :, toks].cpu()  # (1, Hkv, 3072, hd): the support only
        del kd, vd
        n = ks.shape[2]
        ref = A.decode_attention_f64(q[b:b + 1].cpu().float(), ks, vs, n - 1, n, [[]], PAGE, scale)
        err = P.rel_l2(out[b:b + 1].float(), ref.float())
        print(f"C4 seq {b} support {n} rel-L2 {err:.3e}", flush=True)
        assert n == W + PAGE * c["KMAX"] and err <= 2e-3
    # the fused step the bench times: same pages, attention within bf16 summation-order noise
    with torch.no_grad():
        out2, pages2, counts2 = fsi.decode_step_attention(q, qi, cache, pos=pos, window=W,
                                                          completed_pages=CTX // PAGE, top_p=c["TOP_P"],
                                                          min_remote_blocks=0, max_remote_blocks=c["KMAX"],
                                                          scale=scale)
    assert torch.equal(pages2.cpu(), pages.cpu()) and torch.equal(counts2.cpu(), counts.cpu())
    assert P.rel_l2(out2.cpu().float(), out.float()) <= 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prefill_attention_16k_sampled_blocks(fsi, dev, dtype):
    """The timed prefill-attention workload exactly (bench.prefill_attn_inputs:
    16384 tokens, 32 / 8 heads, hd 128, window 1024, <= 32 routed pages, output
    through the same strided view; bf16, and the bench's fp32 leg on the same
    inputs): sampled query blocks, including the first ones, the first with a
    full window, and the last (window and 32 far pages all live), against fp64
    attention under the oracle's sparse_mask (attention.py:148-218), each
    block's keys gathered on the host.  Bars: bf16 2e-3, fp32 1e-5."""
    print(f"[case] prefill attention 16K sampled blocks {dtype}", flush=True)
    c = bench.PREFILL_ATTN
    B, HQ, HKV, HD, T, PAGE, W = c["B"], c["HQ"], c["HKV"], c["HD"], c["T"], c["PAGE"], c["WB"] * c["PAGE"]
    q, k, v, lists, counts = bench.prefill_attn_inputs(fsi, dev)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    tol = 2e-3 if dtype == torch.bfloat16 else 1e-5
    scale = 1.0 / HD ** 0.5
    out = torch.empty(B, T, HQ, HD, dtype=dtype, device=dev)
    with torch.no_grad():
        fsi.sparse_attention(q, k, v, lists, counts, block=PAGE, mode=0, window=W, scale=scale,
                             out=out.transpose(1, 2))
    Qb = T // PAGE
    cnt = counts.cpu()
    assert int(cnt[0, Qb - 1]) == c["KMAX"]  # the last block attends 32 far pages beside its window
    mask = A.sparse_mask(B, T, W, PAGE, lists.cpu(), cnt)  # (1, T, T) bool
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    oc = out.transpose(1, 2).cpu()
    for qb in (0, 1, 15, 16, 17, 100, 200, Qb - 2, Qb - 1):
        q0, q1 = qb * PAGE, (qb + 1) * PAGE
        rows = mask[:, q0:q1]                       # (1, 64, T)
        keys = torch.nonzero(rows[0].any(0))[:, 0]  # the block's key support
        ref = A.weighted_attention_f64(qc[:, :, q0:q1], kc[:, :, keys], vc[:, :, keys], rows[:, :, keys], scale)
        err = P.rel_l2(oc[:, :, q0:q1].float(), ref.float())
        print(f"prefill 16K block {qb}: {keys.numel()} keys, {int(cnt[0, qb])} pages, rel-L2 {err:.3e}", flush=True)
        assert err <= tol


@pytest.mark.parametrize("density", bench.C5["DENSITIES"])
def test_c5_block_sparse_full_size(fsi, dev, density):
    print(f"[case] C5 density {density}", flush=True)
    x, w, scores = bench.c5_inputs(dev)
    mask, n_tiles = bench.c5_mask(scores, density)
    T = bench.C5["T"]
    with torch.no_grad():
        out = fsi.blockwise_matmul(x, w, mask, T, T, rows_per_group=T)
    from oracle import blocksparse as BS

    N, K = w.shape
    wc = w.cpu().double()
    for grp in (0, 21):
        em = BS.expand_tile_mask(mask[grp].cpu(), N, K, T, T)
        ref = x[grp * T:(grp + 1) * T].cpu().double() @ (wc * em).t()
        err = P.rel_l2(out[grp * T:(grp + 1) * T].cpu().float(), ref.float())
        print(f"C5 d={density} group {grp}: {n_tiles} tiles rel-L2 {err:.3e}", flush=True)
        assert err <= 2e-3
