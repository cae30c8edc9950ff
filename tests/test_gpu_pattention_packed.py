"""GPU parity of the packed-weight decode Pattention path (fsi_pattention_pack +
fsi_pattention_fwd_packed) against the CPU oracle, bf16 rel-L2 <= 2e-3 with the
oracle's rounding points, and its use by FovealPattentionMLP."""
import pytest
import torch

from oracle import pattention as P
from oracle import routing as R

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-3


def _weights(N_p, K, D_out, g, v_transposed):
    kg = (torch.randn(N_p, K, generator=g) * 0.03).bfloat16()
    ku = (torch.randn(N_p, K, generator=g) * 0.03).bfloat16()
    if v_transposed:
        v = (torch.randn(D_out, N_p, generator=g) * 0.03).bfloat16().t()  # down_proj storage
    else:
        v = (torch.randn(N_p, D_out, generator=g) * 0.03).bfloat16()
    return kg, ku, v


# M, K, N_p, D_out, block_n, active blocks (None = dense), V in down_proj storage
CASES = [
    (1, 256, 1024, 48, 64, 5, True),         # one token tile, one K chunk, padded channels
    (17, 512, 2048, 304, 32, 21, True),      # 32-wide blocks
    (40, 1024, 4096, 256, 64, 19, False),    # V row-major [N_p, D_out]
    (64, 4096, 4096, 208, 64, 32, True),     # 16 K chunks, 2048 channels
    (64, 2048, 16384, 512, 128, 40, True),   # 5120 channels: 32 steps per down wave
    (33, 256, 8192, 48, 64, 100, True),      # 6400 channels
    (48, 8192, 1024, 64, 64, 3, False),      # 32 K chunks
    (16, 512, 1024, 192, 64, None, True),    # dense: no block list
]


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(len(CASES))])
def test_packed_decode_parity(fsi, dev, case):
    M, K, N_p, D_out, block_n, n_act, vt = case
    print(f"[case] packed decode {case}", flush=True)
    g = torch.Generator().manual_seed(M * 13 + K + N_p)
    x = torch.randn(M, K, generator=g).bfloat16()
    kg, ku, v = _weights(N_p, K, D_out, g, vt)
    active = None if n_act is None else torch.randperm(N_p // block_n, generator=g)[:n_act].to(torch.int32)
    pk = fsi.pack_pattention_weights(kg.to(dev), ku.to(dev), v.to(dev), block_n)
    vc = v.contiguous()
    for rounding in ("eager", "fused", "fp32"):
        got = fsi.pattention_decode_packed(x.to(dev), pk, None if active is None else active.to(dev),
                                           rounding=rounding).cpu()
        if rounding == "fp32":
            ref = P.pattention_fp32_act(x, kg, vc, ku, active, "swiglu", block_n)
        else:
            blocks = torch.arange(N_p // block_n) if active is None else active
            ref = P.mlp_eval_forward(x, kg, ku, vc, blocks, block_n, fused=rounding == "fused")
        err = P.rel_l2(got, ref)
        assert got.shape == (M, D_out)
        assert err <= BF16_TOL, (rounding, err)


# prefill (>= 256 tokens): the 256 x 256 GEMMs over the packed tiles
PREFILL_CASES = [
    (256, 512, 2048, 304, 32, 21, True),      # 32-wide blocks, D_out not a multiple of 256
    (300, 1024, 4096, 256, 64, 19, False),    # V row-major [N_p, D_out], partial row tile
    (257, 256, 8192, 48, 64, 100, True),      # 6400 channels, one row past a tile
    (1024, 1024, 4096, 512, 64, None, True),  # dense: no block list
    (512, 2048, 16384, 640, 128, 40, True),   # 128-wide blocks
]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=[f"p{i}" for i in range(len(PREFILL_CASES))])
def test_packed_prefill_parity(fsi, dev, case):
    test_packed_decode_parity(fsi, dev, case)


def test_packed_prefill_bad_block_masked_and_reported(fsi, dev):
    from foveal_sparse_indexer_amd import _lib

    M, K, N_p, D_out, block_n = 300, 512, 1024, 256, 64
    g = torch.Generator().manual_seed(12)
    x = torch.randn(M, K, generator=g).bfloat16()
    kg, ku, v = _weights(N_p, K, D_out, g, True)
    pk = fsi.pack_pattention_weights(kg.to(dev), ku.to(dev), v.to(dev), block_n)
    _lib.error_word(dev).zero_()
    bad = torch.tensor([3, 99, 7, -1], dtype=torch.int32)
    got = fsi.pattention_decode_packed(x.to(dev), pk, bad.to(dev), rounding="fp32").cpu()
    ref = P.pattention_fp32_act(x, kg, v.contiguous(), ku, torch.tensor([3, 7]), "swiglu", block_n)
    assert P.rel_l2(got, ref) <= BF16_TOL
    assert int(_lib.error_word(dev)[0]) == _lib.FSI_ERR_INDEX_RANGE
    _lib.error_word(dev).zero_()


def test_packed_8b_decode_shape(fsi, dev):
    """C3a at full size: d_model 4096, 14336 parameter tokens, 8 base + 56 remote, batch 64."""
    print("[case] packed 8b decode shape", flush=True)
    D, N_p, base, remote = 4096, 14336, 8, 56
    g = torch.Generator().manual_seed(0)
    kg, ku, v = _weights(N_p, D, D, g, True)
    x = torch.randn(64, D, generator=g).bfloat16()
    active = torch.cat([torch.arange(base), torch.randperm(N_p // 64 - base, generator=g)[:remote] + base])
    active = active.to(torch.int32)
    pk = fsi.pack_pattention_weights(kg.to(dev), ku.to(dev), v.to(dev), 64)
    got = fsi.pattention_decode_packed(x.to(dev), pk, active.to(dev), rounding="fused").cpu()
    ref = P.mlp_eval_forward(x, kg, ku, v.contiguous(), active, 64, fused=True)
    err = P.rel_l2(got, ref)
    print(f"  rel_l2={err:.3e}", flush=True)
    assert err <= BF16_TOL


def test_packed_bad_block_masked_and_reported(fsi, dev):
    from foveal_sparse_indexer_amd import _lib

    M, K, N_p, D_out, block_n = 8, 512, 1024, 128, 64
    g = torch.Generator().manual_seed(11)
    x = torch.randn(M, K, generator=g).bfloat16()
    kg, ku, v = _weights(N_p, K, D_out, g, True)
    pk = fsi.pack_pattention_weights(kg.to(dev), ku.to(dev), v.to(dev), block_n)
    _lib.error_word(dev).zero_()
    bad = torch.tensor([3, 99, 7, -1], dtype=torch.int32)
    got = fsi.pattention_decode_packed(x.to(dev), pk, bad.to(dev), rounding="fp32").cpu()
    ref = P.pattention_fp32_act(x, kg, v.contiguous(), ku, torch.tensor([3, 7]), "swiglu", block_n)
    assert P.rel_l2(got, ref) <= BF16_TOL
    assert int(_lib.error_word(dev)[0]) == _lib.FSI_ERR_INDEX_RANGE
    _lib.error_word(dev).zero_()


def test_packed_rejects_unsupported_shapes(fsi, dev):
    g = torch.Generator().manual_seed(2)
    kg, ku, v = _weights(1024, 320, 64, g, True)  # K = 320 is not 256 x 2^k
    pk = fsi.pack_pattention_weights(kg.to(dev), ku.to(dev), v.to(dev), 64)
    with pytest.raises(ValueError):
        fsi.pattention_decode_packed(torch.randn(4, 320).bfloat16().to(dev), pk, None)
    kg, ku, v = _weights(1024, 256, 64, g, True)
    pk = fsi.pack_pattention_weights(kg.to(dev), ku.to(dev), v.to(dev), 64)
    with pytest.raises(ValueError):  # between the decode (<= 64) and prefill (>= 256) ranges
        fsi.pattention_decode_packed(torch.randn(65, 256).bfloat16().to(dev), pk, None)
    assert fsi.pattention_decode_packed(torch.randn(256, 256).bfloat16().to(dev), pk, None).shape == (256, 64)


def test_module_decode_uses_packed_weights_and_repacks(fsi, dev):
    """FovealPattentionMLP decode steps run on the packed copy, which follows
    in-place weight updates and parameter replacement."""
    torch.manual_seed(0)
    D, N_p, base, remote = 512, 2048, 2, 6
    m = fsi.FovealPattentionMLP(hidden_dim=D, intermediate_dim=N_p, base_blocks=base, remote_blocks=remote,
                                dtype=torch.bfloat16).to(dev).eval()
    x = torch.randn(8, 1, D).bfloat16()
    with torch.no_grad():
        out = m(x.to(dev))
        assert m._packed is not None
        first = m._packed
        cpu = {k: t.detach().cpu() for k, t in m.state_dict().items()}
        active = m._cached_active_blocks.cpu()
        assert torch.equal(active, R.mlp_pooled_route(x.reshape(-1, D), cpu["q_proj_16d.weight"],
                                                      cpu["block_keys_16d"], base, remote))
        ref = P.mlp_eval_forward(x.reshape(-1, D), cpu["k_gate"], cpu["k_up"], cpu["v"], active, 64, fused=True)
        assert P.rel_l2(out.cpu().reshape(-1, D), ref) <= BF16_TOL
        # same weights: the packed copy is reused
        m(x.to(dev))
        assert m._packed is first
        # in-place update of one weight: repacked, output follows
        m.k_up.mul_(-1.0)
        out2 = m(x.to(dev))
        assert m._packed is not first
        ref2 = P.mlp_eval_forward(x.reshape(-1, D), cpu["k_gate"], -cpu["k_up"], cpu["v"], active, 64, fused=True)
        assert P.rel_l2(out2.cpu().reshape(-1, D), ref2) <= BF16_TOL
        # the unpacked path gives the same result within the bf16 bar
        m.pack_decode_weights = False
        out3 = m(x.to(dev))
        assert P.rel_l2(out3.cpu().reshape(-1, D), ref2) <= BF16_TOL


def test_module_data_write_then_clear_cache(fsi, dev):
    """The reference idiom for new weights: write through .data (no version bump),
    then clear_cache(); the next eval forward routes again and reads the new
    weights (foveal_pattention.py:108-122, 310-322), on the packed path too."""
    torch.manual_seed(2)
    D, N_p, base, remote = 512, 2048, 2, 6
    m = fsi.FovealPattentionMLP(hidden_dim=D, intermediate_dim=N_p, base_blocks=base, remote_blocks=remote,
                                dtype=torch.bfloat16).to(dev).eval()
    x = torch.randn(8, 1, D).bfloat16()
    g = torch.Generator().manual_seed(3)
    with torch.no_grad():
        m(x.to(dev))
        assert m._packed is not None
        new = {n: (torch.randn(N_p, D, generator=g) * 0.03).bfloat16() for n in ("k_gate", "k_up", "v")}
        m.k_gate.data.copy_(new["k_gate"].to(dev))
        m.k_up.data.copy_(new["k_up"].to(dev))
        m.v.data = new["v"].to(dev)
        m.clear_cache()
        assert m._packed is None and m._cached_active_blocks is None
        out = m(x.to(dev))
        cpu = {k: t.detach().cpu() for k, t in m.state_dict().items()}
        active = m._cached_active_blocks.cpu()
        assert torch.equal(active, R.mlp_pooled_route(x.reshape(-1, D), cpu["q_proj_16d.weight"],
                                                      cpu["block_keys_16d"], base, remote))
        ref = P.mlp_eval_forward(x.reshape(-1, D), new["k_gate"], new["k_up"], new["v"], active, 64, fused=True)
        assert P.rel_l2(out.cpu().reshape(-1, D), ref) <= BF16_TOL


def test_packed_back_to_back_calls(fsi, dev):
    """Consecutive calls on one stream with different inputs and shapes reuse
    the workspace (partials and arrival counters): each result must match its
    own oracle."""
    D, N_p, D_out, block_n = 1024, 4096, 256, 64
    g = torch.Generator().manual_seed(21)
    kg, ku, v = _weights(N_p, D, D_out, g, True)
    pk = fsi.pack_pattention_weights(kg.to(dev), ku.to(dev), v.to(dev), block_n)
    cases = []
    for i, (M, n_act) in enumerate([(64, 40), (7, 12), (64, 40), (33, 64), (1, 3)]):
        x = torch.randn(M, D, generator=g).bfloat16()
        act = torch.randperm(N_p // block_n, generator=g)[:n_act].to(torch.int32)
        cases.append((x, act, fsi.pattention_decode_packed(x.to(dev), pk, act.to(dev), rounding="fused")))
    for x, act, got in cases:
        ref = P.mlp_eval_forward(x, kg, ku, v.contiguous(), act, block_n, fused=True)
        assert P.rel_l2(got.cpu(), ref) <= BF16_TOL


def test_unpack_inverts_pack(fsi, dev):
    """unpack_pattention_weights of the device pack: every weight back bit-exact,
    also for a block subset, V in either storage order."""
    g = torch.Generator().manual_seed(11)
    for vt in (True, False):
        kg, ku, v = _weights(1024, 512, 96, g, vt)
        pk = fsi.pack_pattention_weights(kg.to(dev), ku.to(dev), v.to(dev), 64)
        ukg, uku, uv = fsi.unpack_pattention_weights(pk)
        assert torch.equal(ukg.cpu(), kg) and torch.equal(uku.cpu(), ku) and torch.equal(uv.cpu(), v)
        blocks = torch.tensor([7, 0, 3])
        skg, sku, sv = fsi.unpack_pattention_weights(pk, blocks.to(dev))
        idx = (blocks.view(-1, 1) * 64 + torch.arange(64)).flatten()
        assert torch.equal(skg.cpu(), kg[idx]) and torch.equal(sku.cpu(), ku[idx]) and torch.equal(sv.cpu(), v[idx])


def test_module_pack_in_place_inference(fsi, dev):
    """release_unpacked_weights: the parameters' storage is freed, eval outputs
    (decode, 65..255 tokens in 64-token pieces, prefill) and input gradients stay
    those of the unreleased module, state_dict and the active-row caches return the
    original weights, training and fp32 input raise, unpack_weights restores the
    parameters bit-exactly."""
    torch.manual_seed(3)
    m = fsi.FovealPattentionMLP(hidden_dim=512, intermediate_dim=2048, block_size=64, base_blocks=2,
                                remote_blocks=6, dtype=torch.bfloat16).to(dev).eval()
    orig = {k: t.detach().clone() for k, t in m.state_dict().items()}
    v_stride = m.v.stride()
    xs = {M: (torch.randn(M, 512, device=dev) * 0.5).bfloat16() for M in (16, 100, 300)}
    m.set_active_blocks(torch.tensor([0, 1, 9, 17, 4, 30, 22, 11], dtype=torch.int32))
    with torch.no_grad():
        before = {M: m(x) for M, x in xs.items()}
    xg = xs[16].clone().requires_grad_()
    m(xg).float().square().sum().backward()
    dx_before = xg.grad.clone()

    freed = m.release_unpacked_weights()
    assert freed == 3 * 2048 * 512 * 2
    assert m.k_gate.numel() == 0 and m.k_up.numel() == 0 and m.v.numel() == 0
    with torch.no_grad():
        after = {M: m(x) for M, x in xs.items()}
    assert torch.equal(after[16], before[16]) and torch.equal(after[300], before[300])
    # 100 tokens ran pattention_forward before and 64-token packed pieces now
    assert P.rel_l2(after[100].cpu().float(), before[100].cpu().float()) <= BF16_TOL
    xg = xs[16].clone().requires_grad_()
    m(xg).float().square().sum().backward()
    assert torch.equal(xg.grad, dx_before)
    sd = m.state_dict()
    for k in ("k_gate", "k_up", "v"):
        assert torch.equal(sd[k], orig[k]), k
    idx = (m._cached_active_blocks.view(-1, 1).long().cpu() * 64 + torch.arange(64)).flatten()
    assert torch.equal(m._cached_kg.cpu(), orig["k_gate"].cpu()[idx])
    assert torch.equal(m._cached_v.cpu(), orig["v"].cpu()[idx])
    with pytest.raises(RuntimeError):
        m.train()(xs[16])
    m.eval()
    with pytest.raises(RuntimeError):
        m(xs[16].float())
    with pytest.raises(RuntimeError):
        m.reset_parameters()

    m.unpack_weights()
    assert m.v.stride() == v_stride
    for k in ("k_gate", "k_up", "v"):
        assert torch.equal(getattr(m, k).detach(), orig[k]), k
    with torch.no_grad():
        assert torch.equal(m(xs[16]), before[16])

    # a module move unpacks first
    m.release_unpacked_weights()
    m.to(dev)
    assert m.k_gate.shape == (2048, 512) and torch.equal(m.k_gate.detach(), orig["k_gate"])
    assert fsi.release_unpacked_weights(m) == freed
