"""BlockwiseMatMul2D tile routing (foveal_indexer/block_matmul.py:355-377) on the
HIP router (fsi_tile_route) against oracle.routing.tile_route given identical
scores: per-row needed counts and the union masks must agree exactly except at
documented near-ties (a running mass within 1e-5 of top_p at the boundary, or
equal probabilities straddling it, where torch.sort's order is unspecified)."""
import pytest
import torch

from oracle import routing as R

pytestmark = pytest.mark.gpu


def _check(got_mask, got_needed, ref, top_p, rows_per_group, base_tiles, tol=1e-5):
    """Returns the number of rows that were compared exactly."""
    needed, cum, sp, order = ref["needed"], ref["cumulative"].double(), ref["sorted_probs"].double(), ref["order"]
    rows, T = order.shape
    groups = ref["mask"].shape[0]
    certain = torch.zeros(groups, T, dtype=torch.bool)
    possible = torch.zeros(groups, T, dtype=torch.bool)
    certain[:, :base_tiles] = True
    possible[:, :base_tiles] = True
    exact_rows = 0
    for r in range(rows):
        n = int(needed[r])
        g = r // rows_per_group
        near = abs(float(cum[r, n - 1]) - top_p) <= tol or (n >= 2 and abs(float(cum[r, n - 2]) - top_p) <= tol)
        if n < T:
            v_last, v_next = float(sp[r, n - 1]), float(sp[r, n])
            near = near or abs(v_last - v_next) <= 1e-6 * max(v_last, 1e-30)
        if near:
            certain[g, order[r, : max(n - 2, 0)]] = True
            possible[g, order[r, : min(n + 1, T)]] = True
            # tiles tied with the boundary value may be taken in any order
            tied = (sp[r] - sp[r, n - 1]).abs() <= 1e-6 * max(float(sp[r, n - 1]), 1e-30)
            possible[g, order[r][tied]] = True
        else:
            exact_rows += 1
            assert int(got_needed[r]) == n, f"row {r}: needed {int(got_needed[r])} != {n}"
            certain[g, order[r, :n]] = True
            possible[g, order[r, :n]] = True
    got = got_mask.cpu()
    assert not (certain & ~got).any(), "a tile every ordering selects is missing"
    assert not (got & ~possible).any(), "a tile no ordering selects is set"
    return exact_rows


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,top_p,scale", [(16, 0.95, 2.0), (64, 0.9, 1.0), (100, 0.5, 3.0), (1024, 0.9, 4.0),
                                           (4096, 0.95, 6.0), (257, 0.99, 0.5)])
def test_tile_route_matches_oracle(fsi, dev, dtype, T, top_p, scale):
    g = torch.Generator().manual_seed(T + int(100 * top_p))
    rows, rpg, base = 96, 32, max(1, T // 4)
    scores = (torch.randn(rows, T, generator=g) * scale).to(dtype)
    mask, probs, needed = fsi.tile_route(scores.to(dev), top_p, base, rows_per_group=rpg)
    ref = R.tile_route(scores, top_p, base, rows_per_group=rpg)
    assert mask.shape == ref["mask"].shape and probs.dtype == dtype
    # bf16 rows: the running mass is compared after rounding to bf16, so a boundary
    # within one bf16 ulp of top_p is a near-tie (ATen accumulates bf16 cumsum in fp32)
    tol = 1e-5 if dtype == torch.float32 else 2 ** -8
    exact = _check(mask, needed.cpu(), ref, top_p, rpg, base, tol=tol)
    if dtype == torch.float32:
        assert exact >= rows * 3 // 4
    # probabilities: softmax in fp32, rounded to the row dtype
    ptol = 1e-6 if dtype == torch.float32 else 2 ** -8
    assert torch.allclose(probs.cpu().float(), ref["probs"].float(), rtol=ptol, atol=1e-7)


def test_tile_route_closed_forms(fsi, dev):
    # flat scores over 16 tiles, top_p 1/2: exactly 8 needed, taken in tile order
    mask, _, needed = fsi.tile_route(torch.zeros(3, 16, device=dev), 0.5, 0)
    assert needed.tolist() == [8, 8, 8] and mask[0].nonzero().flatten().tolist() == list(range(8))
    # top_p above the total: every tile; top_p <= 0: the argmax alone
    mask, _, needed = fsi.tile_route(torch.randn(2, 50, device=dev), 1.5, 0)
    assert needed.tolist() == [50, 50] and bool(mask.all())
    s = torch.randn(1, 40, device=dev)
    mask, _, needed = fsi.tile_route(s, 0.0, 0)
    assert needed.tolist() == [1] and mask[0].nonzero().flatten().tolist() == [int(s[0].argmax())]
    # no rows: only the base tiles
    mask, _, _ = fsi.tile_route(torch.empty(0, 12, device=dev), 0.9, 3)
    assert mask[0].nonzero().flatten().tolist() == [0, 1, 2]


def test_blockwise_matmul2d_route_matches_oracle(fsi, dev):
    """The module's routing against the oracle given the module's own scores, and
    its product against the masked dense matmul X (W o M)^T in fp64."""
    from oracle import blocksparse as BS

    torch.manual_seed(0)
    m = fsi.BlockwiseMatMul2D(256, 512, block_k=64, block_n=64, base_tiles_ratio=0.25, top_p=0.8)
    m = m.to(dev, torch.bfloat16)
    x = torch.randn(2, 16, 256, device=dev).bfloat16()
    with torch.no_grad():
        mask, probs, scores, _ = m.route_tiles(x)
        out, aux = m(x)
    flat = scores.reshape(-1, m.total_tiles)
    _, _, needed = fsi.tile_route(flat, 0.8, m.base_tiles)
    ref = R.tile_route(flat.cpu(), 0.8, m.base_tiles)
    _check(mask[None], needed.cpu(), ref, 0.8, flat.shape[0], m.base_tiles)
    assert aux["active_tiles"] == int(mask.sum())
    em = BS.expand_tile_mask(mask.cpu(), 512, 256, 64, 64)
    dense = x.double().cpu().reshape(-1, 256) @ (m.weight.double().cpu() * em).t()
    ctx = (probs.reshape(-1, m.total_tiles).double().cpu() @ m.tile_keys_and_values()[1].double().cpu())
    ref_out = dense + ctx @ m.out_proj.weight.double().cpu().t()
    err = (out.reshape(-1, 512).double().cpu() - ref_out).norm() / ref_out.norm()
    assert err <= 2e-2  # bf16 output, bf16 context projection
