"""Pins of oracle.routing.tile_route (BlockwiseMatMul2D tile selection,
foveal_indexer/block_matmul.py:364-377) against the pure-Python brute force
and closed forms (CPU only)."""
import pytest
import torch

from oracle import brute
from oracle import routing as R


@pytest.mark.parametrize("T,top_p", [(16, 0.5), (37, 0.9), (100, 0.95), (256, 0.8)])
def test_tile_route_brute_force(T, top_p):
    g = torch.Generator().manual_seed(T)
    rows = 12
    scores = torch.randn(rows, T, generator=g, dtype=torch.float64) * 3
    out = R.tile_route(scores, top_p, base_tiles=0)
    for r in range(rows):
        sel = brute.tile_route_row(scores[r].tolist(), top_p)
        n = int(out["needed"][r])
        # margins: the oracle's sorted running mass must not sit within 1e-9 of top_p
        assert len(sel) == n
        assert out["order"][r, :n].tolist() == sel


def test_tile_route_closed_forms():
    # a single spike: one tile carries (almost) all the mass -> needed 1
    s = torch.zeros(1, 32)
    s[0, 7] = 40.0
    out = R.tile_route(s, 0.9, base_tiles=0)
    assert int(out["needed"][0]) == 1 and out["mask"][0].nonzero().flatten().tolist() == [7]
    # flat scores over 16 tiles, top_p 1/2: cum_k = (k+1)/16 exactly, 7 below -> needed 8
    out = R.tile_route(torch.zeros(1, 16), 0.5, base_tiles=0)
    assert int(out["needed"][0]) == 8
    assert out["mask"][0].nonzero().flatten().tolist() == list(range(8))  # equal p: tile order
    # top_p above the total mass: every tile (needed capped at T)
    out = R.tile_route(torch.randn(3, 20), 1.5, base_tiles=0)
    assert out["needed"].tolist() == [20, 20, 20] and bool(out["mask"].all())
    # base tiles always on; union over rows; one mask per row group
    s = torch.full((4, 10), -30.0)
    for r, t in enumerate([3, 5, 3, 9]):
        s[r, t] = 30.0
    out = R.tile_route(s, 0.9, base_tiles=2)
    assert out["mask"][0].nonzero().flatten().tolist() == [0, 1, 3, 5, 9]
    out = R.tile_route(s, 0.9, base_tiles=2, rows_per_group=2)
    assert out["mask"][0].nonzero().flatten().tolist() == [0, 1, 3, 5]
    assert out["mask"][1].nonzero().flatten().tolist() == [0, 1, 3, 9]
