"""Pins of the block-sparse oracle (CPU only): brute-force loops and the dense
special cases."""
import torch
import torch.nn.functional as F

from oracle import blocksparse as BS


def test_block_sparse_linear_brute_force_and_dense():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 8, generator=g)
    w = torch.randn(12, 8, generator=g)
    b = torch.randn(12, generator=g)
    out = BS.block_sparse_linear_f64(x, w, b, [2, 0], 4)
    for m in range(3):
        for n in range(12):
            ref = 0.0 if n // 4 == 1 else sum(float(x[m, k]) * float(w[n, k]) for k in range(8)) + float(b[n])
            assert abs(float(out[m, n]) - ref) < 1e-9
    dense = BS.block_sparse_linear_f64(x, w, b, [0, 1, 2], 4)
    assert torch.allclose(dense, F.linear(x.double(), w.double(), b.double()))


def test_blockwise_matmul_tile_ids_and_groups():
    g = torch.Generator().manual_seed(1)
    M, K, N, bk, bn = 4, 6, 4, 3, 2  # 2 k blocks x 2 n blocks, tile id = k_b * 2 + n_b
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g)
    mask = torch.tensor([True, False, False, True])  # (k0, n0) and (k1, n1)
    out = BS.blockwise_matmul_f64(x, w, mask, bk, bn, rows_per_group=M)
    ref = torch.zeros(M, N, dtype=torch.float64)
    ref[:, 0:2] = x[:, 0:3].double() @ w[0:2, 0:3].double().t()
    ref[:, 2:4] = x[:, 3:6].double() @ w[2:4, 3:6].double().t()
    assert torch.allclose(out, ref)
    masks = torch.stack([mask, torch.ones(4, dtype=torch.bool)])
    out2 = BS.blockwise_matmul_f64(x, w, masks, bk, bn, rows_per_group=2)
    assert torch.allclose(out2[:2], ref[:2]) and torch.allclose(out2[2:], x[2:].double() @ w.double().t())


def test_eval_active_blocks_closed_forms():
    s = torch.full((1, 1, 6), -30.0)
    s[0, 0, 4] = 10.0  # one dominant remote block
    assert BS.eval_active_blocks(s, 2, 0.9, 3, 6).tolist() == [0, 1, 4]
    flat = torch.zeros(2, 3, 10)
    act = BS.eval_active_blocks(flat, 2, 0.99, 3, 10)  # flat scores: K_max blocks, lowest ids by sort order
    assert act[:2].tolist() == [0, 1] and act.numel() == 2 + 3
