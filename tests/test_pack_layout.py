"""CPU check of unpack_pattention_weights (the torch permutation that inverts the
packed decode layout) against a packed buffer written element by element from
the index formulas of pack_rows_kernel and pack_down_kernel
(csrc/pattention_packed.hip)."""
import numpy as np
import torch


def _pack_reference(kg, ku, v, bn):
    """Byte buffer in the fsi_pattention_pack layout, built with explicit index
    arithmetic: gate / up element i of tile (ct, s), lane l = 16 q + r, is
    W[16 ct + r][32 s + 8 q + e]; down tile (b, dt, cl) holds
    V[b bn + 32 cl + 8 q + e][16 dt + r]."""
    N_p, K = kg.shape
    D = v.shape[1]
    S, DT, CB = K // 32, D // 16, bn // 32
    mat = (2 * N_p * K + 255) // 256 * 256
    total = 2 * mat + (2 * N_p * D + 255) // 256 * 256
    out = np.zeros(total // 2, dtype=np.uint16)
    i = np.arange(N_p // 16 * S * 64)
    lane, ts = i & 63, i >> 6
    s, ct = ts % S, ts // S
    r, q = lane & 15, lane >> 4
    for w, base in ((kg, 0), (ku, mat // 2)):
        wb = w.view(torch.int16).numpy().view(np.uint16)
        for e in range(8):
            out[base + i * 8 + e] = wb[16 * ct + r, 32 * s + 8 * q + e]
    j = np.arange(N_p // bn * DT * CB * 64)
    lane, rest = j & 63, j >> 6
    cl, rest = rest % CB, rest // CB
    dt, b = rest % DT, rest // DT
    r, q = lane & 15, lane >> 4
    vb = v.contiguous().view(torch.int16).numpy().view(np.uint16)
    for e in range(8):
        out[mat + j * 8 + e] = vb[b * bn + 32 * cl + 8 * q + e, 16 * dt + r]
    return torch.from_numpy(out.view(np.uint8).copy())


def test_unpack_matches_pack_index_formulas(fsi):
    g = torch.Generator().manual_seed(0)
    N_p, K, D, bn = 256, 96, 48, 64
    kg, ku, v = (torch.randn(a, b, generator=g).bfloat16() for a, b in ((N_p, K), (N_p, K), (N_p, D)))
    buf = _pack_reference(kg, ku, v, bn)
    pk = fsi.PackedPattentionWeights(buf, N_p, K, D, bn, key=None)
    ukg, uku, uv = fsi.unpack_pattention_weights(pk)
    assert torch.equal(ukg, kg) and torch.equal(uku, ku) and torch.equal(uv, v)
    blocks = torch.tensor([3, 1])
    skg, sku, sv = fsi.unpack_pattention_weights(pk, blocks)
    idx = (blocks.view(-1, 1) * bn + torch.arange(bn)).flatten()
    assert torch.equal(skg, kg[idx]) and torch.equal(sku, ku[idx]) and torch.equal(sv, v[idx])
