"""Pins of the fused indexer-attention oracle (CPU only).

oracle.attention.sram_select (fp32 torch) against the pure-Python fp64 picker
oracle.brute.sram_pick_row on random rows with margins far above fp32 rounding,
and against hand-built known answers for each rule of triton_ops.py:164-182,219-245
(self block excluded, first index on ties, the mass gate applied before a pick
is added, the 1e-4 floor, non-attended rounds still adding their mass).
sram_attention_f64 against attention over explicitly concatenated key blocks."""
import math

import torch

from oracle import attention as A
from oracle import brute


def _q16_for_logits(logits):
    """q16 / k16 rows whose 16-D score (q . k / 4) for block 0 is logits[j]."""
    M = len(logits)
    q16 = torch.zeros(1, M, 16)
    k16 = torch.zeros(1, M, 16)
    q16[0, 0, 0] = 4.0
    for j, s in enumerate(logits):
        k16[0, j, 0] = s
    return q16, k16


def test_select_matches_brute_force_on_separated_rows():
    g = torch.Generator().manual_seed(0)
    checked = 0
    for M, R, top_p in [(4, 2, 0.8), (9, 3, 0.5), (16, 5, 0.9), (33, 4, 0.7), (7, 8, 0.99)]:
        q16 = torch.randn(3, M, 16, generator=g)
        k16 = torch.randn(3, M, 16, generator=g)
        picks, probs = A.sram_select(q16, k16, top_p, R)
        scores = (q16.double() @ k16.double().transpose(1, 2)) * 0.25
        for b in range(3):
            for m in range(M):
                p = probs[b, m].double()
                srt = p.sort(descending=True).values
                cum = srt.cumsum(0)
                gaps = (srt[:-1] - srt[1:]).abs()
                near = bool((gaps[:R] < 1e-5).any()) or bool(((cum[:R] - top_p).abs() < 1e-5).any()) \
                    or bool(((srt[:R] - 1e-4).abs() < 1e-7).any())
                if near:
                    continue
                want = brute.sram_pick_row(scores[b, m].tolist(), m, top_p, R)
                assert picks[b, m].tolist() == want, (M, b, m)
                checked += 1
    assert checked > 150


def test_select_known_answers():
    # block 0 sees the others at 0.5 / 0.3 / 0.2 (the 1e-6 pad shifts them by ~1e-6)
    q16, k16 = _q16_for_logits([7.0, math.log(0.5), math.log(0.3), math.log(0.2)])
    picks, probs = A.sram_select(q16, k16, top_p=0.75, max_remote=4)
    assert probs[0, 0, 0] == 0.0
    assert abs(float(probs[0, 0, 1]) - 0.5) < 1e-5
    # 0.5 then 0.3 (mass 0.5 < 0.75); the third sees mass 0.8 >= 0.75; the fourth
    # round finds only the self block (probability 0) left
    assert picks[0, 0].tolist() == [1, 2, -1, -1]
    # with top_p 0.8 the mass before the third pick is 0.8 / (1 + 1e-6) < 0.8
    assert A.sram_select(q16, k16, top_p=0.8, max_remote=3)[0][0, 0].tolist() == [1, 2, 3]
    # ties go to the lower index; the self block's own score does not matter
    q16, k16 = _q16_for_logits([50.0, 1.0, 2.0, 2.0, 1.0])
    assert A.sram_select(q16, k16, top_p=1.0, max_remote=2)[0][0, 0].tolist() == [2, 3]
    # the 1e-4 floor: a pick below it is not attended though the mass allows it,
    # and a later round (its mass added) is gated as well
    q16, k16 = _q16_for_logits([0.0, 0.0, -10.0, -30.0])
    picks, probs = A.sram_select(q16, k16, top_p=1.0, max_remote=3)
    assert float(probs[0, 0, 2]) < 1e-4
    assert picks[0, 0].tolist() == [1, -1, -1]
    # a single block: nothing to pick
    picks, _ = A.sram_select(torch.randn(2, 1, 16), torch.randn(2, 1, 16), 0.8, 2)
    assert picks.eq(-1).all()


def test_attention_matches_concatenated_blocks():
    g = torch.Generator().manual_seed(3)
    B, H, N, D, bs = 2, 3, 40, 8, 8
    q, k, v = (torch.randn(B, H, N, D, generator=g) for _ in range(3))
    picks = torch.tensor([[[3, -1], [-1, -1], [0, 4], [2, 1], [-1, 0]],
                          [[1, 2], [4, -1], [-1, -1], [0, -1], [3, 2]]])
    got = A.sram_attention_f64(q, k, v, picks, bs, 0.3)
    for b in range(B):
        for m in range(N // bs):
            blocks = [m] + [p for p in picks[b, m].tolist() if p >= 0]
            keys = torch.cat([k[b, :, j * bs:(j + 1) * bs] for j in blocks], dim=1).double()
            vals = torch.cat([v[b, :, j * bs:(j + 1) * bs] for j in blocks], dim=1).double()
            qq = q[b, :, m * bs:(m + 1) * bs].double()
            want = torch.softmax(qq @ keys.transpose(-1, -2) * 0.3, dim=-1) @ vals
            assert torch.allclose(got[b, :, m * bs:(m + 1) * bs], want, atol=1e-12)
