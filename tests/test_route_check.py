"""The tie-tolerant routing comparator accepts the oracle against itself and
rejects planted mistakes (CPU only)."""
import torch

from oracle import routing as R
from route_check import check_rows


def _case():
    g = torch.Generator().manual_seed(0)
    s = torch.randn(2, 6, 40, generator=g) * 3
    kw = dict(causal=False, local_window_blocks=2, top_p=0.8, min_remote_blocks=1, max_remote_blocks=8,
              remote_capacity=10)
    ora = R.select_route(s, **kw)
    _, _, remote = R.route_masks(6, 40, False, 2)
    return ora, remote


def test_oracle_against_itself():
    ora, remote = _case()
    assert check_rows(ora["remote_indices"], ora["remote_counts"], ora, remote, 1e-6, 1e-5) == []


def test_planted_swap_is_caught():
    ora, remote = _case()
    idx = ora["remote_indices"].clone()
    idx[0, 1, [0, 3]] = idx[0, 1, [3, 0]]
    bad = check_rows(idx, ora["remote_counts"], ora, remote, 1e-6, 1e-5)
    assert bad and "slot 0" in bad[0]


def test_planted_count_error_is_caught():
    ora, remote = _case()
    cnt = ora["remote_counts"].clone()
    cnt[1, 2] += 1
    bad = check_rows(ora["remote_indices"], cnt, ora, remote, 1e-6, 1e-5)
    assert bad and "count" in bad[0]


def test_planted_duplicate_and_padding_are_caught():
    ora, remote = _case()
    idx = ora["remote_indices"].clone()
    idx[1, 0, 1] = idx[1, 0, 0]
    assert check_rows(idx, ora["remote_counts"], ora, remote, 1e-6, 1e-5)
    s = torch.randn(1, 1, 3)
    o2 = R.select_route(s, causal=False, top_p=0.9, max_remote_blocks=3, remote_capacity=5)
    rem = torch.ones(1, 3, dtype=torch.bool)
    idx2 = o2["remote_indices"].clone()
    idx2[0, 0, 4] = 1
    assert check_rows(idx2, o2["remote_counts"], o2, rem, 1e-6, 1e-5)


def test_exact_ties_are_accepted_in_any_order():
    s = torch.zeros(1, 1, 6)
    ora = R.select_route(s, causal=False, top_p=0.5, max_remote_blocks=6, remote_capacity=6)
    rem = torch.ones(1, 6, dtype=torch.bool)
    idx = torch.tensor([[[5, 4, 3, 2, 1, 0]]], dtype=torch.int32)
    assert check_rows(idx, ora["remote_counts"], ora, rem, 1e-6, 1e-5) == []
