"""Host logic of the reverse sweep's wrapper (``hsn_amd.state_sweep``) on the CPU: the message
graph by source that the sweep's scatter to message sources reads, and the cache that decides
when it is rebuilt."""

from __future__ import annotations

import pytest
import torch

from hsn_amd import state_sweep as SS


def _brute(pad_src: torch.Tensor, pad_mask: torch.Tensor):
    """Per source, its out-edges as (target, flat index) in ascending flat index."""
    N, D = pad_src.shape
    rows = {n: [] for n in range(N)}
    for t in range(N):
        for s in range(D):
            if bool(pad_mask[t, s]):
                rows[int(pad_src[t, s])].append((t, t * D + s))
    return rows


@pytest.mark.parametrize("seed", range(6))
def test_out_adjacency_matches_brute_force(seed):
    g = torch.Generator().manual_seed(seed)
    N = 3 + 7 * seed
    D = 1 + seed % 5
    pad_src = torch.randint(0, N, (N, D), generator=g)
    pad_mask = torch.rand(N, D, generator=g) < 0.25 + 0.12 * seed
    out_tgt, out_edge = SS.out_adjacency(pad_src, pad_mask)
    rows = _brute(pad_src, pad_mask)
    d_out = max(1, max(len(r) for r in rows.values()))
    assert out_tgt.shape == (N, d_out) and out_edge.shape == (N, d_out)
    assert out_tgt.dtype == torch.int64 and out_edge.dtype == torch.int64
    for n in range(N):
        want = rows[n] + [(-1, 0)] * (d_out - len(rows[n]))  # padding: target -1, edge 0
        got = [(int(out_tgt[n, j]), int(out_edge[n, j])) for j in range(d_out)]
        assert got == want, n


def test_out_adjacency_empty_and_single_source():
    pad_src = torch.zeros(4, 3, dtype=torch.int64)
    out_tgt, out_edge = SS.out_adjacency(pad_src, torch.zeros(4, 3, dtype=torch.bool))
    assert out_tgt.shape == (4, 1) and bool((out_tgt == -1).all()) and bool((out_edge == 0).all())
    # every edge from cell 0: one row of 12, in flat order
    out_tgt, out_edge = SS.out_adjacency(pad_src, torch.ones(4, 3, dtype=torch.bool))
    assert out_edge[0].tolist() == list(range(12))
    assert out_tgt[0].tolist() == [f // 3 for f in range(12)]
    assert bool((out_tgt[1:] == -1).all())


@pytest.mark.parametrize("bad", [-1, 5])
def test_out_adjacency_rejects_a_source_outside_the_cells(bad):
    pad_src = torch.zeros(5, 2, dtype=torch.int64)
    pad_src[3, 1] = bad
    mask = torch.ones(5, 2, dtype=torch.bool)
    with pytest.raises(ValueError, match="outside"):
        SS.out_adjacency(pad_src, mask)
    mask[3, 1] = False  # a padded slot's source is not read
    SS.out_adjacency(pad_src, mask)


def test_graph_token_sees_in_place_changes_of_either_tensor():
    pad_src = torch.zeros(4, 2, dtype=torch.int64)
    pad_mask = torch.ones(4, 2, dtype=torch.bool)
    token = SS._graph_token(pad_src, pad_mask)
    assert SS._same_graph(token, pad_src, pad_mask)
    pad_mask[0, 0] = False
    assert not SS._same_graph(token, pad_src, pad_mask)
    token = SS._graph_token(pad_src, pad_mask)
    pad_src[1, 1] = 2
    assert not SS._same_graph(token, pad_src, pad_mask)
    assert not SS._same_graph(SS._graph_token(pad_src, pad_mask), pad_src.clone(), pad_mask)
    assert not SS._same_graph(None, pad_src, pad_mask)
