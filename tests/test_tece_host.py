"""Host-side bookkeeping of the TECE path (CPU): receiver chunking of the
edge list and the sub-CSR of a chunk."""

import torch

from tace_amd import ops
from tace_amd.tece import receiver_chunks, sub_plan


def _plan(deg):
    dst = torch.repeat_interleave(torch.arange(len(deg)), deg)
    src = torch.arange(len(dst)) % len(deg)
    return ops.EdgePlan.from_edge_index(torch.stack([src, dst]), len(deg)), dst


def test_chunks_tile_receivers_and_edges():
    g = torch.Generator().manual_seed(5)
    deg = torch.randint(0, 9, (200,), generator=g)
    deg[17] = 40  # one receiver above the budget on its own
    deg[100:110] = 0  # receivers without in-edges
    plan, _ = _plan(deg)
    ch = receiver_chunks(plan, 25)
    assert ch[0][0] == 0 and ch[-1][1] == 200 and ch[0][2] == 0 and ch[-1][3] == int(deg.sum())
    for (a, b, c, d), (a2, b2, c2, d2) in zip(ch, ch[1:]):
        assert b == a2 and d == c2
    for a, b, c, d in ch:
        assert d - c <= 25 or b - a == 1
        assert d - c == int(deg[a:b].sum())
    assert any(b - a == 1 and a == 17 for a, b, _, _ in ch)


def test_sub_plan_is_the_chunk_csr():
    deg = torch.tensor([3, 0, 2, 5, 1, 0, 4])
    plan, dst = _plan(deg)
    for n0, n1, e0, e1 in receiver_chunks(plan, 6):
        p = sub_plan(plan, n0, n1, e0, e1)
        assert p.n_nodes == n1 - n0 and p.n_edges == e1 - e0 and p.eid is None
        assert p.rowptr.tolist() == [0] + torch.cumsum(deg[n0:n1], 0).tolist()
        assert torch.equal(p.src, plan.src[e0:e1])
        assert torch.equal(dst[e0:e1] - n0, torch.repeat_interleave(torch.arange(n1 - n0), deg[n0:n1]))


def test_so2_block_layout_round_trip():
    """m-layout rows <-> SO(2) blocks: block 0 holds the m = 0 rows, block m
    the +m rows (GEMM row 2e) and -m rows (row 2e+1) of each edge."""
    for lmax in (1, 2, 3):
        E, ch, K = 5, 3, (lmax + 1) ** 2
        x = torch.arange(E * K * ch, dtype=torch.float64).view(E, K, ch)
        b = ops.so2_to_blocks(x, lmax)
        assert [tuple(t.shape) for t in b] == ops.so2_block_shapes(E, lmax, ch)
        assert torch.equal(ops.so2_from_blocks(b, lmax), x)
        n = lmax + 1
        # edge 2, m = 1: + rows start at row n, - rows at n + lmax
        k = n - 1
        assert torch.equal(b[1][2 * 2].view(k, ch), x[2, n:n + k])
        assert torch.equal(b[1][2 * 2 + 1].view(k, ch), x[2, n + k:n + 2 * k])


def test_group_by_key_is_a_stable_counting_sort():
    """ops.group_by_key (the sender CSR of the grad_x sums) against a
    brute-force grouping: per key, the positions holding it in increasing
    order, and the key ranges; keys that never occur (empty ranges), all
    positions on one key, no positions."""
    g = torch.Generator().manual_seed(3)
    cases = [(torch.randint(0, 40, (3000,), generator=g), 40), (torch.full((17,), 5, dtype=torch.int64), 9),
             (torch.zeros(0, dtype=torch.int64), 4), (torch.randint(0, 3, (1,), generator=g), 3)]
    for keys, n in cases:
        rp, order = ops.group_by_key(keys, n)
        assert rp.dtype == torch.int32 and order.dtype == torch.int32 and rp.shape == (n + 1,)
        kl = keys.tolist()
        want = [i for k in range(n) for i in range(len(kl)) if kl[i] == k]
        assert order.tolist() == want
        starts = [0]
        for k in range(n):
            starts.append(starts[-1] + kl.count(k))
        assert rp.tolist() == starts
