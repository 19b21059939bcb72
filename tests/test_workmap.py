"""Workgroup -> (head pair, block) decode of both kernels (host function shared with the device
code): every block of every (batch, head) pair is owned by exactly one workgroup, so dK/dV rows
(backward) and O rows (forward) have a single writer; blocks of one pair share an XCD when the
pair count allows; pairs go out in chunks whose blocks are dispatched block-major, largest causal
work first, so that a greedy dispatcher that starts workgroups in id order as slots free up
finishes within one block's work of the lower bound."""
import heapq

import numpy as np
import pytest

import metalllm_amd as M


@pytest.mark.parametrize("B,T,H,D", [(16, 256, 6, 64), (128, 256, 6, 64), (32, 1024, 12, 64), (16, 4096, 16, 128),
                                     (1, 192, 3, 128), (3, 320, 1, 64), (1, 64, 1, 64)])
@pytest.mark.parametrize("kind,blk,last_first", [(0, 128, True), (1, 128, False), (2, 128, True)])
def test_partition(B, T, H, D, kind, blk, last_first):
    wm = M.work_map(kind, B, T, H, D)
    npairs, nblk = B * H, -(-T // blk)
    assert wm.shape == (npairs * nblk, 2)
    seen = set(map(tuple, wm.tolist()))
    assert seen == {(p, b) for p in range(npairs) for b in range(nblk)}
    # causal work of a block: a query block qb (forward, dQ) sees qb+1 key blocks, a key block kb
    # (dK/dV) sees T/64 - 2kb query tiles; within a pair the dispatch order is non-increasing in work
    work = (wm[:, 1] + 1) if kind != 1 else (T // 64 - 2 * wm[:, 1])
    for p in range(npairs):
        w = work[wm[:, 0] == p]
        assert (np.diff(w) <= 0).all()
    if npairs % 8 == 0:  # workgroup i runs on XCD i % 8: all blocks of a pair share one XCD
        for p in range(npairs):
            assert len(set((np.nonzero(wm[:, 0] == p)[0] % 8).tolist())) == 1
    # per dispatch group (an XCD's share when the pairs split over 8, else the whole grid): a chunk
    # of C pairs, C * nblk >= 64 workgroups per XCD for the D = 128 backward (one round of resident
    # workgroups, two per CU), 192 for the D = 64 backward (two rounds of three per CU) and 128 for
    # the forward, is dispatched with non-increasing work, and a chunk's pairs are consecutive in
    # the group
    groups = [np.arange(x, len(wm), 8) for x in range(8)] if npairs % 8 == 0 else [np.arange(len(wm))]
    rnd = (128 if kind == 0 else (192 if D == 64 else 64)) * (1 if npairs % 8 == 0 else 8)
    per_xcd = 96 if (kind != 0 and D == 64) else 64  # resident workgroups per XCD
    C = max(1, -(-rnd // nblk))
    for ids in groups:
        w, pr = work[ids], wm[ids, 0]
        for c0 in range(0, len(ids), C * nblk):
            assert (np.diff(w[c0:c0 + C * nblk]) <= 0).all()
            assert len(set(pr[c0:c0 + C * nblk].tolist())) == min(C, len(set(pr.tolist())) - c0 // nblk)
        # greedy dispatch in id order onto one round of slots, block time = its work + 1 (start
        # cost): no later than dispatching the same pairs one after another, each pair's blocks
        # longest first
        def makespan(ws):
            slots = [0.0] * min(per_xcd if npairs % 8 == 0 else 8 * per_xcd, len(ws))
            for d in ws:
                heapq.heappush(slots, heapq.heappop(slots) + d + 1.0)
            return max(slots)
        pair_major = np.concatenate([np.sort(w[pr == p])[::-1] for p in sorted(set(pr.tolist()))])
        assert makespan(w) <= makespan(pair_major)


@pytest.mark.parametrize("B,T,H,D", [(128, 256, 6, 64), (16, 256, 6, 64), (3, 192, 5, 128), (1, 64, 1, 64),
                                     (2, 128, 3, 64)])
@pytest.mark.parametrize("grid", [768, 512, 96, 8, 7, 1])
def test_persistent_forward_items(B, T, H, D, grid):
    """The persistent forward (at most two items per resident workgroup): every (pair, query block) item is run by exactly one
    workgroup; when the pair count and the grid are multiples of 8, all items of a workgroup
    belong to pairs on its XCD (workgroup w runs on XCD w % 8); each workgroup's causal work
    (query block + 1 key tiles per item) is within one item's work of the mean."""
    npairs, nblk = B * H, -(-T // 128)
    items = M.forward_items(B, T, H, D, grid)
    assert items.shape == (npairs * nblk, 3)
    assert set(map(tuple, items[:, 1:].tolist())) == {(p, b) for p in range(npairs) for b in range(nblk)}
    assert ((items[:, 0] >= 0) & (items[:, 0] < grid)).all()
    if npairs % 8 == 0 and grid % 8 == 0:
        assert (items[:, 1] % 8 == items[:, 0] % 8).all()
    work = np.bincount(items[:, 0], weights=items[:, 2] + 1, minlength=grid)
    used = min(grid, npairs * nblk)
    assert work[:used].min() > 0 and (work[used:] == 0).all()
    assert work.max() - work.sum() / used <= nblk
