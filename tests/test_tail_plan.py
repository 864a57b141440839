"""The prefill GEMM2 tail split's workgroup plan (CPU).

A Python restatement of ``tail_plan`` / ``tail_offset`` and of the workgroup
mapping in ``csrc/gemm_prefill.hip`` (the GPU side is covered by the fused-path
parity tests on the shapes that take the tail split).  Checked here are the
invariants the kernels rely on, over tile counts, slot counts and stage counts:
every live logical tile is computed exactly once (whole, or by all S of its
splits), partial-buffer pairs are unique and below the host's capacity
(``tail_pairs_for``), every tail workgroup fits the launched grid, and the
fold's pair ranges stay in the buffer.
"""

import pytest

X = 8          # XCDs (workgroups dispatched round-robin)
MAX_SPLIT = 4  # kTailMaxSplit


def plan(T, x, slots, stages):
    q, r8 = divmod(T, X)
    tx = q + (1 if x < r8 else 0)
    base = x * q + min(x, r8)
    tl = tx % slots
    S = min(MAX_SPLIT, slots // tl, stages) if tl > 0 else 1
    if S < 2:
        S, tl = 1, 0
    return base, tx - tl, tl, S


def offset(T, x, slots, stages):
    total = 0
    for y in range(x):
        _, _, tl, S = plan(T, y, slots, stages)
        total += tl * S
    return total


@pytest.mark.parametrize("slots", [16, 31, 32, 64])
@pytest.mark.parametrize("stages", [1, 3, 16, 224])
def test_every_tile_once_and_pairs_in_capacity(slots, stages):
    for max_t in list(range(0, 400, 7)) + [576, 577, 4864, 9000]:
        cap = min(X * slots, max_t * MAX_SPLIT)  # tail_pairs_for
        per_xcd = (max_t + X - 1) // X
        grid = X * (per_xcd + slots)
        for T in sorted({max_t, max(0, max_t - 5), max_t // 2}):
            seen, pairs = {}, set()
            for b in range(grid):
                x, i = b % X, b // X
                base, full, tl, S = plan(T, x, slots, stages)
                if i < full:
                    seen.setdefault(base + i, []).append((0, 1))
                    continue
                j = i - full
                if j >= tl * S:
                    continue
                pair = offset(T, x, slots, stages) + j
                assert pair < cap and pair not in pairs
                pairs.add(pair)
                seen.setdefault(base + full + j // S, []).append((j % S, S))
            assert sorted(seen) == list(range(T))
            for parts in seen.values():
                S = parts[0][1]
                assert sorted(s for s, _ in parts) == list(range(S))
                assert all(n == S for _, n in parts) and S <= min(MAX_SPLIT, stages)
            for x in range(X):
                base, full, tl, S = plan(T, x, slots, stages)
                assert full + tl * S <= per_xcd + slots  # inside the launched grid
                assert offset(T, x, slots, stages) + tl * S <= cap  # fold ranges


def test_tail_fills_at_most_one_round():
    # a partial last round is split only while its split workgroups fit the
    # XCD's slots; a round more than half full stays whole
    assert plan(8 * 72, 0, 32, 224) == (0, 64, 8, 4)
    assert plan(8 * 60, 0, 32, 224) == (0, 60, 0, 1)
    assert plan(8 * 20, 0, 32, 224) == (0, 20, 0, 1)
    assert plan(8 * 12, 0, 32, 224) == (0, 0, 12, 2)
    assert plan(8 * 72, 0, 32, 3) == (0, 64, 8, 3)
