"""CPU pinning of the route-cache policy restatement (oracle/route_cache.py),
the checker of the HBM expert cache's block choices and counters.

The reference has no tests for RouteCache; it is pinned here by the worked
example of RouteCache::reserve's own comment
(logan-qwen4/src/lib.rs:12180-12189: cap 4, tags [A, B, C, D], cursor 2,
route [C, X, Y, Z]), the stated cold-insert rule (:12183-12185: an insert
into an empty block is a miss, not a hit, and evicts nothing), and
invariants a wrong cursor, a missing pin or a miscount would break, checked
over random routes.
"""
import numpy as np

from oracle.route_cache import RouteCachePolicy

A, B, C, D, X, Y, Z = 10, 11, 12, 13, 20, 21, 22


def test_reserve_comment_example():
    p = RouteCachePolicy(layers=1, blocks=4, topk=4)
    p.tags[0] = [A, B, C, D]
    p.next[0] = 2
    blocks, loads = p.fetch(0, [C, X, Y, Z])
    # rank 0 hits C in block 2; the misses skip that pinned block
    assert blocks == [2, 3, 0, 1]
    assert loads == [(3, X), (0, Y), (1, Z)]
    assert p.tags[0] == [Y, Z, C, X]
    assert (p.hits, p.misses, p.evictions, p.next[0]) == (1, 3, 3, 2)
    # without the pin rank 1 would have taken block 2 and clobbered C
    q = RouteCachePolicy(layers=1, blocks=4, topk=4)
    q.tags[0] = [A, B, C, D]
    q.next[0] = 2
    assert q.reserve(0, X, [False] * 4)[0] == 2


def test_cold_inserts_are_misses():
    p = RouteCachePolicy(layers=2, blocks=3, topk=4)
    blocks, loads = p.fetch(1, [5, 6, 7, 8])
    assert blocks[:3] == [3, 4, 5]                   # layer 1's blocks
    assert blocks[3] == 2 * 3 + 1 * 4 + 3            # arena, parity 1, rank 3
    assert (p.hits, p.misses, p.evictions, p.streamed) == (0, 3, 0, 1)
    assert p.generation == 3
    blocks2, loads2 = p.fetch(1, [7, 5, 6, 9])
    assert blocks2[:3] == [5, 3, 4] and loads2 == [(2 * 3 + 4 + 3, 9)]
    assert (p.hits, p.misses) == (3, 3)
    # the same route on layer 0 shares nothing with layer 1
    blocks3, _ = p.fetch(0, [7, 5, 6, 9])
    assert blocks3 == [0, 1, 2, 2 * 3 + 0 + 3] and p.misses == 6


def test_earlier_miss_can_evict_a_later_ranks_expert():
    """The pin protects blocks the route has claimed, not experts it has yet
    to reach: with the cursor on Q's block, rank 0's miss takes it and rank
    1 (Q) then misses too (reserve's order of operations, :12198-12226)."""
    Q = 30
    p = RouteCachePolicy(layers=1, blocks=2, topk=2)
    p.tags[0] = [Q, A]
    p.next[0] = 0
    blocks, loads = p.fetch(0, [X, Q])
    assert blocks == [0, 1] and loads == [(0, X), (1, Q)]
    assert (p.hits, p.misses, p.evictions) == (0, 2, 2)


def test_zero_capacity_streams_every_rank():
    p = RouteCachePolicy(layers=3, blocks=0, topk=2)
    assert p.fetch(2, [4, 1]) == ([0, 1], [(0, 4), (1, 1)])
    assert p.fetch(1, [4, 1]) == ([2, 3], [(2, 4), (3, 1)])
    assert (p.hits, p.misses, p.streamed) == (0, 0, 4)


def test_random_routes_keep_the_invariants():
    rng = np.random.default_rng(5)
    layers, blocks, topk, E = 3, 5, 8, 24
    p = RouteCachePolicy(layers, blocks, topk)
    for _ in range(400):
        layer = int(rng.integers(0, layers))
        k = int(rng.integers(1, topk + 1))
        route = rng.choice(E, k, replace=False)
        before = list(p.tags[layer])
        h0, m0, e0 = p.hits, p.misses, p.evictions
        got, loads = p.fetch(layer, route)
        retain = min(blocks, k)
        # a hit needs the expert tagged before this route (an earlier rank's
        # miss may evict it first: pins cover claimed blocks only), and every
        # hit keeps its block
        hits = p.hits - h0
        assert hits <= sum(int(route[r]) in before for r in range(retain))
        assert p.misses - m0 == retain - hits
        # each retained rank's block is its layer's, and ranks never share one
        cache = got[:retain]
        assert len(set(cache)) == retain
        assert all(layer * blocks <= b < (layer + 1) * blocks for b in cache)
        for r, b in enumerate(cache):
            assert p.tags[layer][b - layer * blocks] == int(route[r])
        # evictions are misses into blocks that held an expert
        replaced = sum(before[b - layer * blocks] is not None and
                       before[b - layer * blocks] != int(route[r])
                       for r, b in enumerate(cache))
        assert p.evictions - e0 == replaced
        # the tail takes this parity's arena blocks by rank
        for r in range(retain, k):
            assert got[r] == layers * blocks + (layer % 2) * topk + r
        # loads: exactly the misses and the tail
        assert len(loads) == (retain - hits) + (k - retain)
        # other layers untouched
        assert all(len(t) == blocks for t in p.tags)
