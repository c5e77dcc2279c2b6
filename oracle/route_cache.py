"""CPU restatement of the reference's route-driven expert cache policy.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HBM
expert cache (logan_amd/csrc/expert_cache.hip); nothing in the product
imports it.

Follows logan-qwen4/src/lib.rs:
  * RouteCache (:12145-12168) and RouteCache::lookup / reserve
    (:12169-12228): per-layer blocks tagged with an expert id, a replacement
    cursor per layer; a reservation takes the block already holding the
    expert (a hit), else the first block at or after the cursor that the
    current route has not claimed (pinned), counting an eviction when that
    block held another expert and bumping the generation;
  * cache_fetch_route (:12697-12903): the route's first
    retain = min(capacity, k) ranks are reserved in order, each claimed block
    pinned; hits and misses are counted once per retained rank; misses are
    loaded into their blocks, the remaining ranks stream through the route
    arena;
  * RouteArena::index / parity (:12276-12285): rank r of layer L uses arena
    block (L % 2) * topk + r.

Block numbering of the HBM allocation (this build's layout, not the
reference's separate buffers): layer L's cache block b is L * blocks + b;
arena block j is layers * blocks + j.
"""
from __future__ import annotations

from typing import List, Optional, Tuple


class RouteCachePolicy:
    def __init__(self, layers: int, blocks: int, topk: int):
        self.layers, self.blocks, self.topk = layers, blocks, topk
        self.tags: List[List[Optional[int]]] = [[None] * blocks for _ in range(layers)]
        self.next = [0] * layers
        self.generation = self.hits = self.misses = self.evictions = self.streamed = 0

    def lookup(self, layer: int, expert: int) -> Optional[int]:
        """lib.rs:12174-12178"""
        for i, t in enumerate(self.tags[layer]):
            if t == expert:
                return i
        return None

    def reserve(self, layer: int, expert: int, pinned: List[bool]):
        """(block, hit, replaced) or None (lib.rs:12190-12228)."""
        cap = self.blocks
        if cap == 0:
            return None
        i = self.lookup(layer, expert)
        if i is not None:
            return i, True, None
        start = self.next[layer] % cap
        cursor = None
        for off in range(cap):
            c = (start + off) % cap
            if not pinned[c]:
                cursor = c
                break
        if cursor is None:
            return None
        replaced = self.tags[layer][cursor]
        self.tags[layer][cursor] = expert
        self.next[layer] = (cursor + 1) % cap
        if replaced is not None:
            self.evictions += 1
        self.generation += 1
        return cursor, False, replaced

    def fetch(self, layer: int, experts) -> Tuple[List[int], List[Tuple[int, int]]]:
        """One route of `layer`: (block per rank, [(block, expert) loaded])."""
        k = len(experts)
        retain = min(self.blocks, k)
        pinned = [False] * max(self.blocks, 1)
        blocks, loads = [], []
        for r in range(retain):
            res = self.reserve(layer, int(experts[r]), pinned)
            assert res is not None
            b, hit, _ = res
            pinned[b] = True
            if hit:
                self.hits += 1
            else:
                self.misses += 1
                loads.append((layer * self.blocks + b, int(experts[r])))
            blocks.append(layer * self.blocks + b)
        for r in range(retain, k):
            b = self.layers * self.blocks + (layer % 2) * self.topk + r
            blocks.append(b)
            loads.append((b, int(experts[r])))
            self.streamed += 1
        return blocks, loads
