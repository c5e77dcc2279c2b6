"""GPU parity of the route-driven expert cache (logan_hip_expert_cache_*,
logan_hip_moe_block_cached): the reference's RouteCache / RouteArena
(logan-qwen4/src/lib.rs:12110-12300, cache_fetch_route :12697-12903) in HBM.

Bars: the block of every rank, the layer's tags and the hit / miss /
eviction / streamed counts equal the policy restatement's
(oracle/route_cache.py, pinned on the CPU by tests/test_route_cache.py);
bytes loaded = (misses + streamed) x block bytes (hits load nothing); the
MoE block on cache-fed experts is bitwise equal to logan_hip_moe_block on
resident banks read from the same checkpoint (the same kernels and bytes),
its routing bit-exact and its output within 5e-5 normwise of the oracle's
token, on the single-launch and the per-token B = 1 paths.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import checkpoint as ock
from oracle.route_cache import RouteCachePolicy
from logan_amd.synth import bf16_bits, bf16_to_f32

from _util import normwise_rel
from test_checkpoint_gpu import affine_tensors

pytestmark = pytest.mark.gpu

E, K, D, INTER, BITS, GS = 32, 8, 512, 256, 4, 64
LAYERS = 3  # layer 2's banks use groups of 32: a layout the cache declines
ROLES = (("gate_proj", INTER, D), ("up_proj", INTER, D), ("down_proj", D, INTER))


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    rng = np.random.default_rng(3030)
    d = tmp_path_factory.mktemp("cache_ckpt")
    shards = [[], []]
    for layer in range(LAYERS):
        pre = f"language_model.model.layers.{layer}.mlp"
        gs = GS if layer < 2 else 32
        for role, O, I in ROLES:
            shards[layer % 2] += affine_tensors(rng, f"{pre}.switch_mlp.{role}", O, I, BITS, gs, E=E)
            shards[layer % 2] += affine_tensors(rng, f"{pre}.shared_expert.{role}", O, I, BITS, gs)
        seg = bf16_bits(rng.standard_normal(D).astype(np.float32) * np.float32(0.05))
        shards[layer % 2].append((f"{pre}.shared_expert_gate.weight", "BF16", [1, D], seg.tobytes()))
    ock.write_sharded_checkpoint(str(d), [("model-00001-of-00002.safetensors", shards[0]),
                                          ("model-00002-of-00002.safetensors", shards[1])])
    return str(d)


class LayerSet:
    """Per layer: resident banks, the shared expert and its gate row (device),
    the oracle's host arrays, and a cached-bank MoeLayer."""

    def __init__(self, torch, st, ost, cache, layer):
        from logan_amd import checkpoint, device

        pre = f"model.layers.{layer}.mlp"
        banks = {r: checkpoint.load_mlx_quantized_bank(st, f"{pre}.switch_mlp.{r}.weight", E, O, I)
                 for r, O, I in ROLES}
        shared = {r: checkpoint.load_mlx_quantized_wt(st, f"{pre}.shared_expert.{r}.weight", O,
                                                      I).as_bank()
                  for r, O, I in ROLES}
        self.seg = np.frombuffer(st.payload(f"{pre}.shared_expert_gate.weight"), np.uint16).copy()
        segd = torch.from_numpy(self.seg.view(np.int16)).cuda().view(torch.bfloat16)
        sh = (shared["gate_proj"], shared["up_proj"], shared["down_proj"])
        self.resident = device.MoeLayer(banks["gate_proj"], banks["up_proj"], banks["down_proj"], K,
                                        *sh, segd)
        self.cached = device.MoeLayer(*cache.geometry(BITS, GS), K, *sh, segd)
        self._keep = (banks, shared)

        def obank(role, O, I):
            ts = [ock.load_mlx_quantized_expert_wt(ost, f"{pre}.switch_mlp.{role}.weight", e, E, O, I)
                  for e in range(E)]
            return (np.stack([np.frombuffer(t.weights, np.uint8).reshape(O, -1) for t in ts]),
                    np.stack([np.frombuffer(t.scales, np.uint16).reshape(O, -1) for t in ts]),
                    np.stack([np.frombuffer(t.biases, np.uint16).reshape(O, -1) for t in ts]))

        self.host = [obank(r, O, I) for r, O, I in ROLES]
        shh = []
        for r, O, I in ROLES:
            q = ock.load_mlx_quantized_wt(ost, f"{pre}.shared_expert.{r}.weight", O, I)
            shh.append((np.frombuffer(q.weights, np.uint8).reshape(O, -1),
                        np.frombuffer(q.scales, np.uint16).reshape(O, -1),
                        np.frombuffer(q.biases, np.uint16).reshape(O, -1)))
        self.shared_host = tuple(shh)

    def ref(self, xf, lf):
        g, u, dn = self.host
        return oracle.moe_token(xf, lf, K, D, INTER, BITS, GS, g, u, dn, self.shared_host,
                                bf16_to_f32(self.seg))


def _dev_bf16(torch, bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch.bfloat16)


@pytest.mark.parametrize("fused", [1, 0])
def test_cached_block_matches_resident_and_oracle(gpu, ckpt, fused):
    import torch

    from logan_amd import _lib, checkpoint, device

    print(f"expert cache fused={fused}", flush=True)
    ost = ock.StFile.open_dir(ckpt)
    st = checkpoint.StFile.open_dir(ckpt)
    cache = checkpoint.ExpertCache(st, E, D, INTER, blocks_per_layer=4, topk=K)
    assert cache.layers == LAYERS and cache.topk == K
    s0 = cache.stats()
    assert s0["block_bytes"] % 256 == 0
    assert s0["device_bytes"] == s0["block_bytes"] * (LAYERS * 4 + 2 * K)
    layers = [LayerSet(torch, st, ost, cache, l) for l in range(2)]
    policy = RouteCachePolicy(LAYERS, 4, K)
    rng = np.random.default_rng(404 + fused)
    _lib.lib().logan_hip_set_moe_fused(fused)
    try:
        prev = None
        for step in range(10):
            cur = []
            for li, L in enumerate(layers):
                xb = bf16_bits(rng.standard_normal(D).astype(np.float32))
                if step % 3 == 2 and prev is not None:
                    lb = prev[li]  # the same route again: retained ranks hit
                else:
                    lb = bf16_bits(rng.standard_normal(E).astype(np.float32))
                cur.append(lb)
                x, lg = _dev_bf16(torch, xb[None]), _dev_bf16(torch, lb[None])
                idx, _ = device.route_topk(lg, K)
                experts = idx.cpu().numpy()[0]
                blocks = cache.fetch(li, experts)
                want_blocks, _ = policy.fetch(li, experts)
                np.testing.assert_array_equal(blocks, want_blocks)
                out, ridx, _ = device.moe_block_cached(L.cached, cache, experts, blocks, x, lg,
                                                       return_routing=True, out_dtype=torch.float32)
                res = device.moe_block(L.resident, x, lg, out_dtype=torch.float32)
                assert torch.equal(out, res), (step, li)
                np.testing.assert_array_equal(ridx.cpu().numpy()[0], experts)
                if step < 2:
                    ref, oidx, _ = L.ref(bf16_to_f32(xb), bf16_to_f32(lb))
                    np.testing.assert_array_equal(experts, oidx)
                    assert normwise_rel(out.cpu().numpy()[0], ref) <= 5e-5
            prev = cur
        s = cache.stats()
        assert (s["hits"], s["misses"], s["evictions"], s["streamed"]) == \
            (policy.hits, policy.misses, policy.evictions, policy.streamed)
        assert s["generation"] == policy.generation
        assert s["bytes_loaded"] == (policy.misses + policy.streamed) * s["block_bytes"]
        assert policy.hits > 0 and policy.evictions > 0
        for li in range(2):
            want = [-1 if t is None else t for t in policy.tags[li]]
            np.testing.assert_array_equal(cache.tags(li), want)
    finally:
        _lib.lib().logan_hip_set_moe_fused(1)
        cache.close()
    assert _lib.lib().logan_hip_moe_sync_errors() == 0



def test_cache_declines_what_it_cannot_serve(gpu, ckpt):
    """A layer whose banks differ from the cache's block layout (groups of
    32, RouteArena::layout_matches, lib.rs:12266-12275), more ranks than the
    arena holds, an expert id out of range: declined (None), nothing loaded;
    a cache with no retained blocks streams every rank through the arena."""
    from logan_amd import checkpoint

    st = checkpoint.StFile.open_dir(ckpt)
    cache = checkpoint.ExpertCache(st, E, D, INTER, blocks_per_layer=2, topk=4)
    assert cache.fetch(2, [0, 1, 2, 3]) is None
    assert cache.fetch(0, [0, 1, 2, 3, 4]) is None
    assert cache.fetch(0, [0, 1, E, 3]) is None
    assert cache.stats()["bytes_loaded"] == 0
    cache.close()
    arena = checkpoint.ExpertCache(st, E, D, INTER, blocks_per_layer=0, topk=4)
    assert list(arena.fetch(1, [5, 6, 7, 8])) == [3 * 0 + 4 + r for r in range(4)]
    s = arena.stats()
    assert (s["hits"], s["misses"], s["streamed"]) == (0, 0, 4)
    arena.close()
