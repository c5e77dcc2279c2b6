"""GPU parity of the checkpoint loader: weights read from safetensors files
into HBM by logan-hip (include/logan_hip.h layer 3) against the oracle's
restatement of the reference loader (oracle/checkpoint.py).

Bars: every loaded code and parameter reaches the device unchanged — checked
through the bit-exact dequantisation entries (each weight and each scale /
bias takes part in some dequantised value) against the oracle's dequant of
the bytes the reference loader returns; products through the loaded handles
within the GEMV / MoE tests' tolerances (normwise 2e-5 / 5e-5 of the f32
oracle); routing indices bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import checkpoint as ock
from logan_amd.synth import bf16_bits, bf16_to_f32

from _util import normwise_rel

pytestmark = pytest.mark.gpu


def affine_tensors(rng, name, O, I, bits, gs, fp16=False, E=None):
    lead = [] if E is None else [E]
    words = I * bits // 32
    w = rng.integers(0, 2**32, lead + [O, words], dtype=np.uint32)
    s = np.abs(rng.standard_normal(lead + [O, I // gs])).astype(np.float32) * np.float32(0.01)
    if fp16:
        sc = s.astype(np.float16).view(np.uint16)
        bi = (-(2 ** (bits - 1)) * s).astype(np.float16).view(np.uint16)
    else:
        sc = bf16_bits(s)
        bi = bf16_bits(-(2 ** (bits - 1)) * bf16_to_f32(sc))
    dt = "F16" if fp16 else "BF16"
    return [(f"{name}.weight", "U32", lead + [O, words], w.tobytes()),
            (f"{name}.scales", dt, lead + [O, I // gs], np.ascontiguousarray(sc).tobytes()),
            (f"{name}.biases", dt, lead + [O, I // gs], np.ascontiguousarray(bi).tobytes())]


def mx_tensors(rng, name, O, I, E=None):
    lead = [] if E is None else [E]
    w = rng.integers(0, 2**32, lead + [O, I // 8], dtype=np.uint32)
    sc = rng.integers(118, 136, lead + [O, I // 32]).astype(np.uint8)
    return [(f"{name}.weight", "U32", lead + [O, I // 8], w.tobytes()),
            (f"{name}.scales", "U8", lead + [O, I // 32], sc.tobytes())]


def as_arrays(q: ock.QuantWt, rows: int):
    w = np.frombuffer(q.weights, np.uint8).reshape(rows, -1)
    if q.kind == "mxfp4":
        return w, np.frombuffer(q.scales, np.uint8).reshape(rows, -1), None
    return (w, np.frombuffer(q.scales, np.uint16).reshape(rows, -1),
            np.frombuffer(q.biases, np.uint16).reshape(rows, -1))


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    """A two-shard MLX checkpoint: dense 4/5/6/8-bit matrices (bf16 and fp16
    sidecars), a dense MXFP4 matrix, a routed MoE layer's switch_mlp banks
    (E = 64, D = 512, inter = 256, 4-bit g64) with its shared expert, an MXFP4
    expert stack, and one 132 MiB bank that spans several staging slots."""
    rng = np.random.default_rng(2024)
    d = tmp_path_factory.mktemp("ckpt")
    pre = "language_model.model.layers.3"
    s1 = []
    s1 += affine_tensors(rng, f"{pre}.self_attn.q_proj", 96, 512, 4, 64)
    s1 += affine_tensors(rng, f"{pre}.self_attn.k_proj", 64, 256, 5, 32, fp16=True)
    s1 += affine_tensors(rng, f"{pre}.self_attn.v_proj", 48, 384, 6, 64)
    s1 += affine_tensors(rng, f"{pre}.self_attn.o_proj", 80, 512, 8, 128)
    s1 += mx_tensors(rng, f"{pre}.linear_attn.in_proj_a", 72, 256)
    for role, O, I in (("gate_proj", 256, 512), ("up_proj", 256, 512), ("down_proj", 512, 256)):
        s1 += affine_tensors(rng, f"{pre}.mlp.switch_mlp.{role}", O, I, 4, 64, E=64)
        s1 += affine_tensors(rng, f"{pre}.mlp.shared_expert.{role}", O, I, 4, 64)
    s2 = []
    s2 += mx_tensors(rng, f"{pre}.mlp.switch_mlp_mx.gate_proj", 128, 256, E=6)
    s2 += affine_tensors(rng, "model.layers.9.mlp.switch_mlp.gate_proj", 512, 2048, 4, 64, E=256)
    seg = bf16_bits(rng.standard_normal(512).astype(np.float32) * np.float32(0.05))
    s2.append((f"{pre}.mlp.shared_expert_gate.weight", "BF16", [1, 512], seg.tobytes()))
    ock.write_sharded_checkpoint(str(d), [("model-00001-of-00002.safetensors", s1),
                                          ("model-00002-of-00002.safetensors", s2)])
    return str(d)


DENSE = [
    ("model.layers.3.self_attn.q_proj.weight", 96, 512),
    ("model.layers.3.self_attn.k_proj.weight", 64, 256),
    ("model.layers.3.self_attn.v_proj.weight", 48, 384),
    ("model.layers.3.self_attn.o_proj.weight", 80, 512),
]


@pytest.mark.parametrize("name,O,I", DENSE)
def test_dense_affine_load_is_byte_exact_and_computes(gpu, ckpt, name, O, I):
    import torch

    from logan_amd import checkpoint, device

    want = ock.load_mlx_quantized_wt(ock.StFile.open_dir(ckpt), name, O, I)
    w, sc, bi = as_arrays(want, O)
    with checkpoint.StFile.open_dir(ckpt) as st:
        m = checkpoint.load_mlx_quantized_wt(st, name, O, I)
    assert (m.bits, m.group_size, m.aux_fp16) == (want.bits, want.group_size, want.aux_fp16)
    got = device.affine_dequant(m).cpu().numpy()
    ref = oracle.affine_dequant(w, sc, bi, O, I, want.bits, want.group_size, want.aux_fp16)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    rng = np.random.default_rng(O)
    x = bf16_bits(rng.standard_normal((1, I)).astype(np.float32))
    y = device.affine_gemv(m, torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16),
                           out_dtype=torch.float32).cpu().numpy()[0]
    yr = oracle.affine_gemv(bf16_to_f32(x[0]), w, sc, bi, O, I, want.bits, want.group_size,
                            want.aux_fp16)
    assert normwise_rel(y, yr) <= 2e-5


def test_mxfp4_load_is_byte_exact(gpu, ckpt):
    import torch

    from logan_amd import checkpoint, device

    name, O, I = "model.layers.3.linear_attn.in_proj_a.weight", 72, 256
    want = ock.load_mlx_quantized_wt(ock.StFile.open_dir(ckpt), name, O, I)
    assert want.kind == "mxfp4"
    w, sc, _ = as_arrays(want, O)
    with checkpoint.StFile.open_dir(ckpt) as st:
        m = checkpoint.load_mlx_quantized_wt(st, name, O, I)
    assert isinstance(m, checkpoint.LoadedMxfp4)
    got = device.mxfp4_dequant(m).cpu().numpy()
    lib = oracle.lib()
    ref = np.empty((O, I), np.float32)
    for r in range(O):
        for j in range(I):
            b = int(w[r, j // 2])
            ref[r, j] = lib.lo_mxfp4_value(b & 0xF if j % 2 == 0 else b >> 4, int(sc[r, j // 32]))
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    x = np.random.default_rng(1).standard_normal(I).astype(np.float32)
    y = device.mxfp4_gemv([m], [torch.from_numpy(x).cuda()])[0].cpu().numpy()
    yr = oracle.mxfp4_gemv(x, w, sc, O, I)
    assert normwise_rel(y, yr) <= 2e-5


def test_mxfp4_expert_stack(gpu, ckpt):
    from logan_amd import checkpoint, device

    name, E, O, I = "model.layers.3.mlp.switch_mlp_mx.gate_proj.weight", 6, 128, 256
    ost = ock.StFile.open_dir(ckpt)
    with checkpoint.StFile.open_dir(ckpt) as st:
        stack = checkpoint.load_mlx_quantized_bank(st, name, E, O, I)
        one = checkpoint.load_mlx_quantized_expert_wt(st, name, 4, E, O, I)
    for e, m in ((4, stack.expert(4)), (4, one), (0, stack.expert(0)), (5, stack.expert(5))):
        q = ock.load_mlx_quantized_expert_wt(ost, name, e, E, O, I)
        w, sc, _ = as_arrays(q, O)
        got = device.mxfp4_dequant(m).cpu().numpy()
        codes = np.stack([w & 0xF, w >> 4], axis=-1).reshape(O, I)
        lib = oracle.lib()
        lut = np.array([[lib.lo_mxfp4_value(c, s) for s in range(256)] for c in range(16)],
                       np.float32)
        ref = lut[codes, np.repeat(sc, 32, axis=1)]
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_bank_spanning_staging_slots(gpu, ckpt):
    """A 256-expert 512x2048 bank (132 MiB in one transfer, several 32 MiB
    staging slots): experts at the start, middle, slot boundaries and the end
    dequantise bit-exactly; one-expert loads agree with the bank."""
    from logan_amd import checkpoint, device

    name, E, O, I = "model.layers.9.mlp.switch_mlp.gate_proj.weight", 256, 512, 2048
    ost = ock.StFile.open_dir(ckpt)
    with checkpoint.StFile.open_dir(ckpt) as st:
        bank = checkpoint.load_mlx_quantized_bank(st, name, E, O, I)
        part = checkpoint.load_mlx_quantized_bank(st, name, E, O, I, e0=61, count=3)
        single = checkpoint.load_mlx_quantized_expert_wt(st, name, 255, E, O, I)
    assert bank.E == E and part.E == 3
    # expert 63 straddles the first 32 MiB slot boundary (64 experts per slot)
    for e, m in ((0, bank.expert(0)), (63, bank.expert(63)), (64, bank.expert(64)),
                 (127, bank.expert(127)), (200, bank.expert(200)), (255, bank.expert(255)),
                 (62, part.expert(1)), (63, part.expert(2)), (255, single)):
        q = ock.load_mlx_quantized_expert_wt(ost, name, e, E, O, I)
        w, sc, bi = as_arrays(q, O)
        rows = (0, 1, 255, 510, 511)
        got = device.affine_dequant(m).cpu().numpy()[list(rows)]
        ref = oracle.affine_dequant(w, sc, bi, O, I, 4, 64)[list(rows)]
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32), err_msg=str(e))
    # the parameter stacks land whole: their last expert's last row
    q = ock.load_mlx_quantized_expert_wt(ost, name, 255, E, O, I)
    w, sc, bi = as_arrays(q, O)
    got = device.affine_dequant(bank.expert(255), 511, 1).cpu().numpy()
    ref = oracle.affine_dequant(w, sc, bi, O, I, 4, 64, row0=511, nrows=1)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_moe_block_runs_on_loaded_banks(gpu, ckpt):
    """A routed MoE layer read from the checkpoint (switch_mlp banks, shared
    expert and its gate row) runs through moe_block; routing bit-exact and
    outputs within 5e-5 normwise of the oracle's token on the same bytes."""
    import torch

    from logan_amd import checkpoint, device

    E, k, D, inter = 64, 4, 512, 256
    pre = "model.layers.3.mlp"
    ost = ock.StFile.open_dir(ckpt)
    with checkpoint.StFile.open_dir(ckpt) as st:
        banks = {r: checkpoint.load_mlx_quantized_bank(st, f"{pre}.switch_mlp.{r}.weight", E, O, I)
                 for r, O, I in (("gate_proj", inter, D), ("up_proj", inter, D),
                                 ("down_proj", D, inter))}
        shared = {r: checkpoint.load_mlx_quantized_wt(st, f"{pre}.shared_expert.{r}.weight", O,
                                                      I).as_bank()
                  for r, O, I in (("gate_proj", inter, D), ("up_proj", inter, D),
                                  ("down_proj", D, inter))}
        seg = np.frombuffer(st.payload(f"{pre}.shared_expert_gate.weight"), np.uint16).copy()
    # the shared expert is stored dense ([O, words]): a one-expert bank
    layer = device.MoeLayer(banks["gate_proj"], banks["up_proj"], banks["down_proj"], k,
                            shared["gate_proj"], shared["up_proj"], shared["down_proj"],
                            torch.from_numpy(seg.view(np.int16)).cuda().view(torch.bfloat16))

    def obank(role, O, I, n):
        ts = [ock.load_mlx_quantized_expert_wt(ost, f"{pre}.switch_mlp.{role}.weight", e, E, O, I)
              for e in range(n)]
        return (np.stack([np.frombuffer(t.weights, np.uint8).reshape(O, -1) for t in ts]),
                np.stack([np.frombuffer(t.scales, np.uint16).reshape(O, -1) for t in ts]),
                np.stack([np.frombuffer(t.biases, np.uint16).reshape(O, -1) for t in ts]))

    g, u, dn = obank("gate_proj", inter, D, E), obank("up_proj", inter, D, E), obank("down_proj", D, inter, E)
    sh = []
    for role, O, I in (("gate_proj", inter, D), ("up_proj", inter, D), ("down_proj", D, inter)):
        q = ock.load_mlx_quantized_wt(ost, f"{pre}.shared_expert.{role}.weight", O, I)
        sh.append(as_arrays(q, O))
    rng = np.random.default_rng(9)
    for B in (1, 5):
        xb = bf16_bits(rng.standard_normal((B, D)).astype(np.float32))
        lb = bf16_bits(rng.standard_normal((B, E)).astype(np.float32))
        out, idx, wt = device.moe_block(
            layer, torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16),
            torch.from_numpy(lb.view(np.int16)).cuda().view(torch.bfloat16),
            return_routing=True, out_dtype=torch.float32)
        out, idx = out.cpu().numpy(), idx.cpu().numpy()
        for b in range(B):
            ref, ridx, _ = oracle.moe_token(bf16_to_f32(xb[b]), bf16_to_f32(lb[b]), k, D, inter, 4,
                                            64, g, u, dn, tuple(sh), bf16_to_f32(seg))
            assert np.array_equal(idx[b], ridx), (B, b)
            assert normwise_rel(out[b], ref) <= 5e-5, (B, b)


def test_loads_release_their_memory(gpu, ckpt):
    """A 132 MiB bank shows up in the device's used memory while held and is
    gone after quant_free (explicit, and again through the owner's __del__)."""
    import ctypes as C
    import gc

    from logan_amd import _lib as L, checkpoint

    def used():
        u, t = C.c_size_t(0), C.c_size_t(0)
        assert L.lib().logan_hip_mem_info(C.byref(u), C.byref(t)) == 1
        return u.value

    name, E, O, I = "model.layers.9.mlp.switch_mlp.gate_proj.weight", 256, 512, 2048
    nbytes = E * O * I // 2 + 2 * E * O * (I // 64) * 2
    with checkpoint.StFile.open_dir(ckpt) as st:
        u0 = used()
        bank = checkpoint.load_mlx_quantized_bank(st, name, E, O, I)
        assert bank._own.q.weight_bytes == E * O * I // 2
        assert used() - u0 >= nbytes
        q = bank._own.q
        L.lib().logan_hip_quant_free(q)
        assert not q.owner and not q.weights
        assert used() - u0 < nbytes // 2
        del bank
        gc.collect()
        bank = checkpoint.load_mlx_quantized_bank(st, name, E, O, I)
        assert used() - u0 >= nbytes
        del bank
        gc.collect()
        assert used() - u0 < nbytes // 2
