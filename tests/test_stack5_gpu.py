"""Config 5 (Qwen3-Next-80B-A3B-shaped stack, 4-bit g64) under test: the
decode step of one linear-attention and one full-attention layer, made of
the same calls bench.py times (affine_gemv_multi for the projections that
read the hidden state, affine_gemv for the output projections that read the
attention output, then the MoE block), at B = 1, 2 and 32. Every output row
is compared with the oracle: f32 outputs normwise, bf16 outputs within 1 bf16
ulp of RNE(oracle) away from cancellation, routing bit-exact.

Shapes (logan-qwen4/src/lib.rs:16770-16797): full attention q 2048->8192,
k/v 2048->512, o 4096->2048; linear attention qkvz 2048->12288,
ba 2048->64, out 4096->2048; MoE E=512 top-10 + shared expert, D=2048,
inter=512.
"""
import numpy as np
import pytest

import oracle
from logan_amd.synth import bf16_to_f32, make_affine, make_logits, make_x

from _util import bf16_ulp_ok, normwise_rel

pytestmark = pytest.mark.gpu

FULL_ATTN = (("q", 8192, 2048), ("k", 512, 2048), ("v", 512, 2048), ("o", 2048, 4096))
LIN_ATTN = (("qkvz", 12288, 2048), ("ba", 64, 2048), ("out", 2048, 4096))
D = 2048


def to_dev(a, torch, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def check_rows(y16, y32, xf, host, O, I):
    w, sc, bi = host
    for r in range(xf.shape[0]):
        ref = oracle.affine_gemv(xf[r], w, sc, bi, O, I, 4, 64)
        assert normwise_rel(y32[r], ref) <= 2e-5, f"row {r} O={O} I={I}"
        big = np.abs(ref) > 1e-2 * np.abs(ref).max()
        assert bf16_ulp_ok(y16[r][big], ref[big], 1), f"row {r} O={O} I={I}"


@pytest.mark.parametrize("B", [1, 2, 32])
@pytest.mark.parametrize("shapes", [LIN_ATTN, FULL_ATTN], ids=["linear", "full"])
def test_config5_projections(gpu, shapes, B):
    import torch
    from logan_amd.device import AffineMatrix, affine_gemv, affine_gemv_multi

    print(f"config5 projections {shapes[0][0]} B={B}", flush=True)
    rng = np.random.default_rng(500 + B + len(shapes))
    host, dev = [], []
    for _, O, I in shapes:
        w, sc, bi = make_affine(rng, O, I, 4, 64)
        host.append((w, sc, bi))
        dev.append(AffineMatrix(to_dev(w, torch), to_dev(sc.view(np.int16), torch),
                                to_dev(bi.view(np.int16), torch), O, I, 4, 64))
    xb = make_x(rng, B, D)
    ab = make_x(rng, B, 4096)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    att = to_dev(ab.view(np.int16), torch).view(torch.bfloat16)
    sel = [i for i, (_, _, I) in enumerate(shapes) if I == D]
    outs = {}
    for dt in (torch.bfloat16, torch.float32):
        ys = affine_gemv_multi([dev[i] for i in sel], x, out_dtype=dt)
        for i, y in zip(sel, ys):
            outs[(i, dt)] = y.cpu()
        for i, (_, O, I) in enumerate(shapes):
            if I != D:
                outs[(i, dt)] = affine_gemv(dev[i], att, out_dtype=dt).cpu()
    xf, af = bf16_to_f32(xb), bf16_to_f32(ab)
    for i, (_, O, I) in enumerate(shapes):
        y16 = outs[(i, torch.bfloat16)].view(torch.int16).numpy().view(np.uint16)
        y32 = outs[(i, torch.float32)].numpy()
        check_rows(y16, y32, xf if I == D else af, host[i], O, I)


@pytest.mark.parametrize("B", [1, 32])
def test_config5_two_layer_stack(gpu, B):
    """Two layers of the stack back to back on one stream, with one shared
    workspace and output buffer as bench.py does: each layer's MoE output
    and routing against the oracle."""
    import torch
    from logan_amd.device import AffineMatrix, affine_gemv, affine_gemv_multi, moe_block

    from test_moe_gpu import Layer

    print(f"config5 stack B={B}", flush=True)
    moes = [Layer(torch, 512, 10, D, 512, 4, 64, seed=600 + l) for l in range(2)]
    rng = np.random.default_rng(700 + B)
    projs = []
    for l, shapes in enumerate((LIN_ATTN, FULL_ATTN)):
        m = []
        for _, O, I in shapes:
            w, sc, bi = make_affine(rng, O, I, 4, 64)
            m.append(AffineMatrix(to_dev(w, torch), to_dev(sc.view(np.int16), torch),
                                  to_dev(bi.view(np.int16), torch), O, I, 4, 64))
        projs.append((shapes, m))
    xb = make_x(rng, B, D)
    x = to_dev(xb.view(np.int16), torch).view(torch.bfloat16)
    att = to_dev(make_x(rng, B, 4096).view(np.int16), torch).view(torch.bfloat16)
    lgb = [make_logits(rng, B, 512) for _ in range(2)]
    ws = torch.empty(moes[0].dev.workspace_bytes(B), dtype=torch.uint8, device="cuda")
    mo = torch.empty((B, D), dtype=torch.float32, device="cuda")
    results = []
    for l, (shapes, m) in enumerate(projs):
        grp = [mm for (_, _, I), mm in zip(shapes, m) if I == D]
        affine_gemv_multi(grp, x)
        for (_, _, I), mm in zip(shapes, m):
            if I != D:
                affine_gemv(mm, att)
        lg = to_dev(lgb[l].view(np.int16), torch).view(torch.bfloat16)
        _, idx, _ = moe_block(moes[l].dev, x, lg, out=mo, workspace=ws, return_routing=True,
                              out_dtype=torch.float32)
        results.append((mo.cpu().numpy().copy(), idx.cpu().numpy()))
    xf = bf16_to_f32(xb)
    for l in range(2):
        out, idx = results[l]
        lf = bf16_to_f32(lgb[l])
        for t in range(B):
            ref, ridx, _ = moes[l].ref(xf[t], lf[t])
            np.testing.assert_array_equal(idx[t], ridx)
            assert normwise_rel(out[t], ref) <= 5e-5, f"layer {l} token {t}"
