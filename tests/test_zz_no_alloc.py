"""logan_hip_moe_block_static (the MoE block on the library's static device
scratch, allocating nothing) against logan_hip_moe_block with a caller
workspace, through the C ABI: two calls in a row, the second smaller, for
each path (MFMA token batch then per-token; per-token then single-launch
B=1); outputs and routing bit-identical, and the same as the oracle. A call
whose workspace exceeds the static scratch is rejected with 0."""
import numpy as np
import pytest

from logan_amd.synth import bf16_to_f32, make_logits, make_x

from _util import normwise_rel

pytestmark = pytest.mark.gpu


def _run(torch, layer, xb, lb, static):
    from logan_amd.device import moe_block, moe_block_static

    x = torch.from_numpy(xb.view(np.int16)).cuda().view(torch.bfloat16)
    lg = torch.from_numpy(lb.view(np.int16)).cuda().view(torch.bfloat16)
    if static:
        out, idx, w = moe_block_static(layer.dev, x, lg, return_routing=True,
                                       out_dtype=torch.float32)
    else:
        ws = torch.empty(layer.dev.workspace_bytes(xb.shape[0]), dtype=torch.uint8, device="cuda")
        out, idx, w = moe_block(layer.dev, x, lg, workspace=ws, return_routing=True,
                                out_dtype=torch.float32)
    torch.cuda.synchronize()
    return out.cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("sizes", [(64, 16), (16, 1), (1, 1)])
def test_static_scratch_matches_workspace_entry(gpu, sizes):
    import torch

    from test_moe_gpu import Layer

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=91)
    rng = np.random.default_rng(92 + sizes[0])
    for B in sizes:
        print(f"no-alloc moe B={B}", flush=True)
        xb = make_x(rng, B, 2048)
        lb = make_logits(rng, B, 512)
        o1, i1, w1 = _run(torch, layer, xb, lb, static=True)
        o0, i0, w0 = _run(torch, layer, xb, lb, static=False)
        np.testing.assert_array_equal(i1, i0)
        np.testing.assert_array_equal(w1, w0)
        np.testing.assert_array_equal(o1, o0)
        xf, lf = bf16_to_f32(xb), bf16_to_f32(lb)
        for t in range(min(B, 4)):
            ref, ridx, _ = layer.ref(xf[t], lf[t])
            np.testing.assert_array_equal(i1[t], ridx)
            assert normwise_rel(o1[t], ref) <= 5e-5


def test_static_scratch_rejects_oversized_batches(gpu):
    import torch
    from logan_amd import _lib
    from logan_amd.device import LoganHipError, moe_block_static

    from test_moe_gpu import Layer

    layer = Layer(torch, 512, 10, 2048, 512, 4, 64, seed=93)
    B = 1024  # needs ~114 MB of workspace
    assert layer.dev.workspace_bytes(B) > (64 << 20)
    x = torch.zeros((B, 2048), dtype=torch.bfloat16, device="cuda")
    lg = torch.zeros((B, 512), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(LoganHipError):
        moe_block_static(layer.dev, x, lg)
    assert _lib.lib().logan_hip_moe_sync_errors() == 0
