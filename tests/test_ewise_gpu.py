"""GPU parity of the dense SwiGLU element-wise op (logan_hip_silu_mul)
against the oracle's restatement of moe_silu
(logan-metal/metal/backend_metal.mm:698-699).

Bars: f32 within 4e-6 relative per element (the device exp and the C
library's expf may differ by a few ulp); bf16 within one bf16 ulp of the
RNE-rounded oracle value; ragged lengths (tails not a multiple of 8).
"""
import numpy as np
import pytest

import oracle
from logan_amd.synth import bf16_bits, bf16_to_f32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 7, 8, 1000, 14336, 8 * 14336 + 3])
def test_silu_mul_f32(gpu, n):
    import torch
    from logan_amd.device import silu_mul

    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 3).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    gd, ud = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    silu_mul(gd, ud)
    got = gd.cpu().numpy()
    ref = oracle.silu_mul(g, u)
    assert np.all(np.abs(got - ref) <= 4e-6 * np.abs(ref) + 1e-30)
    assert np.array_equal(ud.cpu().numpy(), u)


@pytest.mark.parametrize("n", [5, 8, 4096, 8 * 14336 + 1])
def test_silu_mul_bf16(gpu, n):
    import torch
    from logan_amd.device import silu_mul

    rng = np.random.default_rng(100 + n)
    gb = bf16_bits((rng.standard_normal(n) * 3).astype(np.float32))
    ub = bf16_bits(rng.standard_normal(n).astype(np.float32))
    gd = torch.from_numpy(gb.view(np.int16)).cuda().view(torch.bfloat16)
    ud = torch.from_numpy(ub.view(np.int16)).cuda().view(torch.bfloat16)
    silu_mul(gd, ud)
    got = gd.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = bf16_bits(oracle.silu_mul(bf16_to_f32(gb), bf16_to_f32(ub)))
    # same sign and magnitude within one unit of the last bf16 place
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    zero = (got & 0x7fff) == 0
    assert np.all((diff <= 1) | (zero & ((ref & 0x7fff) <= 1)))
