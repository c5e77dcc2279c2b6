"""logan-hip: MI355X (gfx950) backend for Logan's quantized decode hot path.

* `logan_amd.backend` — host-pointer drop-in mirroring logan-metal's Rust
  surface (hip_matmul_mlx_affine, moe_route_begin/finish, shared_expert, ...).
* `logan_amd.device` — HBM-resident bf16 entry points (affine_gemv,
  route_topk, moe_block) taking torch device tensors as plumbing.
* `logan_amd.synth` — seeded synthetic inputs in the benchmark's data scheme.

All arithmetic runs in liblogan_hip.so (hand-written HIP for gfx950); the
package raises if that library is missing.
"""
from . import _lib  # noqa: F401

__all__ = ["backend", "device", "synth", "lib", "version"]


def lib():
    return _lib.lib()


def version() -> str:
    return _lib.lib().logan_hip_version().decode()
