"""The drop-in surface against logan-metal's own Rust FFI blocks
(logan-metal/src/lib.rs:198-481, :2795-2818, :3382-3585), CPU only.

tests/golden/ffi_symbols.json (written by tests/golden/make_ffi_symbols.py
from the reference's text) lists every function those blocks declare. The
library must export each name, include/logan_metal_ffi.h must declare each
with the C form of the Rust signature, and every declining entry must return
what the reference's non-macOS build hands its callers (nothing done, the
caller keeps its CPU path).
"""
import ctypes as C
import json
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
FIX = json.loads((Path(__file__).parent / "golden" / "ffi_symbols.json").read_text())
HDR = ROOT / "include" / "logan_metal_ffi.h"

RUST_TO_C = {"u16": "uint16_t", "i32": "int32_t", "i64": "int64_t", "u32": "uint32_t",
             "u64": "uint64_t", "usize": "size_t", "f32": "float", "f64": "double",
             "c_void": "void", "std::os::raw::c_void": "void", "std::os::raw::c_char": "char",
             "ColiMetalMatmulDescRaw": "ColiMetalMatmulDesc", "ColiMetalTensor": "ColiMetalTensor",
             "ColiMetalioRegion": "ColiMetalioRegion", "ColiMetalioStats": "ColiMetalioStats",
             "ColiApple8MetalioExpert": "ColiApple8MetalioExpert", "()": "void"}


def c_type(rust: str) -> str:
    rust = rust.strip()
    if rust.startswith("*mut "):
        return c_type(rust[5:]) + "*"
    if rust.startswith("*const "):
        return "const " + c_type(rust[7:]) + "*"
    return RUST_TO_C[rust]


def norm(c: str) -> str:
    c = re.sub(r"\s*\*\s*", "*", " ".join(c.split()))
    return c.strip()


def header_decls():
    text = re.sub(r"/\*.*?\*/", "", HDR.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(\w+)\s*\(([^;{]*?)\)\s*;", text, re.S):
        ret, name, params = m.group(1), m.group(2), m.group(3)
        plist = [] if params.strip() in ("", "void") else [p.strip() for p in params.split(",")]
        # drop the parameter name: the last identifier of each parameter
        ptypes = [norm(re.sub(r"\b\w+\s*$", "", p)) for p in plist]
        out[name] = (norm(ret), ptypes)
    return out


@pytest.fixture(scope="module")
def so():
    from logan_amd import _lib

    if not _lib.LIB_PATH.exists():
        from logan_amd import build

        build.build()
    return _lib.LIB_PATH


def test_fixture_is_the_whole_block():
    assert FIX["count"] == len(FIX["symbols"]) == 100
    names = [s["name"] for s in FIX["symbols"]]
    assert len(set(names)) == len(names)
    for must in ("coli_metal_matmul", "coli_metal_moe_route_begin", "coli_metal_llama_layer",
                 "coli_metal_silu_mul", "metalio_loadv", "coli_apple8_metalio_gdn_token"):
        assert must in names


def test_library_exports_every_reference_symbol(so):
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [s["name"] for s in FIX["symbols"] if s["name"] not in exported]
    assert not missing, f"not exported: {missing}"


def test_header_declares_the_reference_signatures():
    decls = header_decls()
    for s in FIX["symbols"]:
        assert s["name"] in decls, s["name"]
        ret, ptypes = decls[s["name"]]
        assert ret == norm(c_type(s["ret"])), (s["name"], ret)
        want = [norm(c_type(t)) for _, t in s["params"]]
        assert ptypes == want, (s["name"], ptypes, want)


def _ctype(rust: str):
    rust = rust.strip()
    if rust.startswith("*"):
        return C.c_void_p
    return {"u16": C.c_uint16, "i32": C.c_int32, "i64": C.c_int64, "u32": C.c_uint32,
            "u64": C.c_uint64, "usize": C.c_size_t, "f32": C.c_float, "f64": C.c_double,
            "()": None}[rust]


IMPLEMENTED = {"coli_metal_init", "coli_metal_available", "coli_metal_profile_set_on",
               "coli_metal_profile_reset", "coli_metal_profile_get", "coli_metal_matmul",
               "coli_metal_matmul_multi", "coli_metal_shared_mxfp4",
               "coli_metal_shared_mxfp4_drop_model", "coli_metal_rmsnorm", "coli_metal_add",
               "coli_metal_silu_mul", "coli_metal_tensor_free", "coli_metal_shutdown",
               "coli_metal_moe_route_begin", "coli_metal_moe_route_finish",
               "coli_metal_moe_route_discard", "coli_metal_moe_route_drop_model"}
ADVISORY = {"coli_metal_wrap_stats", "coli_metal_register", "coli_metal_unregister",
            "coli_metal_ptr_registered"}
# MetalIO failure values as its Rust callers test them (lib.rs:2890-2990, :3050, :3301)
MINUS_ONE = {"metalio_file_add", "metalio_slot_alloc", "metalio_slot_alloc_alias",
             "metalio_loadv", "metalio_wait", "metalio_batch_wait", "metalio_probe"}


def test_every_declining_entry_declines(so):
    """Called with null pointers and zero sizes: 0 / NULL / -1 as the
    reference's callers read a decline, and nothing else happens."""
    lib = C.CDLL(str(so))
    for s in FIX["symbols"]:
        name = s["name"]
        if name in IMPLEMENTED or name in ADVISORY:
            continue
        fn = getattr(lib, name)
        fn.restype = _ctype(s["ret"])
        fn.argtypes = [_ctype(t) for _, t in s["params"]]
        args = [None if a is C.c_void_p else 0 for a in fn.argtypes]
        got = fn(*args)
        if s["ret"] == "()":
            assert got is None
        elif s["ret"].startswith("*"):
            assert got is None, name
        else:
            assert got == (-1 if name in MINUS_ONE else 0), (name, got)


def test_advisory_registration(so):
    lib = C.CDLL(str(so))
    buf = (C.c_uint8 * 4096)()
    lib.coli_metal_register(buf, C.c_size_t(4096))
    lib.coli_metal_ptr_registered.restype = C.c_int32
    assert lib.coli_metal_ptr_registered(buf) == 0
    lib.coli_metal_unregister(buf)
    vals = [C.c_uint64(7) for _ in range(4)]
    lib.coli_metal_wrap_stats(*[C.byref(v) for v in vals])
    assert [v.value for v in vals] == [0, 0, 0, 0]


def test_regenerating_the_fixture_is_stable(tmp_path):
    """The generator reproduces the committed fixture when the reference is
    present (it reads the reference as text)."""
    ref = Path("/root/reference")
    if not (ref / "logan-metal" / "src" / "lib.rs").exists():
        pytest.skip("reference sources not present")
    import importlib.util

    spec = importlib.util.spec_from_file_location(
        "make_ffi_symbols", Path(__file__).parent / "golden" / "make_ffi_symbols.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    assert mod.extract(ref) == FIX["symbols"]
