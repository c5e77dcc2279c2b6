"""CPU-side checks of the C ABI: the library loads, exports every symbol the
headers declare, and its struct layouts match the Python mirror. No GPU
compute is issued here."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


@pytest.fixture(scope="module")
def so():
    from logan_amd import _lib

    if not _lib.LIB_PATH.exists():
        from logan_amd import build

        build.build()
    return _lib.LIB_PATH


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b((?:logan_hip|coli_metal)_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_both_layers():
    names = declared_functions()
    assert "logan_hip_moe_block" in names and "logan_hip_affine_gemv" in names
    assert "coli_metal_moe_route_begin" in names and "coli_metal_matmul" in names


def test_library_exports_every_declared_symbol(so):
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"not exported: {missing}"
    lib = C.CDLL(str(so))
    for n in declared_functions():
        getattr(lib, n)


def test_python_signatures_cover_the_abi(so):
    from logan_amd import _lib

    ours = {n for n in declared_functions() if n.startswith("logan_hip_")}
    bound = {n for n in _lib.SIGNATURES if n.startswith("logan_hip_")}
    assert ours == bound, ours ^ bound
    # the few logan-metal names bound directly are declared in the FFI header
    ffi = (ROOT / "include" / "logan_metal_ffi.h").read_text()
    for n in set(_lib.SIGNATURES) - bound:
        assert n + "(" in ffi, n


def test_struct_layouts_match_ctypes(tmp_path):
    """Compile a probe against include/logan_hip.h and compare sizeof/offsetof
    with the ctypes structures."""
    from logan_amd import _lib as L

    src = tmp_path / "probe.c"
    fields = {
        "LoganHipMatmulDesc": (L.MatmulDesc, [f[0] for f in L.MatmulDesc._fields_]),
        "LoganHipAffine": (L.Affine, [f[0] for f in L.Affine._fields_]),
        "LoganHipMxfp4": (L.Mxfp4, [f[0] for f in L.Mxfp4._fields_]),
        "LoganHipDense": (L.Dense, [f[0] for f in L.Dense._fields_]),
        "LoganHipLlamaLayer": (L.LlamaLayer, [f[0] for f in L.LlamaLayer._fields_]),
        "LoganHipAffineBank": (L.AffineBank, [f[0] for f in L.AffineBank._fields_]),
        "LoganHipMoeBlock": (L.MoeBlock, [f[0] for f in L.MoeBlock._fields_]),
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "logan_hip.h"', "int main(void){"]
    for cname, (_, names) in fields.items():
        lines.append(f'printf("{cname} %zu\\n", sizeof({cname}));')
        for n in names:
            lines.append(f'printf("{cname}.{n} %zu\\n", offsetof({cname}, {n}));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)],
                   check=True)
    got = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                         check=True).stdout.splitlines())
    for cname, (cls, names) in fields.items():
        assert int(got[cname]) == C.sizeof(cls), cname
        for n in names:
            assert int(got[f"{cname}.{n}"]) == getattr(cls, n).offset, f"{cname}.{n}"


def test_coli_desc_layout_matches_reference_declaration(tmp_path):
    """ColiMetalMatmulDesc as declared in logan-metal (backend_metal.h:68-88)
    restated field by field; the exported coli_metal_* symbols take it."""
    src = tmp_path / "coli.c"
    src.write_text("""
#include <stdio.h>
#include <stddef.h>
#include "logan_hip.h"
typedef struct ColiMetalMatmulDesc { void *tensor; float *y; const void *weights;
  const float *scales; int fmt; int I; int O; int gs; const float *x; int S; } ColiMetalMatmulDesc;
int main(void){
  printf("%d\\n", sizeof(ColiMetalMatmulDesc) == sizeof(LoganHipMatmulDesc)
    && offsetof(ColiMetalMatmulDesc, x) == offsetof(LoganHipMatmulDesc, x)
    && offsetof(ColiMetalMatmulDesc, S) == offsetof(LoganHipMatmulDesc, S)
    && offsetof(ColiMetalMatmulDesc, gs) == offsetof(LoganHipMatmulDesc, gs));
  return 0; }
""")
    exe = tmp_path / "coli"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)],
                   check=True)
    assert subprocess.run([str(exe)], capture_output=True, text=True).stdout.strip() == "1"


def test_fmt_mapping_matches_reference():
    """logan-metal/src/lib.rs:860-880 (bf16 16..19, fp16 21..24)."""
    from logan_amd.backend import mlx_affine_fmt

    assert [mlx_affine_fmt(b, False) for b in (4, 5, 6, 8)] == [16, 17, 18, 19]
    assert [mlx_affine_fmt(b, True) for b in (4, 5, 6, 8)] == [21, 22, 23, 24]
    assert mlx_affine_fmt(3, False) is None and mlx_affine_fmt(7, True) is None


def test_declines_without_a_device(so):
    """With no GPU every entry point declines with 0 / NULL and touches
    nothing (the reference's non-macOS stubs, logan-metal/src/lib.rs:4322-5069)."""
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from logan_amd import _lib as L

    lib = L.lib()
    assert lib.logan_hip_init() == 0
    assert lib.logan_hip_available() == 0
    y = (C.c_float * 4)()
    x = (C.c_float * 64)()
    w = (C.c_uint8 * 128)()
    a = (C.c_uint16 * 8)()
    t = C.c_void_p()
    assert lib.logan_hip_matmul(C.byref(t), y, x, w, a, 16, 1, 64, 4, 64) == 0
    assert t.value is None
    d = (L.MatmulDesc * 3)()
    assert lib.logan_hip_moe_route_begin(0, 0, d, 1, x, 64, 64) is None
    assert lib.logan_hip_moe_route_finish(None, y, 1) == 0
    assert lib.logan_hip_shared_expert(0, 0, d, 3, x, y, 64, 64) == 0
    assert lib.logan_hip_matmul_multi(x, 1, d, 0) == 0
    assert lib.logan_hip_matmul_multi(x, 1, d, 17) == 0


def test_integration_build_rs_builds_every_source():
    """INTEGRATION.md's build.rs compiles what logan_amd/build.py compiles:
    the same source directory and extension filter (so every csrc/*.hip,
    not a fixed list that can drift), include path and hipcc flags."""
    from logan_amd import build

    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```rust\n(.*?)```", text, flags=re.S)
    snip = [b for b in blocks if "build.rs" in b]
    assert len(snip) == 1
    rs = snip[0]
    consts = dict(re.findall(r'const (CSRC|INCLUDE): &str = "([^"]+)";', rs))
    assert (ROOT / consts["CSRC"]).resolve() == build.CSRC
    assert (ROOT / consts["INCLUDE"]).resolve() == build.INCLUDE
    flags = re.search(r"const HIPFLAGS: &\[&str\] = &\[(.*?)\];", rs, flags=re.S).group(1)
    assert re.findall(r'"([^"]+)"', flags) == build.HIPFLAGS
    # sources: read_dir(CSRC) filtered on the .hip extension, as build.py's glob
    assert "fs::read_dir(CSRC)" in rs and 'x == "hip"' in rs
    assert ".args(HIPFLAGS)" in rs and ".arg(INCLUDE)" in rs
    srcs = sorted(p.name for p in build.CSRC.glob("*.hip"))
    assert "ffi.hip" in srcs and "abi.hip" in srcs and len(srcs) >= 10
