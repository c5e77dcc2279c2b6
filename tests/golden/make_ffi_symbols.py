"""Write ffi_symbols.json: every function that logan-metal's Rust FFI blocks
declare (`unsafe extern "C" { ... }` in logan-metal/src/lib.rs), with its
parameter names, Rust types, return type and source line.

This reads the reference as text (it is not compiled or run). The fixture is
the drop-in contract: liblogan_hip.so must export each of these names
(tests/test_ffi_surface.py) and include/logan_metal_ffi.h must declare each
with the C equivalent of the Rust signature.

    python tests/golden/make_ffi_symbols.py [/root/reference]
"""
from __future__ import annotations

import json
import re
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = "logan-metal/src/lib.rs"


def _blocks(src: str):
    for m in re.finditer(r'unsafe extern "C" \{', src):
        start, depth, i = m.end(), 1, m.end()
        while depth:
            depth += {"{": 1, "}": -1}.get(src[i], 0)
            i += 1
        yield start, src[start:i - 1]


def _split_params(text: str):
    out = []
    for part in [p.strip() for p in text.split(",")]:
        if not part:
            continue
        name, ty = part.split(":", 1)
        out.append([name.strip(), " ".join(ty.split())])
    return out


def extract(ref_root: Path):
    src = (ref_root / SRC).read_text()
    syms = []
    for start, body in _blocks(src):
        line0 = src[:start].count("\n") + 1
        # strip line comments so that commented-out declarations do not count
        clean = re.sub(r"//[^\n]*", lambda m: " " * len(m.group(0)), body)
        for fm in re.finditer(r"(?:pub\s+)?fn\s+(\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+))?;", clean, re.S):
            syms.append({
                "name": fm.group(1),
                "line": line0 + clean[:fm.start()].count("\n"),
                "params": _split_params(fm.group(2)),
                "ret": " ".join(fm.group(3).split()) if fm.group(3) else "()",
            })
    return syms


def main() -> None:
    ref = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    syms = extract(ref)
    out = {"source": SRC, "count": len(syms), "symbols": syms}
    (HERE / "ffi_symbols.json").write_text(json.dumps(out, indent=1) + "\n")
    print(f"{len(syms)} symbols -> {HERE / 'ffi_symbols.json'}")


if __name__ == "__main__":
    main()
