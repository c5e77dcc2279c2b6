"""CPU oracle for the checkpoint loader — TEST INFRASTRUCTURE ONLY.

A pure-Python restatement of the reference's safetensors reader and MLX
quantized loaders, returning the exact bytes the reference would hold and the
exact error text it would return:

* parse_shard                    logan-qwen4/src/lib.rs:326-421
* element_bytes                  lib.rs:437-447
* register (engine aliases)      lib.rs:460-503 (the in-layer PLE alias is
                                 not part of the quantized path and is left out)
* StFile::open / open_dir        lib.rs:508-595
* payload / payload_range        lib.rs:686-760
* load_mlx_quantized_wt          lib.rs:11818-11937
* load_mlx_quantized_expert_wt   lib.rs:11939-12078

Only tests/ use it, as the checker of logan_amd's C loader. Pinning
(tests/test_checkpoint.py): the reference's own two checkpoint tests
(lib.rs:16870-16985) as vectors, the `safetensors` package's reader on files
it wrote (an independent parser of the same format), and the invariant that
the E one-expert slices of a stacked bank concatenate to the whole payload.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple


class StError(Exception):
    pass


def element_bytes(dtype: str) -> Optional[int]:
    return {"F32": 4, "I32": 4, "U32": 4, "BF16": 2, "F16": 2, "U8": 1, "F8_E4M3": 1,
            "F8_E4M3FN": 1, "I64": 8}.get(dtype)


def _u64(v) -> Optional[int]:
    if isinstance(v, bool) or not isinstance(v, int) or v < 0 or v >= 1 << 64:
        return None
    return v


def _shape(s: List[int]) -> str:
    return "[" + ", ".join(str(d) for d in s) + "]"


def parse_shard(path: str) -> List[Tuple[str, List[int], str, int, int]]:
    with open(path, "rb") as f:
        raw = f.read()
    file_len = len(raw)
    if file_len < 8:
        raise StError(f"{path}: failed to fill whole buffer")
    n = struct.unpack("<Q", raw[:8])[0]
    data_start = 8 + n
    if data_start > file_len:
        raise StError(f"{path}: header extends past EOF ({data_start} > {file_len})")
    try:
        header = json.loads(raw[8:data_start])
    except ValueError as e:
        raise StError(f"{path}: {e}")
    if not isinstance(header, dict):
        raise StError(f"{path}: header is not an object")
    out = []
    for name in sorted(header):
        if name == "__metadata__":
            continue
        spec = header[name]
        spec = spec if isinstance(spec, dict) else {}
        dtype = spec.get("dtype")
        if not isinstance(dtype, str):
            raise StError(f"{name}: missing dtype")
        if element_bytes(dtype) is None:
            raise StError(f"{name}: unsupported dtype `{dtype}` (supported: F32, I32, I64, U32, "
                          f"U8, BF16, F16, F8_E4M3, F8_E4M3FN)")
        shape = spec.get("shape")
        if not isinstance(shape, list):
            raise StError(f"{name}: missing shape")
        dims = []
        for v in shape:
            u = _u64(v)
            if u is None:
                raise StError(f"{name}: invalid shape")
            dims.append(u)
        offs = spec.get("data_offsets")
        if not isinstance(offs, list):
            raise StError(f"{name}: missing data_offsets")
        if len(offs) != 2:
            raise StError(f"{name}: invalid data_offsets")
        begin, end = _u64(offs[0]), _u64(offs[1])
        if begin is None:
            raise StError(f"{name}: invalid start offset")
        if end is None:
            raise StError(f"{name}: invalid end offset")
        if end < begin or data_start + end > file_len:
            raise StError(f"{name}: tensor range is outside {path}")
        elems = 1
        for d in dims:
            elems = min(elems * d, (1 << 64) - 1)
        elems = max(elems, 1)
        expected = min(elems * element_bytes(dtype), (1 << 64) - 1)
        if end - begin != expected:
            raise StError(f'{name}: span {end - begin} != {elems} x "{dtype}" = {expected}')
        out.append((name, dims, dtype, data_start + begin, end - begin))
    return out


@dataclass
class StFile:
    paths: List[str] = field(default_factory=list)
    # name -> (shard, shape, dtype, abs offset, len)
    tensors: Dict[str, Tuple[int, List[int], str, int, int]] = field(default_factory=dict)

    def _register(self, shard, name, shape, dtype, off, ln):
        for pre, to in (("model.language_model.", "model."), ("language_model.model.", "model."),
                        ("language_model.lm_head.", "lm_head.")):
            if name.startswith(pre):
                alias = to + name[len(pre):]
                if alias not in self.tensors:
                    self.tensors[alias] = (shard, shape, dtype, off, ln)
        self.tensors[name] = (shard, shape, dtype, off, ln)

    @classmethod
    def open(cls, path: str) -> "StFile":
        st = cls([str(path)])
        for name, shape, dtype, off, ln in parse_shard(str(path)):
            st.tensors[name] = (0, shape, dtype, off, ln)
        return st

    @classmethod
    def open_dir(cls, d: str) -> "StFile":
        d = str(d)
        st = cls()
        index = os.path.join(d, "model.safetensors.index.json")
        if os.path.isfile(index):
            try:
                with open(index, "rb") as f:
                    value = json.loads(f.read())
            except ValueError as e:
                raise StError(f"{index}: {e}")
            wm = value.get("weight_map") if isinstance(value, dict) else None
            if not isinstance(wm, dict):
                raise StError(f"{index}: missing weight_map")
            shards = sorted({v for v in wm.values() if isinstance(v, str)})
            for i, sh in enumerate(shards):
                p = os.path.join(d, sh)
                ents = parse_shard(p)
                st.paths.append(p)
                for name, shape, dtype, off, ln in ents:
                    st._register(i, name, shape, dtype, off, ln)
            if not st.tensors:
                raise StError(f"{index}: weight_map names no tensors")
        else:
            single = os.path.join(d, "model.safetensors")
            if not os.path.isfile(single):
                raise StError(f"{d}: neither model.safetensors.index.json nor model.safetensors")
            st.paths.append(single)
            for name, shape, dtype, off, ln in parse_shard(single):
                st._register(0, name, shape, dtype, off, ln)
        return st

    def shard_count(self) -> int:
        return len(self.paths)

    def dtype_counts(self) -> Dict[str, int]:
        seen, out = set(), {}
        for shard, _s, dtype, off, ln in self.tensors.values():
            if (shard, off, ln) not in seen:
                seen.add((shard, off, ln))
                out[dtype] = out.get(dtype, 0) + 1
        return out

    def shape_of(self, name: str) -> Optional[List[int]]:
        t = self.tensors.get(name)
        return None if t is None else list(t[1])

    def payload(self, name: str) -> bytes:
        t = self.tensors.get(name)
        if t is None:
            raise StError(f"missing tensor {name}")
        return self.payload_range(name, 0, t[4])

    def payload_range(self, name: str, within: int, ln: int) -> bytes:
        t = self.tensors.get(name)
        if t is None:
            raise StError(f"missing tensor {name}")
        shard, _s, _d, off, total = t
        if within + ln > total:
            raise StError(f"{name}: requested byte range {within}..{within + ln} exceeds payload "
                          f"length {total}")
        with open(self.paths[shard], "rb") as f:
            f.seek(off + within)
            return f.read(ln)


@dataclass
class QuantWt:
    kind: str  # "affine" | "mxfp4"
    bits: int
    group_size: int
    aux_fp16: bool
    weights: bytes
    scales: bytes
    biases: bytes  # b"" for MXFP4


def load_mlx_quantized_wt(st: StFile, name: str, o: int, i: int) -> QuantWt:
    if o == 0 or i == 0:
        raise StError(f"{name}: quantized matrix dimensions must be non-zero")
    t = st.tensors.get(name)
    if t is None:
        raise StError(f"missing tensor {name}")
    _, wshape, wdtype, _, _ = t
    if wdtype != "U32" or len(wshape) != 2 or wshape[0] != o:
        raise StError(f"{name}: expected U32 packed matrix with {o} rows, got "
                      f"{wdtype}/{_shape(wshape)}")
    words = wshape[1]
    row_bits = words * 32
    if row_bits % i:
        raise StError(f"{name}: {words} U32 words cannot represent {i} logical columns exactly")
    bits = row_bits // i
    if bits > 255:
        raise StError(f"{name}: inferred bit width overflows u8")
    if bits not in (4, 5, 6, 8):
        raise StError(f"{name}: inferred unsupported MLX quantization width {bits} from "
                      f"{_shape(wshape)} -> {o}x{i}")
    if not name.endswith(".weight"):
        raise StError(f"{name}: quantized matrix name must end in .weight")
    base = name[: -len(".weight")]
    sname = f"{base}.scales"
    s = st.tensors.get(sname)
    if s is None:
        raise StError(f"missing quantization sidecar {sname}")
    weights = st.payload(name)
    _, sshape, sdtype, _, _ = s
    if sdtype in ("BF16", "F16"):
        if len(sshape) != 2 or sshape[0] != o or sshape[1] == 0:
            raise StError(f"{sname}: expected [rows, groups] BF16/F16 scales for {o} rows, got "
                          f"{sdtype}/{_shape(sshape)}")
        groups = sshape[1]
        if i % groups:
            raise StError(f"{sname}: {groups} groups do not divide {i} logical columns")
        bname = f"{base}.biases"
        b = st.tensors.get(bname)
        if b is None:
            raise StError(f"missing affine quantization sidecar {bname}")
        if b[2] != sdtype or b[1] != sshape:
            raise StError(f"{bname}: expected {sdtype} shape {_shape(sshape)}, got "
                          f"{b[2]}/{_shape(b[1])}")
        return QuantWt("affine", bits, i // groups, sdtype == "F16", weights, st.payload(sname),
                       st.payload(bname))
    if sdtype == "U8":
        if bits != 4:
            raise StError(f"{name}: U8 scale sidecar identifies MLX MXFP4, but inferred weight "
                          f"width is {bits}")
        want = (i + 31) // 32
        if sshape != [o, want]:
            raise StError(f"{sname}: expected MLX MXFP4 scale shape [{o}, {want}], got "
                          f"{_shape(sshape)}")
        return QuantWt("mxfp4", 4, 32, False, weights, st.payload(sname), b"")
    raise StError(f"{sname}: unsupported MLX quantization scale dtype {sdtype}; expected "
                  f"BF16/F16 affine or U8 MXFP4")


def load_mlx_quantized_expert_wt(st: StFile, name: str, expert: int, experts: int, o: int,
                                 i: int) -> QuantWt:
    if expert >= experts or o == 0 or i == 0:
        raise StError(f"{name}: invalid expert geometry expert={expert}/{experts} matrix={o}x{i}")
    t = st.tensors.get(name)
    if t is None:
        raise StError(f"missing tensor {name}")
    _, wshape, wdtype, _, _ = t
    if wdtype != "U32" or len(wshape) != 3 or wshape[0] != experts or wshape[1] != o:
        raise StError(f"{name}: expected stacked U32 [{experts}, {o}, words], got "
                      f"{wdtype}/{_shape(wshape)}")
    words = wshape[2]
    row_bits = words * 32
    if row_bits % i:
        raise StError(f"{name}: {words} U32 words cannot represent {i} logical columns exactly")
    bits = row_bits // i
    if bits > 255:
        raise StError(f"{name}: inferred bit width overflows u8")
    if bits not in (4, 5, 6, 8):
        raise StError(f"{name}: unsupported MLX expert bit width {bits}")
    if not name.endswith(".weight"):
        raise StError(f"{name}: quantized expert name must end in .weight")
    base = name[: -len(".weight")]
    sname = f"{base}.scales"
    s = st.tensors.get(sname)
    if s is None:
        raise StError(f"missing expert sidecar {sname}")
    _, sshape, sdtype, _, _ = s
    if len(sshape) != 3 or sshape[0] != experts or sshape[1] != o or sshape[2] == 0:
        raise StError(f"{sname}: expected [{experts}, {o}, groups], got {_shape(sshape)}")
    groups = sshape[2]
    if i % groups:
        raise StError(f"{sname}: {groups} groups do not divide {i} logical columns")
    gs = i // groups
    wslice = o * words * 4
    weights = st.payload_range(name, expert * wslice, wslice)
    if sdtype in ("BF16", "F16"):
        pslice = o * groups * 2
        bname = f"{base}.biases"
        b = st.tensors.get(bname)
        if b is None:
            raise StError(f"missing affine expert sidecar {bname}")
        if b[2] != sdtype or b[1] != sshape:
            raise StError(f"{bname}: expected {sdtype} shape {_shape(sshape)}, got "
                          f"{b[2]}/{_shape(b[1])}")
        return QuantWt("affine", bits, gs, sdtype == "F16", weights,
                       st.payload_range(sname, expert * pslice, pslice),
                       st.payload_range(bname, expert * pslice, pslice))
    if sdtype == "U8":
        if bits != 4 or gs != 32:
            raise StError(f"{name}: MLX MXFP4 expert requires 4-bit/group-32, got "
                          f"{bits}-bit/group-{gs}")
        sslice = o * groups
        return QuantWt("mxfp4", 4, 32, False, weights,
                       st.payload_range(sname, expert * sslice, sslice), b"")
    raise StError(f"{sname}: unsupported MLX expert scale dtype {sdtype}")


def write_checkpoint(path: str, tensors, metadata: Optional[dict] = None) -> None:
    """One safetensors file from [(name, dtype, shape, payload bytes)], laid
    out in the given order (the reference tests' writer, lib.rs:16819-16858)."""
    header, payload = {}, bytearray()
    for name, dtype, shape, data in tensors:
        b = len(payload)
        payload += data
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [b, len(payload)]}
    if metadata is not None:
        header["__metadata__"] = metadata
    hb = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        f.write(payload)


def write_sharded_checkpoint(d: str, shards) -> str:
    """shards: [(file name, [(name, dtype, shape, payload)])] plus the index
    naming every tensor's file."""
    os.makedirs(d, exist_ok=True)
    wm = {}
    for fname, tensors in shards:
        write_checkpoint(os.path.join(d, fname), tensors)
        for t in tensors:
            wm[t[0]] = fname
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": wm}, f)
    return d
