"""Checkpoint loader, CPU side: the oracle's restatement of the reference
reader pinned by the reference's own checkpoint tests and by the
`safetensors` package's independent reader; then logan-hip's C parser and
quantized-load planner compared with the oracle on valid and malformed
checkpoints (same tensors, same bytes, same error text). Nothing here
touches a GPU: the planner validates and sizes without allocating."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from oracle import checkpoint as ock

# ---------------------------------------------------------------- helpers


def bf16(v: float) -> bytes:
    """The reference tests' truncating bf16 (lib.rs:16860-16863)."""
    return struct.pack("<H", struct.unpack("<I", struct.pack("<f", v))[0] >> 16)


def bf16_val(b: bytes) -> float:
    return struct.unpack("<f", struct.pack("<I", struct.unpack("<H", b)[0] << 16))[0]


def u32s(*ws) -> bytes:
    return b"".join(struct.pack("<I", w) for w in ws)


@pytest.fixture(scope="module")
def ck():
    from logan_amd import _lib

    if not _lib.LIB_PATH.exists():
        from logan_amd import build

        build.build()
    from logan_amd import checkpoint

    return checkpoint


def shard_alias_dir(tmp_path):
    """lib.rs:16870-16918: two shards, the backbone under the HF prefix."""
    return ock.write_sharded_checkpoint(str(tmp_path / "alias"), [
        ("model-00001-of-00002.safetensors",
         [("model.language_model.embed_tokens.weight", "BF16", [2], bf16(1.5) + bf16(-0.5))]),
        ("model-00002-of-00002.safetensors",
         [("model.language_model.layers.0.mlp.gate.weight", "BF16", [1], bf16(-2.25))]),
    ])


def mlx_alias_dir(tmp_path):
    """lib.rs:16920-16985: MLX-prefixed quantized payloads across shards."""
    return ock.write_sharded_checkpoint(str(tmp_path / "mlx"), [
        ("model-00001-of-00002.safetensors", [
            ("language_model.model.layers.0.linear_attn.in_proj_a.weight", "U32", [1, 2],
             u32s(0x01234567, 0x89ABCDEF)),
            ("language_model.model.layers.0.linear_attn.in_proj_a.scales", "BF16", [1, 1],
             bf16(0.5)),
            ("language_model.model.layers.0.linear_attn.in_proj_a.biases", "BF16", [1, 1],
             bf16(-1.0)),
        ]),
        ("model-00002-of-00002.safetensors", [
            ("language_model.model.layers.0.mlp.switch_mlp.gate_proj.scales", "U8", [1, 1, 1],
             bytes([127])),
        ]),
    ])


# ------------------------------------------------ oracle pinning (reference tests)


def test_oracle_reference_shard_alias_test(tmp_path):
    st = ock.StFile.open_dir(shard_alias_dir(tmp_path))
    assert st.shard_count() == 2
    assert st.dtype_counts().get("BF16") == 2
    via_hf = st.payload("model.language_model.layers.0.mlp.gate.weight")
    via_engine = st.payload("model.layers.0.mlp.gate.weight")
    assert bf16_val(via_hf) == -2.25 and via_hf == via_engine
    emb = st.payload("model.embed_tokens.weight")
    assert (bf16_val(emb[:2]), bf16_val(emb[2:])) == (1.5, -0.5)


def test_oracle_reference_mlx_alias_test(tmp_path):
    st = ock.StFile.open_dir(mlx_alias_dir(tmp_path))
    assert st.dtype_counts().get("U32") == 1 and st.dtype_counts().get("U8") == 1
    assert st.shape_of("model.layers.0.linear_attn.in_proj_a.weight") == [1, 2]
    assert st.shape_of("model.layers.0.linear_attn.in_proj_a.scales") == [1, 1]
    assert st.shape_of("model.layers.0.linear_attn.in_proj_a.biases") == [1, 1]


def _safetensors_file(tmp_path, rng):
    from safetensors.numpy import save_file

    arrs = {
        "a.weight": rng.integers(0, 2**32, (6, 16), dtype=np.uint32),
        "a.scales": rng.integers(0, 2**16, (6, 2), dtype=np.uint16).view(np.float16),
        "b": rng.standard_normal((3, 5)).astype(np.float32),
        "c": rng.integers(0, 256, (7,), dtype=np.uint8),
        "d": rng.integers(-9, 9, (2, 2, 2), dtype=np.int64),
        "e": rng.integers(-9, 9, (4,), dtype=np.int32),
    }
    p = str(tmp_path / "np.safetensors")
    save_file(arrs, p, metadata={"format": "np"})
    return p, arrs


def test_oracle_reader_agrees_with_the_safetensors_package(tmp_path):
    """An independent reader of the same format: every tensor's shape, dtype
    and bytes as the package wrote them."""
    rng = np.random.default_rng(3)
    p, arrs = _safetensors_file(tmp_path, rng)
    st = ock.StFile.open(p)
    names = {"float32": "F32", "float16": "F16", "uint32": "U32", "uint8": "U8", "int64": "I64",
             "int32": "I32"}
    for k, a in arrs.items():
        t = st.tensors[k]
        assert t[1] == list(a.shape) and t[2] == names[a.dtype.name]
        assert st.payload(k) == a.tobytes()


def test_oracle_expert_slices_tile_the_bank(tmp_path):
    """The E one-expert slices of each stacked tensor concatenate to the
    whole payload, and each slice's codes/params are that expert's rows."""
    rng = np.random.default_rng(4)
    E, O, I, bits, gs = 5, 6, 64, 5, 32
    words = I * bits // 32
    w = rng.integers(0, 2**32, (E, O, words), dtype=np.uint32)
    sc = rng.integers(0, 2**16, (E, O, I // gs), dtype=np.uint16)
    bi = rng.integers(0, 2**16, (E, O, I // gs), dtype=np.uint16)
    p = str(tmp_path / "bank.safetensors")
    ock.write_checkpoint(p, [("m.weight", "U32", [E, O, words], w.tobytes()),
                             ("m.scales", "BF16", [E, O, I // gs], sc.tobytes()),
                             ("m.biases", "BF16", [E, O, I // gs], bi.tobytes())])
    st = ock.StFile.open(p)
    parts = [ock.load_mlx_quantized_expert_wt(st, "m.weight", e, E, O, I) for e in range(E)]
    assert b"".join(q.weights for q in parts) == w.tobytes()
    assert b"".join(q.scales for q in parts) == sc.tobytes()
    assert b"".join(q.biases for q in parts) == bi.tobytes()
    for e, q in enumerate(parts):
        assert q.weights == w[e].tobytes() and q.bits == bits and q.group_size == gs


def test_oracle_rejects_a_planted_slice_error(tmp_path):
    """A mistake planted in the oracle's expert offset (expert e reads e+1's
    rows) fails the tiling invariant above: the check can fail."""
    rng = np.random.default_rng(5)
    E, O, I = 3, 4, 64
    w = rng.integers(0, 2**32, (E, O, I // 8), dtype=np.uint32)
    sc = rng.integers(0, 2**16, (E, O, 1), dtype=np.uint16)
    p = str(tmp_path / "b.safetensors")
    ock.write_checkpoint(p, [("m.weight", "U32", [E, O, I // 8], w.tobytes()),
                             ("m.scales", "BF16", [E, O, 1], sc.tobytes()),
                             ("m.biases", "BF16", [E, O, 1], sc.tobytes())])
    st = ock.StFile.open(p)
    wslice = O * (I // 8) * 4
    planted = [st.payload_range("m.weight", min(e + 1, E - 1) * wslice, wslice) for e in range(E)]
    assert b"".join(planted) != w.tobytes()


# ------------------------------------------------ the C reader against the oracle


def test_reference_shard_alias_test_through_logan_hip(ck, tmp_path):
    d = shard_alias_dir(tmp_path)
    with ck.StFile.open_dir(d) as st:
        assert st.shard_count() == 2
        assert st.dtype_counts().get("BF16") == 2
        via_hf = st.payload("model.language_model.layers.0.mlp.gate.weight")
        assert bf16_val(via_hf) == -2.25
        assert st.payload("model.layers.0.mlp.gate.weight") == via_hf
        emb = st.payload("model.embed_tokens.weight")
        assert (bf16_val(emb[:2]), bf16_val(emb[2:])) == (1.5, -0.5)


def test_reference_mlx_alias_test_through_logan_hip(ck, tmp_path):
    with ck.StFile.open_dir(mlx_alias_dir(tmp_path)) as st:
        assert st.dtype_counts() == {"U32": 1, "U8": 1, "BF16": 2}
        assert st.shape_of("model.layers.0.linear_attn.in_proj_a.weight") == [1, 2]
        assert st.shape_of("model.layers.0.linear_attn.in_proj_a.scales") == [1, 1]
        assert st.shape_of("model.layers.0.linear_attn.in_proj_a.biases") == [1, 1]
        assert st.shape_of("model.layers.0.mlp.switch_mlp.gate_proj.scales") == [1, 1, 1]
        assert st.dtype_of("model.layers.0.mlp.switch_mlp.gate_proj.scales") == "U8"


def test_c_reader_agrees_with_the_safetensors_package(ck, tmp_path):
    rng = np.random.default_rng(6)
    p, arrs = _safetensors_file(tmp_path, rng)
    with ck.StFile.open(p) as st:
        assert st.shard_count() == 1
        for k, a in arrs.items():
            assert st.shape_of(k) == list(a.shape)
            assert st.payload(k) == a.tobytes()
            n = a.nbytes
            assert st.payload_range(k, n // 3, n - n // 3) == a.tobytes()[n // 3:]
        with pytest.raises(ck.CheckpointError, match=r"^b: requested byte range 4\.\.64 exceeds "
                                                     r"payload length 60$"):
            st.payload_range("b", 4, 60)
        assert st.shape_of("nope") is None


def _raw_file(path, header, payload=b"", hlen=None):
    hb = header if isinstance(header, bytes) else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb) if hlen is None else hlen))
        f.write(hb)
        f.write(payload)
    return str(path)


BAD_HEADERS = [
    ("past_eof", None, 10**6),
    ("not_object", [1, 2], None),
    ("no_dtype", {"t": {"shape": [1], "data_offsets": [0, 4]}}, None),
    ("bad_dtype", {"t": {"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}}, None),
    ("no_shape", {"t": {"dtype": "F32", "data_offsets": [0, 4]}}, None),
    ("neg_shape", {"t": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, None),
    ("float_shape", {"t": {"dtype": "F32", "shape": [1.0], "data_offsets": [0, 4]}}, None),
    ("no_offsets", {"t": {"dtype": "F32", "shape": [1]}}, None),
    ("three_offsets", {"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4, 8]}}, None),
    ("bad_start", {"t": {"dtype": "F32", "shape": [1], "data_offsets": ["0", 4]}}, None),
    ("bad_end", {"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, -4]}}, None),
    ("reversed", {"t": {"dtype": "F32", "shape": [1], "data_offsets": [8, 4]}}, None),
    ("outside", {"t": {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]}}, None),
    ("span", {"t": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 16]}}, None),
    ("zero_dim_span", {"t": {"dtype": "BF16", "shape": [0, 4], "data_offsets": [0, 0]}}, None),
]


@pytest.mark.parametrize("case,header,hlen", BAD_HEADERS, ids=[c[0] for c in BAD_HEADERS])
def test_malformed_headers_fail_as_the_reference_does(ck, tmp_path, case, header, hlen):
    p = _raw_file(tmp_path / f"{case}.safetensors", header if header is not None else {},
                  b"\0" * 16, hlen)
    with pytest.raises(ock.StError) as want:
        ock.StFile.open(p)
    with pytest.raises(ck.CheckpointError) as got:
        ck.StFile.open(p)
    assert str(got.value) == str(want.value), case


def test_duplicate_keys_and_metadata(ck, tmp_path):
    """The last duplicate wins and __metadata__ is skipped, as serde_json
    reads the header."""
    hb = (b'{"__metadata__":{"k":"v"},"t":{"dtype":"U8","shape":[1],"data_offsets":[0,1]},'
          b'"t":{"dtype":"U8","shape":[2],"data_offsets":[1,3]}}')
    p = _raw_file(tmp_path / "dup.safetensors", hb, b"\x01\x02\x03")
    for st in (ock.StFile.open(p), ck.StFile.open(p)):
        assert st.shape_of("t") == [2]
        assert st.payload("t") == b"\x02\x03"
        assert st.shape_of("__metadata__") is None


def test_directory_errors(ck, tmp_path):
    empty = tmp_path / "empty"
    empty.mkdir()
    for opener in (ock.StFile.open_dir, ck.StFile.open_dir):
        with pytest.raises(Exception, match="neither model.safetensors.index.json nor "
                                            "model.safetensors"):
            opener(str(empty))
    noidx = tmp_path / "noidx"
    noidx.mkdir()
    (noidx / "model.safetensors.index.json").write_text('{"metadata": {}}')
    for opener in (ock.StFile.open_dir, ck.StFile.open_dir):
        with pytest.raises(Exception, match="missing weight_map$"):
            opener(str(noidx))
    single = tmp_path / "single"
    single.mkdir()
    ock.write_checkpoint(str(single / "model.safetensors"),
                         [("language_model.lm_head.weight", "U8", [1], b"\x07")])
    with ck.StFile.open_dir(str(single)) as st:
        assert st.payload("lm_head.weight") == b"\x07"


# ------------------------------------------------ quantized-load planning


def quant_checkpoint(path, rng):
    """Tensors covering every accept and reject branch of the two loaders."""
    T = []

    def aff(name, O, I, bits, gs, sdt="BF16", E=None, bdt=None, bshape=None):
        lead = [] if E is None else [E]
        words = I * bits // 32
        w = rng.integers(0, 2**32, lead + [O, words], dtype=np.uint32)
        p = rng.integers(0, 2**16, lead + [O, I // gs], dtype=np.uint16)
        T.append((f"{name}.weight", "U32", lead + [O, words], w.tobytes()))
        T.append((f"{name}.scales", sdt, lead + [O, I // gs], p.tobytes()))
        bs = bshape or lead + [O, I // gs]
        bsz = int(np.prod(bs)) * 2
        T.append((f"{name}.biases", bdt or sdt, bs, rng.bytes(bsz)))

    def mx(name, O, I, E=None, sshape=None):
        lead = [] if E is None else [E]
        w = rng.integers(0, 2**32, lead + [O, I // 8], dtype=np.uint32)
        T.append((f"{name}.weight", "U32", lead + [O, I // 8], w.tobytes()))
        ss = sshape or lead + [O, (I + 31) // 32]
        T.append((f"{name}.scales", "U8", ss, rng.bytes(int(np.prod(ss)))))

    aff("d4", 8, 128, 4, 64)
    aff("d5", 8, 128, 5, 32, "F16")
    aff("d6", 4, 192, 6, 64)
    aff("d8", 4, 64, 8, 64)
    aff("bdt", 4, 64, 4, 64, bdt="F16")
    aff("bsh", 4, 64, 4, 64, bshape=[4, 2])
    aff("g3", 4, 96, 4, 32)  # 3 groups of 32 (I/groups uneven elsewhere)
    mx("mx", 8, 96)
    mx("mxbad", 8, 96, sshape=[8, 4])
    aff("e4", 16, 128, 4, 64, E=6)
    aff("e6", 8, 128, 6, 32, "F16", E=3)
    mx("emx", 8, 64, E=4)
    T.append(("w3.weight", "U32", [4, 3], rng.bytes(48)))          # 3 words: 96 bits
    T.append(("w3.scales", "BF16", [4, 1], rng.bytes(8)))
    T.append(("w3.biases", "BF16", [4, 1], rng.bytes(8)))
    T.append(("f32.weight", "F32", [4, 8], rng.bytes(128)))
    T.append(("nosc.weight", "U32", [4, 8], rng.bytes(128)))
    T.append(("nobi.weight", "U32", [4, 8], rng.bytes(128)))
    T.append(("nobi.scales", "BF16", [4, 1], rng.bytes(8)))
    T.append(("i32sc.weight", "U32", [4, 8], rng.bytes(128)))
    T.append(("i32sc.scales", "I32", [4, 1], rng.bytes(16)))
    T.append(("u8w5.weight", "U32", [4, 10], rng.bytes(160)))     # 5-bit codes, U8 scales
    T.append(("u8w5.scales", "U8", [4, 2], rng.bytes(8)))
    T.append(("rows.scales", "BF16", [5, 1], rng.bytes(10)))
    T.append(("rows.weight", "U32", [4, 8], rng.bytes(128)))
    T.append(("ezero.weight", "U32", [2, 4, 8], rng.bytes(256)))
    # a zero dimension still spans one element (the reader counts max(1, product))
    T.append(("ezero.scales", "BF16", [2, 4, 0], rng.bytes(2)))
    T.append(("plain", "U32", [4, 8], rng.bytes(128)))
    T.append(("ebits.weight", "U32", [2, 4, 3], rng.bytes(96)))
    T.append(("ebits.scales", "BF16", [2, 4, 1], rng.bytes(16)))
    T.append(("ebits.biases", "BF16", [2, 4, 1], rng.bytes(16)))
    T.append(("emx64.weight", "U32", [2, 4, 8], rng.bytes(256)))   # MXFP4 with group 64
    T.append(("emx64.scales", "U8", [2, 4, 1], rng.bytes(8)))
    ock.write_checkpoint(path, T)
    return path


DENSE_CASES = [
    ("d4.weight", 8, 128), ("d5.weight", 8, 128), ("d6.weight", 4, 192), ("d8.weight", 4, 64),
    ("mx.weight", 8, 96), ("g3.weight", 4, 96),
    ("d4.weight", 0, 128), ("d4.weight", 8, 0), ("missing.weight", 4, 4), ("d4.weight", 7, 128),
    ("f32.weight", 4, 8), ("e4.weight", 16, 128), ("d4.weight", 8, 100), ("w3.weight", 4, 32),
    ("w3.weight", 4, 12), ("d4.weight", 8, 8), ("plain", 4, 64), ("nosc.weight", 4, 64),
    ("nobi.weight", 4, 64), ("bdt.weight", 4, 64), ("bsh.weight", 4, 64),
    ("mxbad.weight", 8, 96), ("i32sc.weight", 4, 64), ("u8w5.weight", 4, 64),
    ("rows.weight", 4, 64), ("d6.weight", 4, 128),
]

EXPERT_CASES = [
    ("e4.weight", 0, 6, 16, 128), ("e4.weight", 5, 6, 16, 128), ("e6.weight", 2, 3, 8, 128),
    ("emx.weight", 3, 4, 8, 64),
    ("e4.weight", 6, 6, 16, 128), ("e4.weight", 0, 6, 0, 128), ("e4.weight", 0, 6, 16, 0),
    ("missing.weight", 0, 1, 4, 4), ("d4.weight", 0, 1, 8, 128), ("e4.weight", 0, 5, 16, 128),
    ("e4.weight", 0, 6, 15, 128), ("e4.weight", 0, 6, 16, 100), ("ebits.weight", 0, 2, 4, 32),
    ("ebits.weight", 0, 2, 4, 12), ("ezero.weight", 0, 2, 4, 64), ("e6.weight", 0, 3, 8, 100),
    ("emx64.weight", 1, 2, 4, 64), ("e4.weight", 0, 6, 16, 96),
]


def _oracle_plan(fn, *a):
    try:
        q = fn(*a)
        return ("ok", q)
    except ock.StError as e:
        return ("err", str(e))


@pytest.fixture(scope="module")
def qpath(tmp_path_factory):
    return quant_checkpoint(str(tmp_path_factory.mktemp("q") / "q.safetensors"),
                            np.random.default_rng(11))


def _same(q, want, L):
    kind = L.LOGAN_HIP_WT_AFFINE if want.kind == "affine" else L.LOGAN_HIP_WT_MXFP4
    assert q.kind == kind
    assert (q.bits, q.group_size, bool(q.aux_fp16)) == (want.bits, want.group_size, want.aux_fp16)
    assert (q.weight_bytes, q.scale_bytes, q.bias_bytes) == (
        len(want.weights), len(want.scales), len(want.biases))
    assert not q.weights and not q.owner


@pytest.mark.parametrize("name,o,i", DENSE_CASES)
def test_dense_plan_matches_the_reference_loader(ck, qpath, name, o, i):
    from logan_amd import _lib as L

    ost = ock.StFile.open(qpath)
    want = _oracle_plan(ock.load_mlx_quantized_wt, ost, name, o, i)
    with ck.StFile.open(qpath) as st:
        if want[0] == "err":
            with pytest.raises(ck.CheckpointError) as got:
                ck.plan_mlx_quantized_wt(st, name, o, i)
            assert str(got.value) == want[1]
        else:
            q = ck.plan_mlx_quantized_wt(st, name, o, i)
            _same(q, want[1], L)
            assert (q.E, q.O, q.I) == (1, o, i)


@pytest.mark.parametrize("name,e,E,o,i", EXPERT_CASES)
def test_expert_plan_matches_the_reference_loader(ck, qpath, name, e, E, o, i):
    from logan_amd import _lib as L

    ost = ock.StFile.open(qpath)
    want = _oracle_plan(ock.load_mlx_quantized_expert_wt, ost, name, e, E, o, i)
    with ck.StFile.open(qpath) as st:
        if want[0] == "err":
            with pytest.raises(ck.CheckpointError) as got:
                ck.plan_mlx_quantized_experts(st, name, e, 1, E, o, i)
            assert str(got.value) == want[1]
        else:
            q = ck.plan_mlx_quantized_experts(st, name, e, 1, E, o, i)
            _same(q, want[1], L)
            assert (q.E, q.O, q.I) == (1, o, i)


def test_bank_plan_covers_a_range_of_experts(ck, qpath):
    """count > 1 is this library's whole-bank form: the byte counts are the
    sum of the one-expert slices; a range past the bank is rejected."""
    ost = ock.StFile.open(qpath)
    with ck.StFile.open(qpath) as st:
        q = ck.plan_mlx_quantized_experts(st, "e4.weight", 1, 5, 6, 16, 128)
        one = ock.load_mlx_quantized_expert_wt(ost, "e4.weight", 1, 6, 16, 128)
        assert q.E == 5 and q.weight_bytes == 5 * len(one.weights)
        assert q.scale_bytes == 5 * len(one.scales) == q.bias_bytes
        with pytest.raises(ck.CheckpointError, match=r"invalid expert geometry expert=2/6 "
                                                     r"matrix=16x128 count=5$"):
            ck.plan_mlx_quantized_experts(st, "e4.weight", 2, 5, 6, 16, 128)
