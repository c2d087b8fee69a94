"""GGUF v3 reader: header, metadata, tensor directory, storage ranges and the
packed-expert mapping (inferno_amd/gguf.py), on files written in the test.

The cases follow the reference reader's checks (crates/gguf/src/lib.rs
:164-294, :1654-1730, :1821-1875, :1903-1915) and layer naming
(crates/model/src/index.rs:417-429)."""

import struct

import numpy as np
import pytest

from inferno_amd import gguf as G

rng = np.random.default_rng(3)


def _blocks(ty, rows, width):
    per, size = G.BLOCKS[ty]
    return rng.integers(0, 256, size=rows * (width // per) * size, dtype=np.uint8).tobytes()


def _moe_tensors(layer, H, I, E, Is, q=G.GGML_Q2_K, bias=True):
    p = f"blk.{layer}"
    ts = [(f"{p}.ffn_gate_inp.weight", (H, E), G.GGML_F32,
           rng.standard_normal(E * H).astype(np.float32).tobytes())]
    if bias:
        ts.append((f"{p}.exp_probs_b.bias", (E,), G.GGML_F32,
                   rng.standard_normal(E).astype(np.float32).tobytes()))
    ts += [(f"{p}.ffn_gate_exps.weight", (H, I, E), q, _blocks(q, E * I, H)),
           (f"{p}.ffn_up_exps.weight", (H, I, E), q, _blocks(q, E * I, H)),
           (f"{p}.ffn_down_exps.weight", (I, H, E), q, _blocks(q, E * H, I))]
    if Is:
        ts += [(f"{p}.ffn_gate_shexp.weight", (H, Is), G.GGML_Q8_0, _blocks(8, Is, H)),
               (f"{p}.ffn_up_shexp.weight", (H, Is), G.GGML_Q8_0, _blocks(8, Is, H)),
               (f"{p}.ffn_down_shexp.weight", (Is, H), G.GGML_Q8_0, _blocks(8, H, Is))]
    return ts


META = [("general.architecture", G.MT_STRING, "glm"),
        ("general.quantization_version", G.MT_U32, 2),
        ("glm.expert_count", G.MT_U64, 8),
        ("glm.rope.freq_base", G.MT_F32, 1.0e6),
        ("glm.use_bias", G.MT_BOOL, True),
        ("tokenizer.scores", G.MT_ARRAY, (G.MT_F32, [0.5, -1.0, 2.0])),
        ("nested", G.MT_ARRAY, (G.MT_ARRAY, [(G.MT_I16, [1, -2]), (G.MT_I16, [3])])),
        ("big", G.MT_ARRAY, (G.MT_U8, list(range(256)) * 5))]


def test_roundtrip_metadata_tensors_and_zero_copy_bytes(tmp_path):
    path = tmp_path / "m.gguf"
    ts = _moe_tensors(3, 512, 256, 4, 256)
    G.write_gguf(path, META, ts)
    with G.GGUFFile(path) as g:
        assert g.version == 3 and g.tensor_count == len(ts) and g.alignment == 32
        assert g.metadata["general.architecture"] == "glm"
        assert g.metadata["glm.expert_count"] == 8 and g.metadata["glm.use_bias"] is True
        assert g.metadata["tokenizer.scores"].values == [0.5, -1.0, 2.0]
        nested = g.metadata["nested"].values
        assert [a.values for a in nested] == [[1, -2], [3]]
        big = g.metadata["big"]
        assert big.length == 1280 and big.values is None  # parsed, not kept
        assert g.tensor_data_offset % 32 == 0
        for name, dims, ty, data in ts:
            t = g.tensor(name)
            assert t.dims == dims and t.ty == ty and t.absolute_offset % 32 == 0
            b = g.tensor_bytes(name)
            assert b.tobytes() == data
            assert not b.flags.owndata  # a view of the mapping
        # storage range: up to the next tensor's start (padding included)
        by = sorted(g.tensors.values(), key=lambda t: t.absolute_offset)
        for a, b in zip(by, by[1:]):
            assert a.storage_byte_len == b.absolute_offset - a.absolute_offset >= a.nbytes
        assert by[-1].storage_byte_len == g.file_size - by[-1].absolute_offset
        del b


def test_packed_expert_mapping(tmp_path):
    path = tmp_path / "m.gguf"
    G.write_gguf(path, META[:1], _moe_tensors(1, 768, 512, 6, 0, q=G.GGML_Q3_K))
    with G.GGUFFile(path) as g:
        px = G.packed_experts(g, 1)
        assert (px.hidden, px.intermediate, px.experts) == (768, 512, 6)
        # expert e's gate rows start at e * I * (H / 256) * 110 bytes
        assert px.gate.nbytes == 6 * 512 * 3 * 110
        assert px.down.nbytes == 6 * 768 * 2 * 110
        with pytest.raises(G.GGUFError, match="missing GGUF tensor blk.0"):
            G.packed_experts(g, 0)


def test_packed_expert_shape_mismatch(tmp_path):
    path = tmp_path / "m.gguf"
    ts = _moe_tensors(0, 512, 256, 4, 0)
    name, _, q, _ = ts[-1]
    ts[-1] = (name, (256, 512, 2), q, _blocks(q, 2 * 512, 256))  # down with 2 experts
    G.write_gguf(path, [], ts)
    with G.GGUFFile(path) as g, pytest.raises(G.GGUFError, match="expected"):
        G.packed_experts(g, 0)


def _header(version=3, kv=(), tensors=(), magic=b"GGUF"):
    out = magic + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, t, payload in kv:
        kb = k.encode()
        out += struct.pack("<Q", len(kb)) + kb + struct.pack("<I", t) + payload
    for name, dims, ty, off in tensors:
        nb = name.encode()
        out += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims))
        out += struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", ty, off)
    return out


@pytest.mark.parametrize("blob,msg", [
    (_header(magic=b"GGUG"), "bad magic"),
    (_header(version=2), "unsupported GGUF version 2"),
    (_header(kv=[("a..b", G.MT_U8, b"\x01")]), "hierarchical"),
    (_header(kv=[(".a", G.MT_U8, b"\x01")]), "hierarchical"),
    (_header(kv=[("a", G.MT_U8, b"\x01"), ("a", G.MT_U8, b"\x02")]), "duplicate GGUF metadata key"),
    (_header(kv=[("a", G.MT_BOOL, b"\x02")]), "invalid GGUF bool"),
    (_header(kv=[("a", 13, b"")]), "unknown GGUF metadata value type"),
    (_header(kv=[("general.alignment", G.MT_U32, struct.pack("<I", 12))]), "multiple of 8"),
    (_header(tensors=[("t", (), 0, 0)]), "at least one dimension"),
    (_header(tensors=[("t", (1, 1, 1, 1, 1), 0, 0)]), "max supported is 4"),
    (_header(tensors=[("t", (4, 0), 0, 0)]), "zero dimension"),
    (_header(tensors=[("t", (4,), 0, 16)]), "not aligned to 32"),
    (_header(tensors=[("t", (4,), 0, 1 << 20)]), "exceeds file size"),
    (_header(tensors=[("x" * 65, (4,), 0, 0)]), "limit"),
    (_header(kv=[("a", G.MT_STRING, struct.pack("<Q", 1000))]), "ends inside"),
])
def test_rejects_malformed(tmp_path, blob, msg):
    path = tmp_path / "bad.gguf"
    path.write_bytes(blob + b"\0" * 64)
    with pytest.raises(G.GGUFError, match=msg):
        G.GGUFFile(path)


def test_nesting_depth_limit(tmp_path):
    # nine nested array levels exceed the depth limit of 8
    payload = b""
    inner = struct.pack("<IQ", G.MT_U8, 0)
    for _ in range(9):
        inner = struct.pack("<IQ", G.MT_ARRAY, 1) + inner
    payload = inner
    path = tmp_path / "deep.gguf"
    path.write_bytes(_header(kv=[("deep", G.MT_ARRAY, payload)]) + b"\0" * 64)
    with pytest.raises(G.GGUFError, match="too deep"):
        G.GGUFFile(path)


def test_overlapping_tensors_and_short_storage(tmp_path):
    path = tmp_path / "o.gguf"
    path.write_bytes(_header(tensors=[("a", (8,), 0, 0), ("b", (8,), 0, 0)]) + b"\0" * 64)
    with pytest.raises(G.GGUFError, match="invalid storage range"):
        G.GGUFFile(path)
    # a Q8_0 tensor of 64 values (68 bytes) whose range holds 32 bytes
    path.write_bytes(_header(tensors=[("q", (64,), 8, 0), ("n", (8,), 0, 32)]) + b"\0" * 128)
    with G.GGUFFile(path) as g:
        with pytest.raises(G.GGUFError, match="needs 68 bytes"):
            g.tensor_bytes("q")
        assert g.tensor_bytes("n").size == 32


@pytest.mark.parametrize("t,v", [(G.MT_I32, 64), (G.MT_F32, 64.0), (G.MT_STRING, "64")])
def test_alignment_key_of_another_type_falls_back_to_32(tmp_path, t, v):
    # metadata_alignment (lib.rs:1821-1840) reads only unsigned integers;
    # any other value type means the default alignment
    path = tmp_path / "a.gguf"
    G.write_gguf(path, [("general.alignment", t, v)],
                 [("x.weight", (8,), G.GGML_F32, np.zeros(8, np.float32).tobytes())])
    with G.GGUFFile(path) as g:
        assert g.alignment == 32


def test_unstored_array_strings_are_skipped_unchecked(tmp_path):
    # strings inside arrays of more than 1024 values are skipped without
    # UTF-8 validation (skip_string, lib.rs:1741-1746)
    path = tmp_path / "s.gguf"
    G.write_gguf(path, [("tok", G.MT_ARRAY, (G.MT_STRING, ["ok"] * 1100))],
                 [("x.weight", (8,), G.GGML_F32, np.zeros(8, np.float32).tobytes())])
    raw = bytearray(path.read_bytes())
    i = raw.index(struct.pack("<Q", 2) + b"ok") + 8
    raw[i] = 0xFF  # an invalid UTF-8 byte in an unstored string
    path.write_bytes(bytes(raw))
    with G.GGUFFile(path) as g:
        assert g.metadata["tok"].length == 1100 and g.metadata["tok"].values is None


def test_quant_rows_must_be_whole_blocks(tmp_path):
    # block_count_for_quant_block (lib.rs:1877-1900) checks the first
    # dimension before the element count: Q4_K [48, 16] holds 768 values (3
    # whole blocks) but its 48-value rows are not whole 256-value blocks
    path = tmp_path / "r.gguf"
    path.write_bytes(_header(tensors=[("q", (48, 16), G.GGML_Q4_K, 0)]) + b"\0" * 512)
    with pytest.raises(G.GGUFError, match="first dimension 48 is not divisible by Q4_K block size 256"):
        with G.GGUFFile(path) as g:
            g.tensor_bytes("q")
    # rows of 512 values are whole blocks: 3 rows of 2 blocks
    path.write_bytes(_header(tensors=[("q", (512, 3), G.GGML_Q4_K, 0)]) + b"\0" * 1024)
    with G.GGUFFile(path) as g:
        assert g.tensor_bytes("q").size == 6 * 144
