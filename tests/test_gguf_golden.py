"""The GGUF reader (inferno_amd/gguf.py) on the files the reference's own
reader tests build (tests/golden/gguf/, written by make_gguf_fixtures.py with
a writer independent of ours), with the reference tests' expected values:
crates/gguf/src/lib.rs:1929-2299 and crates/model/src/moe_router.rs:1139-1240.
Block values are decoded by the oracle (the same formulas the GPU dequant is
checked against bit for bit)."""
import struct
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as orc
from golden import make_gguf_fixtures as mk
from inferno_amd import gguf as G
from inferno_amd._lib import Q2_K, Q3_K, Q4_K, Q6_K, Q8_0

GDIR = Path(__file__).resolve().parent / "golden" / "gguf"


def test_fixture_files_match_their_generator():
    for name, data in mk.build_all().items():
        assert (GDIR / name).read_bytes() == data, name


def test_header_metadata_and_tensor_directory():
    # parses_header_metadata_and_tensor_directory (lib.rs:1929-1958)
    with G.GGUFFile(GDIR / "tiny.gguf") as g:
        assert g.version == 3 and g.tensor_count == 2 and g.metadata_kv_count == 5
        assert g.alignment == 32
        assert g.metadata["general.architecture"] == "glm-dsa"
        assert g.metadata["general.quantization_version"] == 2
        assert g.metadata["general.file_type"] == 12
        assert len({t.ty for t in g.tensors.values()}) == 2
        q = g.tensor("blk.0.attn_q.weight")
        assert q.dims == (32,) and q.ty == G.GGML_Q8_0 and q.relative_offset == 0
        assert q.absolute_offset % 32 == 0 and q.storage_byte_len == 64
        assert q.elements == 32 and len(q.dims) == 1
        tokens = g.metadata["tokenizer.ggml.tokens"]
        assert tokens.length == 1025 and tokens.values is None  # omitted (> 1024 values)


def test_storage_ranges_are_checked_payload_ranges():
    # tensor_storage_returns_checked_mapped_payload_range (lib.rs:1960-1977)
    with G.GGUFFile(GDIR / "tiny.gguf") as g:
        q, e = g.tensor("blk.0.attn_q.weight"), g.tensor("token_embd.weight")
        raw = np.frombuffer((GDIR / "tiny.gguf").read_bytes(), np.uint8)
        qb = raw[q.absolute_offset:q.absolute_offset + q.storage_byte_len]
        eb = raw[e.absolute_offset:e.absolute_offset + e.storage_byte_len]
        assert q.ty == G.GGML_Q8_0 and len(qb) == 64 and qb[0] == 0 and qb[63] == 63
        assert e.ty == G.GGML_Q2_K and len(eb) == 96 and eb[0] == 64 and eb[95] == 159
        assert g.tensor_bytes("token_embd.weight")[0] == 64  # the 84-byte block view
        with pytest.raises(G.GGUFError, match="missing GGUF tensor"):
            g.tensor("missing.weight")


@pytest.mark.parametrize("name,match", [("tiny_unaligned_offset.gguf", "not aligned"),
                                        ("bad_alignment.gguf", "general.alignment")])
def test_rejects_what_the_reference_rejects(name, match):
    # rejects_unaligned_tensor_offset / rejects_bad_alignment_metadata
    # (lib.rs:2276-2299)
    with pytest.raises(G.GGUFError, match=match):
        G.GGUFFile(GDIR / name)


def test_rejects_bad_magic(tmp_path):
    # rejects_invalid_magic (lib.rs:2264-2274)
    b = bytearray((GDIR / "tiny.gguf").read_bytes())
    b[0] = ord("X")
    p = tmp_path / "bad.gguf"
    p.write_bytes(bytes(b))
    with pytest.raises(G.GGUFError, match="magic"):
        G.GGUFFile(p)


def test_f32_payload_without_padding():
    # tensor_f32_values_decodes_raw_payload_without_padding (lib.rs:1992-2001)
    with G.GGUFFile(GDIR / "tiny_f32.gguf") as g:
        v = g.tensor_bytes("output_norm.weight").view(np.float32)
        assert v.tolist() == [1.0, -2.0, 3.5, 0.25]


def test_supported_quant_payload_sizes():
    # tensor_quantized_storage_validates_supported_payload_sizes (lib.rs:2016-2035)
    with G.GGUFFile(GDIR / "supported_quant.gguf") as g:
        q2, q8 = g.tensor_bytes("q2.weight"), g.tensor_bytes("q8.weight")
        assert len(q2) == 84 and q2[0] == 0x22
        assert len(q8) == 34 and q8[0] == 0x88
        assert g.tensor("q2.weight").elements // 256 == 1


def _values(name, tensor, quant):
    with G.GGUFFile(GDIR / name) as g:
        return orc.dequantize(quant, np.array(g.tensor_bytes(tensor)))


def test_q8_0_values():
    # tensor_q8_0_f32_values_decodes_standard_payload (lib.rs:2037-2054)
    v = _values("q8_0_values.gguf", "q8.weight", Q8_0)
    assert len(v) == 32 and v[0] == -4.0 and v[1] == -3.5 and v[16] == 4.0 and v[31] == 11.5


def test_q2_k_values():
    # tensor_q2_k_f32_values_decodes_standard_payload (lib.rs:2056-2081)
    v = _values("q2_k_values.gguf", "q2.weight", Q2_K)
    want = [0.0, -0.5, 2.0, 2.5, 8.0, 9.5, 18.0, 20.5, -4.0, -4.5, 6.0, 6.5, 20.0, 21.5, 38.0,
            -7.5]
    assert len(v) == 256 and [v[16 * i] for i in range(16)] == want


def test_q3_k_values():
    # tensor_q3_k_f32_values_decodes_standard_payload (lib.rs:2083-2105)
    v = _values("q3_k_values.gguf", "q3.weight", Q3_K)
    want = [0, 0, 1, 1, 2, 2, 3, 3, 0, 0, 1, 1, 2, 2, 3, 3]
    for g_, w in enumerate(want):
        assert v[16 * g_] == w and v[16 * g_ + 15] == w


def test_q4_k_values():
    # tensor_q4_k_f32_values_decodes_standard_payload (lib.rs:2107-2125)
    v = _values("q4_k_values.gguf", "q4.weight", Q4_K)
    for g_ in range(8):
        w = 1.0 if g_ % 2 == 0 else 2.0
        assert v[32 * g_] == w and v[32 * g_ + 31] == w


def test_q6_k_values():
    # tensor_q6_k_f32_values_decodes_standard_payload (lib.rs:2127-2140)
    assert (_values("q6_k_values.gguf", "q6.weight", Q6_K) == -32.0).all()


@pytest.mark.parametrize("name", ["router_f32.gguf", "router_q2_k.gguf"])
def test_router_fixture_directory_and_bias(name):
    # write_router_fixture_with_bias (moe_router.rs:1139-1152): norm f32 [256]
    # of ones, router [256, 4], correction bias [0, 0.4, 0.2, 0.8], each
    # tensor at a 32-byte aligned offset
    with G.GGUFFile(GDIR / name) as g:
        norm = g.tensor("blk.1.ffn_norm.weight")
        gate = g.tensor("blk.1.ffn_gate_inp.weight")
        bias = g.tensor("blk.1.exp_probs_b.bias")
        assert norm.relative_offset == 0 and norm.dims == (256,)
        assert gate.relative_offset == 1024 and gate.dims == (256, 4)
        gate_bytes = 4096 if gate.ty == G.GGML_F32 else 4 * 84
        assert bias.relative_offset == 1024 + (-(-gate_bytes // 32) * 32)
        assert (g.tensor_bytes(norm.name).view(np.float32) == 1.0).all()
        assert g.tensor_bytes(bias.name).view(np.float32).tolist() == \
            [float(np.float32(b)) for b in (0.0, 0.4, 0.2, 0.8)]
        assert len(g.tensor_bytes(gate.name)) == gate_bytes
