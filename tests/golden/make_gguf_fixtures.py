"""Writes the GGUF files that the reference's own reader tests build in memory
(crates/gguf/src/lib.rs:2301-2460 with its test GgufWriter :2626-2684, and
the router fixture crates/model/src/moe_router.rs:1139-1330), byte for byte,
into tests/golden/gguf/. The steps (header, metadata keys and values, tensor
directory, padding to the 32-byte alignment, payload) are restated here with
a writer of our own that is independent of inferno_amd.gguf.write_gguf, so
the reader is pinned against bytes the reference defines, not against its
own writer. Block payloads come from the reference's block builders
(tests/kat_blocks.py).

    python tests/golden/make_gguf_fixtures.py        # rewrite the files
"""
import struct
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import kat_blocks as kb  # noqa: E402

OUT = HERE / "gguf"

# ggml type codes / metadata value types (gguf/src/lib.rs GgmlType,
# GgufMetadataValueType)
F32, Q8_0, Q2K, Q3K, Q4K, Q6K = 0, 8, 10, 11, 12, 14
MT_U32, MT_F32, MT_STRING, MT_ARRAY = 4, 6, 8, 9


class Writer:
    def __init__(self):
        self.b = bytearray()
        self.data_start = None

    def u32(self, v):
        self.b += struct.pack("<I", v)

    def u64(self, v):
        self.b += struct.pack("<Q", v)

    def string(self, s):
        e = s.encode()
        self.u64(len(e))
        self.b += e

    def header(self, tensors, kvs):
        self.b += b"GGUF"
        self.u32(3)
        self.u64(tensors)
        self.u64(kvs)

    def kv_u32(self, key, v):
        self.string(key)
        self.u32(MT_U32)
        self.u32(v)

    def kv_str(self, key, v):
        self.string(key)
        self.u32(MT_STRING)
        self.string(v)

    def tensor_info(self, name, dims, ty, offset):
        self.string(name)
        self.u32(len(dims))
        for d in dims:
            self.u64(d)
        self.u32(ty)
        self.u64(offset)

    def pad_to(self, a):
        self.b += b"\0" * (-len(self.b) % a)
        self.data_start = len(self.b)

    def pad_to_data_offset(self, off):
        target = self.data_start + off
        if len(self.b) < target:
            self.b += b"\0" * (target - len(self.b))

    def bytes(self, data):
        self.b += bytes(data)


def tiny(second_offset=64):
    # tiny_gguf_with_second_offset (lib.rs:2305-2331)
    w = Writer()
    w.header(2, 5)
    w.kv_str("general.architecture", "glm-dsa")
    w.kv_u32("general.alignment", 32)
    w.kv_u32("general.quantization_version", 2)
    w.kv_u32("general.file_type", 12)
    w.string("tokenizer.ggml.tokens")
    w.u32(MT_ARRAY)
    w.u32(MT_STRING)
    w.u64(1025)
    for _ in range(1025):
        w.string("")
    w.tensor_info("blk.0.attn_q.weight", [32], Q8_0, 0)
    w.tensor_info("token_embd.weight", [256], Q2K, second_offset)
    w.pad_to(32)
    w.bytes(range(160))
    return bytes(w.b)


def single(arch, name, dims, ty, payload):
    # the one-tensor fixtures (lib.rs:2333-2460): 2 metadata keys, one tensor
    # at offset 0, payload, 16 trailing zero bytes
    w = Writer()
    w.header(1, 2)
    w.kv_str("general.architecture", arch)
    w.kv_u32("general.alignment", 32)
    w.tensor_info(name, dims, ty, 0)
    w.pad_to(32)
    w.bytes(payload)
    w.bytes(b"\0" * 16)
    return bytes(w.b)


def supported_quant():
    # tiny_supported_quant_gguf (lib.rs:2350-2370)
    w = Writer()
    w.header(2, 2)
    w.kv_str("general.architecture", "glm-dsa")
    w.kv_u32("general.alignment", 32)
    w.tensor_info("q2.weight", [256], Q2K, 0)
    w.tensor_info("q8.weight", [32], Q8_0, 96)
    w.pad_to(32)
    w.bytes(b"\x22" * 84)
    w.bytes(b"\0" * (96 - 84))
    w.bytes(b"\x88" * 34)
    w.bytes(b"\0" * 16)
    return bytes(w.b)


def bad_alignment():
    # rejects_bad_alignment_metadata (lib.rs:2286-2299)
    w = Writer()
    w.header(0, 1)
    w.kv_u32("general.alignment", 7)
    return bytes(w.b)


def router(gate_ty, bias=(0.0, 0.4, 0.2, 0.8)):
    # write_router_fixture_with_bias + write_gguf (moe_router.rs:1143-1240):
    # tensors laid out at 32-byte aligned offsets, F32 values default 1.0,
    # Q2_K payload zero blocks
    specs = [("blk.1.ffn_norm.weight", [256], F32, None),
             ("blk.1.ffn_gate_inp.weight", [256, 4], gate_ty, None),
             ("blk.1.exp_probs_b.bias", [len(bias)], F32, list(bias))]

    def payload_len(dims, ty):
        n = 1
        for d in dims:
            n *= d
        return n * 4 if ty == F32 else n // 256 * 84

    w = Writer()
    w.header(len(specs), 2)
    w.kv_str("general.architecture", "glm-dsa")
    w.kv_u32("general.alignment", 32)
    offsets, off = [], 0
    for name, dims, ty, _ in specs:
        offsets.append(off)
        off = -(-(off + payload_len(dims, ty)) // 32) * 32
    for (name, dims, ty, _), o in zip(specs, offsets):
        w.tensor_info(name, dims, ty, o)
    w.pad_to(32)
    for (name, dims, ty, vals), o in zip(specs, offsets):
        w.pad_to_data_offset(o)
        if ty == F32:
            n = payload_len(dims, ty) // 4
            for v in (vals if vals is not None else [1.0] * n):
                w.bytes(struct.pack("<f", v))
        else:
            w.bytes(b"\0" * payload_len(dims, ty))
    w.pad_to_data_offset(off)
    return bytes(w.b)


def q2_values_block():
    sm = [(i + 1 if i < 15 else 0, i) for i in range(16)]
    return kb.q2_k_block(0x3C00, 0x3800, sm, 0xE4)


FIXTURES = {
    "tiny.gguf": lambda: tiny(64),
    "tiny_unaligned_offset.gguf": lambda: tiny(33),
    "tiny_f32.gguf": lambda: single("glm-dsa", "output_norm.weight", [4], F32,
                                    struct.pack("<4f", 1.0, -2.0, 3.5, 0.25)),
    "supported_quant.gguf": supported_quant,
    "q8_0_values.gguf": lambda: single("glm-dsa", "q8.weight", [32], Q8_0,
                                       kb.q8_0_block(0x3800, -8)),
    "q2_k_values.gguf": lambda: single("glm-dsa", "q2.weight", [256], Q2K, q2_values_block()),
    "q3_k_values.gguf": lambda: single("laguna", "q3.weight", [256], Q3K,
                                       kb.q3_k_block(0x3C00, [33] * 16, 0xE4, 0xFF)),
    "q4_k_values.gguf": lambda: single("laguna", "q4.weight", [256], Q4K,
                                       kb.q4_k_block(0x3C00, 0x0000, 1, 0, 0x21)),
    "q6_k_values.gguf": lambda: single("laguna", "q6.weight", [256], Q6K,
                                       kb.q6_k_block(0x3C00, 1, 0x00, 0x00)),
    "bad_alignment.gguf": bad_alignment,
    "router_f32.gguf": lambda: router(F32),
    "router_q2_k.gguf": lambda: router(Q2K),
}


def build_all():
    return {name: f() for name, f in FIXTURES.items()}


if __name__ == "__main__":
    OUT.mkdir(exist_ok=True)
    for name, data in build_all().items():
        (OUT / name).write_bytes(data)
        print(f"{name}: {len(data)} bytes")
