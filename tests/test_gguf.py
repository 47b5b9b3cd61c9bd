"""GGUF v3 ingestion (aipu_amd/gguf.py) on the CPU: the container bytes against a hand-built
file, the write -> read round trip over the reference's synthetic tensor set
(tools/ckpt_pack_q4k.py:228-292: Q4_K, Q6_K, Q8_0, F16 and an F32 norm tail) plus BF16 and a
fused expert stack, the bounded header parser against the in-memory one, the hot/expert
rule of tools/provision_image.py:60-83, and the error paths."""
import struct

import numpy as np
import pytest

from aipu_amd import gguf
from oracle import q4k_oracle as qo


def _s(b):
    return struct.pack("<Q", len(b)) + b


def _hand_file():
    """A GGUF v3 file assembled field by field from the published layout (not with the
    module under test): KV of every kind, one F32 tensor [4] and one Q8_0 tensor [32, 2]."""
    kv = [
        _s(b"general.alignment") + struct.pack("<II", 4, 64),
        _s(b"general.name") + struct.pack("<I", 8) + _s(b"tiny"),
        _s(b"x.f") + struct.pack("<If", 6, 1.5),
        _s(b"x.b") + struct.pack("<I?", 7, True),
        _s(b"x.arr_u32") + struct.pack("<IIQ", 9, 4, 3) + struct.pack("<3I", 7, 8, 9),
        _s(b"x.arr_str") + struct.pack("<IIQ", 9, 8, 2) + _s(b"ab") + _s(b"cde"),
        _s(b"x.nested") + struct.pack("<IIQ", 9, 9, 1) + struct.pack("<IQ", 5, 2) + struct.pack("<2i", -1, 2),
    ]
    f32 = np.array([1.0, -2.0, 0.5, 3.25], np.float32).tobytes()
    q8 = bytes(range(68))
    infos = (_s(b"norm.weight") + struct.pack("<I", 1) + struct.pack("<Q", 4) + struct.pack("<IQ", 0, 0)
             + _s(b"blk.0.attn_q.weight") + struct.pack("<I", 2) + struct.pack("<2Q", 32, 2)
             + struct.pack("<IQ", 8, 64))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, len(kv)) + b"".join(kv) + infos
    head += b"\0" * (-len(head) % 64)
    blob = f32 + b"\0" * 48 + q8
    return head + blob, f32, q8


def test_magic_and_counts_bytes():
    buf = gguf.write_gguf([])
    assert buf[:4] == b"GGUF"
    assert struct.unpack_from("<IQQ", buf, 4) == (3, 0, 3)
    assert len(buf) % 32 == 0


def test_read_hand_built_file(tmp_path):
    buf, f32, q8 = _hand_file()
    meta, ts = gguf.read_gguf(buf)
    assert meta["general.alignment"] == 64 and meta["general.name"] == "tiny"
    assert meta["x.f"] == 1.5 and meta["x.b"] is True
    assert meta["x.arr_u32"] == [7, 8, 9] and meta["x.arr_str"] == ["ab", "cde"] and meta["x.nested"] == [[-1, 2]]
    assert ts["norm.weight"] == (0, [4], f32)
    assert ts["blk.0.attn_q.weight"] == (8, [32, 2], q8)
    p = tmp_path / "hand.gguf"
    p.write_bytes(buf)
    hdr = gguf.read_header(str(p))
    assert hdr.alignment == 64 and hdr.data_start % 64 == 0
    assert "x.arr_str" not in hdr.meta          # skipped without being held
    info = hdr.by_name()
    assert buf[info["blk.0.attn_q.weight"].offset:][:68] == q8
    assert info["norm.weight"].kind == "resident_hot"


def _synthetic(rng):
    """The reference self-test's tensor set (names, types, ne) and two more."""
    def f16(n):
        return rng.uniform(-2, 2, n).astype(np.float16).tobytes()
    t = [
        ("blk.0.ffn_down.weight", gguf.GGML_Q4_K, [512, 8], qo.random_q4k_blocks(rng, 16).tobytes()),
        ("blk.0.ffn_gate.weight", gguf.GGML_Q4_K, [256, 8], qo.random_q4k_blocks(rng, 8).tobytes()),
        ("blk.0.attn_output.weight", gguf.GGML_Q6_K, [256, 4], qo.random_q6k_blocks(rng, 4).tobytes()),
        ("blk.0.attn_q.weight", gguf.GGML_Q8_0, [256, 4], qo.random_q8_0_blocks(rng, 32).tobytes()),
        ("output.weight", gguf.GGML_F16, [256, 4], f16(1024)),
        ("blk.0.attn_norm.weight", gguf.GGML_F32, [64], rng.uniform(-1, 1, 64).astype(np.float32).tobytes()),
        ("token_embd.weight", gguf.GGML_BF16, [64, 5], qo.random_bf16(rng, 320).tobytes()),
        ("blk.1.ffn_gate_exps.weight", gguf.GGML_Q4_K, [256, 16, 3], qo.random_q4k_blocks(rng, 48).tobytes()),
    ]
    return t


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_round_trip(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    tens = _synthetic(rng)
    buf = gguf.write_gguf(tens, alignment=alignment)
    meta, got = gguf.read_gguf(buf)
    assert meta["general.architecture"] == "glm" and meta["general.alignment"] == alignment
    assert meta["general.quantization_version"] == 2
    for name, ttype, dims, raw in tens:
        assert got[name] == (ttype, dims, raw), name
    p = tmp_path / "s.gguf"
    p.write_bytes(buf)
    hdr = gguf.read_header(str(p))
    for t in hdr.tensors:
        assert t.offset % alignment == 0
        assert buf[t.offset:t.offset + t.nbytes] == got[t.name][2]
    f = gguf.GGUFFile(str(p))
    assert bytes(f.host_bytes("output.weight")) == got["output.weight"][2]
    assert [t.name for t in f.tensors] == [n for n, *_ in tens]


def test_q4k_blocks_survive_and_dequantise(tmp_path):
    """Bytes read back dequantise bit-exactly to the same weights (the reference's
    dequant cross-check, tools/ckpt_pack_q4k.py:454-480)."""
    rng = np.random.default_rng(7)
    raw = qo.random_q4k_blocks(rng, 24)
    buf = gguf.write_gguf([("w", gguf.GGML_Q4_K, [768, 8], raw.tobytes())])
    _, got = gguf.read_gguf(buf)
    a = qo.dequant_q4k(raw)
    b = qo.dequant_q4k(np.frombuffer(got["w"][2], np.uint8))
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("name,kind", [
    ("blk.3.ffn_gate_exps.weight", "streamed_expert"),
    ("blk.3.ffn_down_exps.weight", "streamed_expert"),
    ("model.layers.3.mlp.experts.7.down_proj.weight", "streamed_expert"),
    ("blk.3.ffn_gate_inp.weight", "resident_hot"),
    ("blk.3.ffn_down_shexp.weight", "resident_hot"),
    ("output.weight", "resident_hot"),
    ("token_embd.weight", "resident_hot"),
])
def test_classify(name, kind):
    assert gguf.classify(name) == kind


def test_tnbytes_table():
    assert gguf.tnbytes(gguf.GGML_Q4_K, 6144 * 6144) == 147456 * 144
    assert gguf.tnbytes(gguf.GGML_Q6_K, 512) == 420
    assert gguf.tnbytes(gguf.GGML_Q8_0, 64) == 68
    assert gguf.tnbytes(gguf.GGML_BF16, 10) == 20
    with pytest.raises(gguf.GGUFError):
        gguf.tnbytes(gguf.GGML_Q4_K, 300)
    with pytest.raises(gguf.GGUFError):
        gguf.tnbytes(99, 4)


def test_errors(tmp_path):
    good = gguf.write_gguf([("a", gguf.GGML_F32, [4], bytes(16))])
    with pytest.raises(gguf.GGUFError, match="magic"):
        gguf.read_gguf(b"GGUX" + good[4:])
    with pytest.raises(gguf.GGUFError, match="version"):
        gguf.read_gguf(good[:4] + struct.pack("<I", 2) + good[8:])
    with pytest.raises(gguf.GGUFError, match="truncated"):
        gguf.read_gguf(good[:40])
    with pytest.raises(gguf.GGUFError, match="past the end"):
        gguf.read_gguf(good[:-24])
    p = tmp_path / "short.gguf"
    p.write_bytes(good[:-24])
    with pytest.raises(gguf.GGUFError, match="past the end"):
        gguf.read_header(str(p))
    with pytest.raises(gguf.GGUFError):
        gguf.write_gguf([("a", gguf.GGML_F32, [4], bytes(15))])
    with pytest.raises(gguf.GGUFError):
        gguf.write_gguf([("a", gguf.GGML_Q4_K, [100], bytes(144))])
    f = gguf.GGUFFile(_write(tmp_path, [("i", 26, [4], bytes(16))]))
    with pytest.raises(gguf.GGUFError, match="not a type"):
        f.upload("i", device="cpu")


def _write(tmp_path, tensors):
    p = tmp_path / "t.gguf"
    p.write_bytes(gguf.write_gguf(tensors))
    return str(p)
