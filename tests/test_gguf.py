"""GGUF payload oracle (gguf.rs:486-550, 283-296) and the host container code, on the CPU.

The reference's own tests hold no GGUF numbers: frontend_tests.rs:180-219 checks an
IR -> GGUF -> IR round trip by tensor count and commercial_readiness_tests.rs:182-189 that an
oversized tensor count is refused.  The oracle is pinned here by hand-computed known answers
(asymmetric nibble patterns, so a low/high swap or a missing -8 fails), numpy's independent
IEEE f16 decoder, the truncating f16 rule against a value where it differs from rounding, and
encode -> decode round trips.
"""
import struct

import numpy as np
import pytest

import oracle_lib as O
from castforge_amd import gguf

Q4_0, Q8_0, F32, F16, BF16 = 2, 8, 0, 1, 30


def _f16_bytes(bits: int) -> np.ndarray:
    return np.frombuffer(struct.pack("<H", bits), np.uint8)


def test_q4_0_known_block_low_nibble_first():
    # d = 0.5 (0x3800); byte j = (j & 15) | ((15 - j) << 4): element 2j = j - 8, 2j+1 = 7 - j
    blk = np.concatenate([_f16_bytes(0x3800), np.array([(j & 15) | ((15 - j) << 4) for j in range(16)], np.uint8)])
    got = O.gguf_decode(Q4_0, blk, 32)
    want = []
    for j in range(16):
        want += [0.5 * (j - 8), 0.5 * (7 - j)]
    np.testing.assert_array_equal(got, np.array(want, np.float32))


def test_q8_0_known_block_signed_bytes():
    d = 0x4000  # 2.0
    q = np.array([0x00, 0x01, 0x7F, 0x80, 0xFF, 0xFE] + [0x10] * 26, np.uint8)
    got = O.gguf_decode(Q8_0, np.concatenate([_f16_bytes(d), q]), 32)
    np.testing.assert_array_equal(got[:6], np.array([0, 2, 254, -256, -2, -4], np.float32))
    np.testing.assert_array_equal(got[6:], np.full(26, 32.0, np.float32))


def test_partial_last_block_is_truncated():
    rng = np.random.default_rng(1)
    for ty, bb in ((Q4_0, 18), (Q8_0, 34)):
        raw = rng.integers(0, 256, 2 * bb, dtype=np.uint8)
        raw[0:2] = _f16_bytes(0x3C00)
        raw[bb:bb + 2] = _f16_bytes(0x3C00)
        full = O.gguf_decode(ty, raw, 64)
        part = O.gguf_decode(ty, raw, 33)
        np.testing.assert_array_equal(part, full[:33])


def test_block_scales_match_numpy_f16_for_every_pattern_class():
    # d over normal, subnormal, zero, negative, Inf: numpy's float16 is an independent decoder
    rng = np.random.default_rng(2)
    for bits in (0x0001, 0x03FF, 0x0400, 0x3C00, 0x8001, 0xBC00, 0x7BFF, 0x7C00, 0xFC00, 0x0000, 0x8000):
        d = np.frombuffer(struct.pack("<H", bits), np.float16)[0].astype(np.float32)
        codes = rng.integers(-128, 128, 32).astype(np.int8)
        raw = np.concatenate([_f16_bytes(bits), codes.view(np.uint8)])
        got = O.gguf_decode(Q8_0, raw, 32)
        with np.errstate(invalid="ignore", over="ignore"):
            want = codes.astype(np.float32) * d
        np.testing.assert_array_equal(got, want)


def test_f16_bf16_f32_payloads():
    rng = np.random.default_rng(3)
    h = rng.integers(0, 1 << 16, 999, dtype=np.uint16)
    h = h[(h & 0x7C00) != 0x7C00]  # NaN payloads aside (both sides NaN)
    got = O.gguf_decode(F16, h.view(np.uint8), h.size)
    np.testing.assert_array_equal(got.view(np.uint32), h.view(np.float16).astype(np.float32).view(np.uint32))
    got = O.gguf_decode(BF16, h.view(np.uint8), h.size)
    np.testing.assert_array_equal(got.view(np.uint32), h.astype(np.uint32) << 16)
    f = rng.standard_normal(77).astype(np.float32)
    np.testing.assert_array_equal(O.gguf_decode(F32, f.view(np.uint8), f.size), f)


def test_q8_0_encode_truncates_scale_and_pads():
    codes = np.arange(-20, 20, dtype=np.int8)  # 40 codes -> 2 blocks, 24 zero pads
    scale = np.float32(1.0 + 3 * 2.0 ** -12)    # f16 truncation 0x3C00; round-to-nearest 0x3C01
    raw = O.gguf_encode_q8_0(codes, scale)
    assert raw.size == 68
    assert raw[0] == 0x00 and raw[1] == 0x3C and raw[34] == 0x00 and raw[35] == 0x3C
    np.testing.assert_array_equal(raw[2:34].view(np.int8), codes[:32])
    np.testing.assert_array_equal(raw[36:44].view(np.int8), codes[32:])
    assert not raw[44:].any()
    back = O.gguf_decode(Q8_0, raw, 40)
    np.testing.assert_array_equal(back, codes.astype(np.float32))  # d = 1.0 after truncation
    # an empty tensor still writes one block (gguf.rs:285, data.len().max(1))
    assert O.gguf_encode_q8_0(np.zeros(0, np.int8), 0.5).size == 34


def test_q8_0_roundtrip_property():
    rng = np.random.default_rng(4)
    codes = rng.integers(-127, 128, 1000).astype(np.int8)
    scale = np.float32(0.0123)
    back = O.gguf_decode(Q8_0, O.gguf_encode_q8_0(codes, scale), codes.size)
    d = np.float32(O.lib().orc_f16_to_f32(O.lib().orc_f32_to_f16_trunc(scale)))
    np.testing.assert_array_equal(back, codes.astype(np.float32) * d)
    assert d <= scale


# ------------------------------------------------------------------- container (host) ----
def test_header_roundtrip_and_layout():
    p1 = np.arange(18 * 4, dtype=np.uint8)           # Q4_0 [1, 128]
    p2 = np.arange(8, dtype=np.float32).view(np.uint8)  # F32 [2, 4]
    raw = gguf.write_gguf_tensors([("a.weight", (1, 128), Q4_0, p1), ("b", (2, 4), F32, p2)], name="my-model")
    name, infos, base = gguf.read_gguf_header(raw)
    assert name == "my_model"
    assert base % 32 == 0
    assert infos[0][:3] == ("a.weight", (1, 128), Q4_0)
    assert infos[1][:3] == ("b", (2, 4), F32)
    assert infos[1][3] == 96  # 72 payload bytes padded to 32
    assert bytes(raw[base:base + 72]) == p1.tobytes()
    assert bytes(raw[base + 96:base + 128]) == p2.tobytes()


def test_header_refuses_bad_input():
    # commercial_readiness_tests.rs:182-189: tensor_count > 65536 is refused
    bad = b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", 1_000_000) + struct.pack("<Q", 0)
    with pytest.raises(gguf.GgufError, match="exceed safety limit"):
        gguf.read_gguf_header(bad)
    with pytest.raises(gguf.GgufError, match="header magic"):
        gguf.read_gguf_header(b"GGUX" + bytes(40))
    with pytest.raises(gguf.GgufError, match="Unsupported GGUF version: 4"):
        gguf.read_gguf_header(b"GGUF" + struct.pack("<IQQ", 4, 0, 0))
    raw = gguf.write_gguf_tensors([("t", (32,), 7, np.zeros(32, np.uint8))])
    with pytest.raises(gguf.GgufError, match="Unsupported GGML tensor type id: 7"):
        gguf.read_gguf_header(raw)
    raw = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + struct.pack("<Q", 1) + b"t" + struct.pack("<I", 17)
    with pytest.raises(gguf.GgufError, match="rank 17 exceeds maximum rank 16"):
        gguf.read_gguf_header(raw)


def test_metadata_values_are_skipped_and_alignment_read():
    kv = b""
    def s(x):
        return struct.pack("<Q", len(x)) + x
    kv += s(b"general.alignment") + struct.pack("<I", 4) + struct.pack("<I", 64)
    kv += s(b"some.array") + struct.pack("<I", 9) + struct.pack("<I", 5) + struct.pack("<Q", 3) + bytes(12)
    kv += s(b"some.u8") + struct.pack("<I", 0) + b"\x01"
    kv += s(b"general.name") + struct.pack("<I", 8) + s(b"tiny")
    ti = s(b"w") + struct.pack("<I", 1) + struct.pack("<Q", 4) + struct.pack("<I", 0) + struct.pack("<Q", 0)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, 4) + kv + ti
    name, infos, base = gguf.read_gguf_header(head + bytes(200))
    assert name == "tiny" and infos == [("w", (4,), 0, 0)]
    assert base % 64 == 0 and base >= len(head) and base - len(head) < 64
