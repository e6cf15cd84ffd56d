"""Pins the CPU oracle (oracle/) before results are checked against it.

* FIPS-197 and SP 800-38D / McGrew-Viega published known answers.
* OpenSSL (the reference's host AES-128-GCM) fixtures in tests/golden/.
* Closed-form layouts of the reference's IV and AAD (secure_infer.cpp).
* The codec against the REFERENCE's own decode (fixture made by running
  optimized_decode.decode_into) and against an independent NumPy restatement.
"""
import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLD = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- AES / GCM KATs

def test_fips197_c1():
    key = bytes(range(16))
    pt = bytes.fromhex("00112233445566778899aabbccddeeff")
    assert O.aes128_encrypt_block(key, pt).hex() == "69c4e0d86a7b0430d8cdb78070b4c55a"


def test_fips197_appendix_a_key_expansion():
    rk = O.round_keys(bytes.fromhex("2b7e151628aed2a6abf7158809cf4f3c"))
    assert rk[-16:].hex() == "d014f9a8c9ee2589e13f0cc8b6630ca6"


def test_sbox_is_the_aes_sbox():
    s = O.sbox()
    assert s[0] == 0x63 and s[1] == 0x7C and s[0x53] == 0xED and s[0xFF] == 0x16
    assert sorted(s) == list(range(256))


def _gcm(key, iv12, aad, pt):
    h = O.hash_subkey(key)
    words = struct.unpack(">III", iv12) + (2,)
    return O.gcm_encrypt_tag(key, h, words, aad, pt)


def test_gcm_tc1_tc2():
    k = bytes(16)
    assert O.hash_subkey(k).hex() == "66e94bd4ef8a2c3b884cfa59ca342b2e"
    c, t = _gcm(k, bytes(12), b"", b"")
    assert t.hex() == "58e2fccefa7e3061367f1d57a4e7455a"
    c, t = _gcm(k, bytes(12), b"", bytes(16))
    assert c.tobytes().hex() == "0388dace60b6a392f328c2b971b2fe78"
    assert t.hex() == "ab6e47d42cec13bdf53a67b21257bddf"


TC3_K = bytes.fromhex("feffe9928665731c6d6a8f9467308308")
TC3_IV = bytes.fromhex("cafebabefacedbaddecaf888")
TC3_P = bytes.fromhex(
    "d9313225f88406e5a55909c5aff5269a86a7a9531534f7da2e4c303d8a318a72"
    "1c3c0c95956809532fcf0e2449a6b525b16aedf5aa0de657ba637b391aafd255")
TC3_C = (
    "42831ec2217774244b7221b784d0d49ce3aa212f2c02a4e035c17e2329aca12e"
    "21d514b25466931c7d8f6a5aac84aa051ba30b396a0aac973d58e091473f5985")


def test_gcm_tc3():
    c, t = _gcm(TC3_K, TC3_IV, b"", TC3_P)
    assert c.tobytes().hex() == TC3_C
    assert t.hex() == "4d5c2af327cd64a62cf35abd2ba6fab4"


def test_gcm_tc4_aad_and_partial_block():
    aad = bytes.fromhex("feedfacedeadbeeffeedfacedeadbeefabaddad2")
    c, t = _gcm(TC3_K, TC3_IV, aad, TC3_P[:60])
    assert c.tobytes().hex() == TC3_C[:120]
    assert t.hex() == "5bc94fbc3221a5db94fae95ae7121a47"


def test_gf128_mul_identity_and_commutativity():
    rng = np.random.default_rng(1)
    one = bytes([0x80]) + bytes(15)
    for _ in range(8):
        a = rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
        b = rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
        c = rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
        assert O.gf128_mul(a, one) == a
        assert O.gf128_mul(a, b) == O.gf128_mul(b, a)
        # distributivity over XOR
        bc = bytes(x ^ y for x, y in zip(b, c))
        lhs = O.gf128_mul(a, bc)
        rhs = bytes(x ^ y for x, y in zip(O.gf128_mul(a, b), O.gf128_mul(a, c)))
        assert lhs == rhs


def test_gf128_reduction_polynomial():
    # x^127 * x = x^128 = x^7 + x^2 + x + 1 -> bytes e1 00..00
    x127 = bytes(15) + b"\x01"
    x1 = b"\x40" + bytes(15)
    assert O.gf128_mul(x127, x1) == b"\xe1" + bytes(15)


@pytest.mark.parametrize("vec", json.loads((GOLD / "gcm_openssl_vectors.json").read_text())["vectors"],
                         ids=lambda v: str(v["bytes"]))
def test_oracle_matches_openssl_fixture(vec):
    n = vec["bytes"]
    key, iv, aad = (bytes.fromhex(vec[k]) for k in ("key", "iv", "aad"))
    pt = np.random.default_rng(vec["pt_seed"]).integers(0, 256, n, dtype=np.uint8)
    words = struct.unpack(">III", iv) + (2,)
    h = O.hash_subkey(key)
    c, tag = O.gcm_encrypt_tag(key, h, words, aad, pt)
    assert hashlib.sha256(c.tobytes()).hexdigest() == vec["ct_sha256"]
    assert tag.hex() == vec["tag"]
    st, back = O.gcm_decrypt_verify(key, h, words, aad, c, tag)
    assert st == 1 and np.array_equal(back, pt)


@pytest.mark.parametrize("n", [16, 31, 4096, 262144])
def test_oracle_matches_live_openssl(n):
    rng = np.random.default_rng(n)
    key = rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
    iv = rng.integers(0, 256, 12, dtype=np.uint8).tobytes()
    aad = rng.integers(0, 256, 64, dtype=np.uint8).tobytes()
    pt = rng.integers(0, 256, n, dtype=np.uint8)
    c1, t1 = O.ossl_gcm_encrypt(key, iv, aad, pt)
    c2, t2 = _gcm(key, iv, aad, pt)
    assert np.array_equal(c1, c2) and t1 == t2
    ok, back = O.ossl_gcm_decrypt(key, iv, aad, c1, t1)
    assert ok == 1 and np.array_equal(back, pt)


@pytest.mark.parametrize("where", ["ct", "tag", "aad"])
def test_fail_closed(where):
    rng = np.random.default_rng(3)
    key = rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
    words = (0x01020304, 5, 6, 2)
    aad = bytearray(rng.integers(0, 256, 64, dtype=np.uint8).tobytes())
    pt = rng.integers(0, 256, 1000, dtype=np.uint8)
    h = O.hash_subkey(key)
    c, tag = O.gcm_encrypt_tag(key, h, words, bytes(aad), pt)
    tag = bytearray(tag)
    if where == "ct":
        c[500] ^= 0x01
    elif where == "tag":
        tag[7] ^= 0x80
    else:
        aad[40] ^= 0x10
    st, out = O.gcm_decrypt_verify(key, h, words, bytes(aad), c, bytes(tag))
    assert st == 0 and not out.any()
    ok, _ = O.ossl_gcm_decrypt(key, O.iv12_from_words(words), bytes(aad), c, bytes(tag))
    assert ok == 0


def test_ctr_counter_wraps_in_32_bits():
    key = bytes(range(16))
    words = (1, 2, 3, 0xFFFFFFFF)
    ks = O.keystream(key, words, 48)
    blocks = [struct.pack(">IIII", 1, 2, 3, c) for c in (0xFFFFFFFF, 0, 1)]
    expect = b"".join(O.aes128_encrypt_block(key, b) for b in blocks)
    assert ks.tobytes() == expect


# ---------------------------------------------------------------- IV / AAD

def test_transfer_iv_layout():
    base = bytes.fromhex("a1b2c3d4") + bytes(12)
    iv = O.derive_transfer_iv(base, ticket=0x0102030405060708, block_offset=0, session_nonce=0)
    assert iv.hex() == "a1b2c3d4" + "0102030405060708" + "00000002"
    iv = O.derive_transfer_iv(base, ticket=1, block_offset=5, session_nonce=0x10)
    assert iv.hex() == "a1b2c3d4" + "0000000000000011" + "00000007"
    assert O.pack_iv_words(iv) == (0xA1B2C3D4, 0, 0x11, 7)


def test_aad_layout():
    aad = O.build_gcm_aad(direction=1, tensor_kind=1, layer=31, block_id=0x1234, byte_offset=0,
                          nbytes=262144, ticket=77, transfer_offset=0, session_nonce=0)
    assert len(aad) == 64
    assert aad[:8] == b"SFAD\x01\x01\x01\x00"
    assert aad[8:12] == (31).to_bytes(4, "big")
    assert aad[12:20] == (0x1234).to_bytes(8, "big")
    assert aad[20:28] == bytes(8)
    assert aad[28:36] == (262144).to_bytes(8, "big")
    assert aad[36:44] == (77).to_bytes(8, "big")
    assert aad[44:64] == bytes(20)


# ---------------------------------------------------------------- codec

CODEC = np.load(GOLD / "codec_decode_vectors.npz")


@pytest.mark.parametrize("heads", [1, 4, 8])
@pytest.mark.parametrize("bits,kind", [(8, 0), (8, 1), (4, 0), (4, 1)])
def test_codec_decode_matches_reference_fixture(heads, bits, kind):
    """decode_into's own output (optimized_decode.py:5-26) at 1, 4 and 8 kv
    heads x 128: the K (2, h, d) and V (128, h, d/64) parameter layouts are
    pinned where the head axis is not trivial."""
    pre = "" if heads == 1 else f"h{heads}_"
    pkt = CODEC[f"{pre}packet_b{bits}_k{kind}"]
    expect = CODEC[f"{pre}decoded_b{bits}_k{kind}"]
    assert expect.shape == (128, heads, 128)
    assert np.array_equal(O.codec_decode(pkt, heads, 128, bits, kind), expect)
    assert np.array_equal(O.np_codec_decode(pkt, heads, 128, bits, kind), expect)


@pytest.mark.parametrize("bits,kind", [(8, 0), (8, 1), (4, 0), (4, 1)])
def test_codec_encode_c_matches_numpy(bits, kind):
    rng = np.random.default_rng(bits * 10 + kind)
    x = O.f32_to_bf16(rng.standard_normal((128, 4, 128), dtype=np.float32) * 3)
    a = O.codec_encode(x, bits, kind, layer=5)
    b = O.np_codec_encode(x, bits, kind, layer=5)
    assert np.array_equal(a, b)
    assert np.array_equal(O.codec_encode(CODEC["block_bf16"], bits, kind, 3),
                          CODEC[f"packet_b{bits}_k{kind}"])


@pytest.mark.parametrize("bits,kind", [(8, 0), (8, 1), (4, 0), (4, 1)])
def test_codec_roundtrip_error_bound(bits, kind):
    rng = np.random.default_rng(99 + bits + kind)
    heads, dim = 2, 128
    x = O.f32_to_bf16(rng.standard_normal((128, heads, dim), dtype=np.float32))
    pkt = O.codec_encode(x, bits, kind, layer=0)
    y = O.bf16_to_f32(O.codec_decode(pkt, heads, dim, bits, kind))
    xf = O.bf16_to_f32(x)
    qb, sb, width = O.codec_sizes(bits, heads, dim)
    assert width == pkt.size and width % 16 == 0
    scale = pkt[qb:qb + sb].view(np.float32)
    smax = float(scale.max())
    # |x^ - x| <= scale/2 (+ one bf16 ulp of |x| for the final rounding)
    ulp = np.abs(xf) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(y - xf) <= smax / 2 + ulp + 1e-6)
    hdr = pkt[qb + 2 * sb:qb + 2 * sb + 16].view(np.int32)
    assert hdr.tolist() == [1, 0, kind, bits]


def test_codec_constant_group():
    x = np.full((128, 1, 128), O.f32_to_bf16(np.float32([1.5]))[0], np.uint16)
    for bits in (8, 4):
        for kind in (0, 1):
            pkt = O.codec_encode(x, bits, kind, 0)
            qb, sb, _ = O.codec_sizes(bits, 1, 128)
            assert not pkt[:qb].any()
            assert np.all(pkt[qb:qb + sb].view(np.float32) == np.float32(1e-12))
            assert np.all(pkt[qb + sb:qb + 2 * sb].view(np.float32) == np.float32(1.5))
            assert np.array_equal(O.codec_decode(pkt, 1, 128, bits, kind), x)


def nonfinite_block(seed: int, heads: int = 2, dim: int = 128) -> np.ndarray:
    """bf16 block with NaN and +-inf in a few K groups / V rows."""
    x = np.random.default_rng(seed).standard_normal((128, heads, dim), dtype=np.float32)
    x[5, 0, 3] = np.nan                        # K (t 0-63, h0, d3);   V (t5, h0, d 0-63)
    x[70, 1, 9] = np.inf                       # K (t 64-127, h1, d9); V (t70, h1, d 0-63)
    x[20, 1, 100], x[30, 1, 100] = np.inf, -np.inf  # K (t 0-63, h1, d100); V (t20 / t30, h1, d 64-127)
    x[99, 0, 64] = -np.inf                     # K (t 64-127, h0, d64); V (t99, h0, d 64-127)
    return O.f32_to_bf16(x)


def params_match(a: np.ndarray, b: np.ndarray) -> bool:
    """float32 parameter arrays equal bit for bit, NaN payloads aside."""
    fa, fb = a.view(np.float32), b.view(np.float32)
    na, nb_ = np.isnan(fa), np.isnan(fb)
    return bool(np.array_equal(na, nb_) and np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb_]))


@pytest.mark.parametrize("bits,kind", [(8, 0), (8, 1), (4, 0), (4, 1)])
def test_codec_nonfinite_inputs(bits, kind):
    # x.amin / x.amax propagate NaN (transport_codec.py:30-31): a group with a
    # NaN gets NaN scale and low, its q are 0 (round().clamp() keeps NaN and
    # the uint8 cast gives 0) and it decodes to NaN; an inf makes the scale
    # inf and the group decodes to NaN (0 * inf).  C and NumPy agree.
    x = nonfinite_block(7 + bits + kind)
    a = O.codec_encode(x, bits, kind, 1)
    b = O.np_codec_encode(x, bits, kind, 1)
    qb, sb, width = O.codec_sizes(bits, 2, 128)
    assert np.array_equal(a[:qb], b[:qb])
    assert params_match(a[qb:qb + 2 * sb], b[qb:qb + 2 * sb])
    assert np.array_equal(a[qb + 2 * sb:], b[qb + 2 * sb:])
    scale = a[qb:qb + sb].view(np.float32)
    low = a[qb + sb:qb + 2 * sb].view(np.float32)
    if kind == 0:
        nan_p, inf_p = (0 * 2 + 0) * 128 + 3, (1 * 2 + 1) * 128 + 9   # param (group, h, d)
    else:
        nan_p, inf_p = (5 * 2 + 0) * 2 + 0, (70 * 2 + 1) * 2 + 0      # param (t, h, dim group)
    assert np.isnan(scale[nan_p]) and np.isnan(low[nan_p])
    assert np.isinf(scale[inf_p])
    y = O.codec_decode(a, 2, 128, bits, kind)
    assert np.array_equal(y, O.np_codec_decode(a, 2, 128, bits, kind))
    if kind == 0:
        assert np.all(y[0:64, 0, 3] == 0x7FC0) and np.all(y[64:128, 1, 9] == 0x7FC0)
    else:
        assert np.all(y[5, 0, 0:64] == 0x7FC0) and np.all(y[70, 1, 0:64] == 0x7FC0)
    fin = np.isfinite(O.bf16_to_f32(y))
    assert fin.sum() > 0.9 * fin.size


def test_codec_widths_match_reference_shapes():
    assert O.codec_sizes(8, 8, 128)[2] == 147472
    assert O.codec_sizes(4, 8, 128)[2] == 81936
    assert O.codec_sizes(4, 4, 128)[2] == 40976
    assert O.codec_sizes(8, 4, 128)[2] == 73744


def test_int4_nibble_order():
    # element 2i in the low nibble (transport_codec.py:34, optimized_decode.py:14-16)
    x = np.zeros((128, 1, 128), np.float32)
    x[:, 0, 0] = 0.0
    x[:, 0, 1] = 1.0
    x[:, 0, 64:] = 1.0
    pkt = O.codec_encode(O.f32_to_bf16(x), 4, 1, 0)  # V: groups over dims
    assert pkt[0] == 0xF0  # elements 0 (q=0) and 1 (q=15)
