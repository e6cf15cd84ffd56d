"""Python face of the CPU oracle (test infrastructure only).

Loaded by tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` to check results against.  Product code under ``secure_infer_amd/`` never
imports this module.

* ``lib``      -- ctypes bindings of ``oracle/si_oracle.c`` (FIPS-197 AES-128,
                  SP 800-38D GHASH/GCM, reference IV/AAD builders, codec).
* ``ossl``     -- ctypes bindings of ``oracle/openssl_host.c`` (OpenSSL EVP
                  AES-128-GCM as the reference's host half calls it,
                  secure_infer.cpp:6486-6550 / :2470-2547).
* ``np_codec_*`` -- an independent NumPy float32 restatement of the codec
                  (transport_codec.py:22-42, optimized_decode.py:5-26) used to
                  cross-check the C restatement.
"""
from __future__ import annotations

import ctypes as ct
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BUILD = HERE / "_build"

_u8p = ct.POINTER(ct.c_uint8)


def build() -> None:
    """Compile the oracle libraries (gcc; OpenSSL's libcrypto for the host leg)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def _load(name: str) -> ct.CDLL:
    path = BUILD / name
    if not path.exists():
        build()
    return ct.CDLL(str(path))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ct.c_void_p)


class _Lib:
    def __init__(self, cdll: ct.CDLL):
        self.c = cdll
        v, u64, u32 = ct.c_void_p, ct.c_uint64, ct.c_uint32
        sig = {
            "si_or_aes128_expand": ([v, v], None),
            "si_or_aes128_encrypt": ([v, v, v], None),
            "si_or_sbox": ([v], None),
            "si_or_gf128_mul": ([v, v, v], None),
            "si_or_ghash": ([v, v, u64, v, u64, v], None),
            "si_or_keystream": ([v, v, v, u64], None),
            "si_or_aes_ctr": ([v, v, v, v, u64], None),
            "si_or_gcm_encrypt_tag": ([v, v, v, v, u64, v, u64, v, v], None),
            "si_or_gcm_decrypt_verify": ([v, v, v, v, u64, v, u64, v, v], u32),
            "si_or_derive_transfer_iv": ([v, u64, u64, u64, v], None),
            "si_or_pack_iv_words": ([v, v], None),
            "si_or_build_gcm_aad": ([ct.c_uint8, u32, u32, u64, u64, u64, u64, u64, u64, v], None),
            "si_or_codec_qbytes": ([u32, u32, u32], u64),
            "si_or_codec_sbytes": ([u32, u32], u64),
            "si_or_codec_width": ([u32, u32, u32], u64),
            "si_or_codec_encode": ([v, u32, u32, u32, u32, u32, v], None),
            "si_or_codec_decode": ([v, u32, u32, u32, u32, v], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(cdll, name)
            fn.argtypes = args
            fn.restype = res


_lib: _Lib | None = None
_ossl: ct.CDLL | None = None


def lib() -> _Lib:
    global _lib
    if _lib is None:
        _lib = _Lib(_load("libsi_oracle.so"))
    return _lib


def ossl() -> ct.CDLL:
    global _ossl
    if _ossl is None:
        c = _load("libsi_openssl.so")
        v, u64, u32 = ct.c_void_p, ct.c_uint64, ct.c_uint32
        c.si_ossl_gcm_encrypt.argtypes = [v, v, v, u64, v, u64, v, v]
        c.si_ossl_gcm_encrypt.restype = ct.c_int
        c.si_ossl_gcm_decrypt.argtypes = [v, v, v, u64, v, u64, v, v]
        c.si_ossl_gcm_decrypt.restype = ct.c_int
        c.si_ossl_version.restype = ct.c_char_p
        c.si_ossl_layer.argtypes = [ct.c_int, v, v, v, u64, u64, u64, u64, u32, v, v, u64,
                                    v, v, u32, u32, u32, u32, v, u32]
        c.si_ossl_layer.restype = ct.c_int64
        _ossl = c
    return _ossl


def _b(x: bytes | np.ndarray) -> np.ndarray:
    if isinstance(x, np.ndarray):
        return np.ascontiguousarray(x, dtype=np.uint8)
    return np.frombuffer(bytes(x), dtype=np.uint8).copy()


def _w(words) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(words, dtype=np.uint32))


# ---------------------------------------------------------------- primitives

def aes128_encrypt_block(key: bytes, block: bytes) -> bytes:
    rk = np.zeros(176, np.uint8)
    out = np.zeros(16, np.uint8)
    k, b = _b(key), _b(block)
    lib().c.si_or_aes128_expand(_ptr(k), _ptr(rk))
    lib().c.si_or_aes128_encrypt(_ptr(rk), _ptr(b), _ptr(out))
    return out.tobytes()


def hash_subkey(key: bytes) -> bytes:
    """H = E_K(0^128) (secure_infer.cpp:549-562)."""
    return aes128_encrypt_block(key, bytes(16))


def round_keys(key: bytes) -> bytes:
    rk = np.zeros(176, np.uint8)
    lib().c.si_or_aes128_expand(_ptr(_b(key)), _ptr(rk))
    return rk.tobytes()


def sbox() -> bytes:
    out = np.zeros(256, np.uint8)
    lib().c.si_or_sbox(_ptr(out))
    return out.tobytes()


def gf128_mul(x: bytes, y: bytes) -> bytes:
    out = np.zeros(16, np.uint8)
    lib().c.si_or_gf128_mul(_ptr(_b(x)), _ptr(_b(y)), _ptr(out))
    return out.tobytes()


def ghash(h: bytes, aad: bytes, data) -> bytes:
    a, d = _b(aad), _b(data)
    out = np.zeros(16, np.uint8)
    lib().c.si_or_ghash(_ptr(_b(h)), _ptr(a), a.size, _ptr(d), d.size, _ptr(out))
    return out.tobytes()


def keystream(key: bytes, iv_words, nbytes: int) -> np.ndarray:
    out = np.zeros(nbytes, np.uint8)
    lib().c.si_or_keystream(_ptr(_b(key)), _ptr(_w(iv_words)), _ptr(out), nbytes)
    return out


def aes_ctr(key: bytes, iv_words, data) -> np.ndarray:
    d = _b(data)
    out = np.zeros_like(d)
    lib().c.si_or_aes_ctr(_ptr(_b(key)), _ptr(_w(iv_words)), _ptr(d), _ptr(out), d.size)
    return out


def gcm_encrypt_tag(key: bytes, h: bytes, iv_words, aad, pt):
    """secure_infer_gcm_encrypt_tag semantics -> (ciphertext ndarray, tag bytes)."""
    a, p = _b(aad), _b(pt)
    c = np.zeros_like(p)
    tag = np.zeros(16, np.uint8)
    lib().c.si_or_gcm_encrypt_tag(_ptr(_b(key)), _ptr(_b(h)), _ptr(_w(iv_words)), _ptr(a),
                                  a.size, _ptr(p), p.size, _ptr(c), _ptr(tag))
    return c, tag.tobytes()


def gcm_decrypt_verify(key: bytes, h: bytes, iv_words, aad, ct_, tag: bytes):
    """secure_infer_gcm_decrypt_verify semantics -> (status, masked plaintext)."""
    a, c = _b(aad), _b(ct_)
    out = np.zeros_like(c)
    st = lib().c.si_or_gcm_decrypt_verify(_ptr(_b(key)), _ptr(_b(h)), _ptr(_w(iv_words)),
                                          _ptr(a), a.size, _ptr(c), c.size, _ptr(_b(tag)),
                                          _ptr(out))
    return int(st), out


def derive_transfer_iv(base_iv: bytes, ticket: int, block_offset: int = 0,
                       session_nonce: int = 0) -> bytes:
    out = np.zeros(16, np.uint8)
    lib().c.si_or_derive_transfer_iv(_ptr(_b(base_iv)), session_nonce, ticket, block_offset,
                                     _ptr(out))
    return out.tobytes()


def pack_iv_words(iv: bytes) -> tuple:
    w = np.zeros(4, np.uint32)
    lib().c.si_or_pack_iv_words(_ptr(_b(iv)), _ptr(w))
    return tuple(int(x) for x in w)


def build_gcm_aad(direction: int, tensor_kind: int, layer: int, block_id: int,
                  byte_offset: int, nbytes: int, ticket: int, transfer_offset: int = 0,
                  session_nonce: int = 0) -> bytes:
    out = np.zeros(64, np.uint8)
    lib().c.si_or_build_gcm_aad(direction, tensor_kind, layer, block_id, byte_offset, nbytes,
                                ticket, transfer_offset, session_nonce, _ptr(out))
    return out.tobytes()


# ---------------------------------------------------------------- codec

def codec_sizes(bits: int, heads: int, dim: int) -> tuple[int, int, int]:
    c = lib().c
    return (int(c.si_or_codec_qbytes(bits, heads, dim)), int(c.si_or_codec_sbytes(heads, dim)),
            int(c.si_or_codec_width(bits, heads, dim)))


def codec_encode(block_bf16: np.ndarray, bits: int, kind: int, layer: int) -> np.ndarray:
    """block_bf16: uint16 [128, h, d] -> packet uint8 [width] (C restatement)."""
    blk = np.ascontiguousarray(block_bf16, dtype=np.uint16)
    _, h, d = blk.shape
    width = codec_sizes(bits, h, d)[2]
    out = np.zeros(width, np.uint8)
    lib().c.si_or_codec_encode(_ptr(blk), h, d, bits, kind, layer, _ptr(out))
    return out


def codec_decode(packet: np.ndarray, heads: int, dim: int, bits: int, kind: int) -> np.ndarray:
    """packet -> uint16 bf16 [128, h, d] (C restatement)."""
    p = np.ascontiguousarray(packet, dtype=np.uint8)
    out = np.zeros((128, heads, dim), np.uint16)
    lib().c.si_or_codec_decode(_ptr(p), heads, dim, bits, kind, _ptr(out))
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (torch's .to(bfloat16))."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = 0x7FC0
    return r


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    return (np.asarray(x, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _np_groups(x: np.ndarray, kind: int) -> np.ndarray:
    t, h, d = x.shape
    if kind == 0:
        return x.reshape(t // 64, 64, h, d), 1
    return x.reshape(t, h, d // 64, 64), 3


def np_codec_encode(block_bf16: np.ndarray, bits: int, kind: int, layer: int) -> np.ndarray:
    """Independent NumPy restatement of transport_codec.encode for one record."""
    x = bf16_to_f32(block_bf16)
    t, h, d = x.shape
    g, axis = _np_groups(x, kind)
    low = g.min(axis=axis, keepdims=True)
    high = g.max(axis=axis, keepdims=True)
    with np.errstate(all="ignore"):
        scale = ((high - low) / np.float32((1 << bits) - 1)).astype(np.float32)
        scale = np.maximum(scale, np.float32(1e-12))
        q = np.rint(((g - low) / scale).astype(np.float32))
    q = np.clip(q, 0, (1 << bits) - 1).reshape(-1)
    if bits == 4:  # packed in float: a NaN in either element makes the byte NaN
        q = q[0::2] + np.float32(16) * q[1::2]
    q = np.where(np.isnan(q), 0, q)  # torch's NaN -> uint8 cast gives 0 on x86
    q = q.astype(np.uint8)
    qb, sb = q.size, scale.size * 4
    width = (qb + 2 * sb + 16 + 15) // 16 * 16
    pkt = np.zeros(width, np.uint8)
    pkt[:qb] = q
    pkt[qb:qb + sb] = np.ascontiguousarray(scale.astype(np.float32)).view(np.uint8).reshape(-1)
    pkt[qb + sb:qb + 2 * sb] = np.ascontiguousarray(low.astype(np.float32)).view(np.uint8).reshape(-1)
    pkt[qb + 2 * sb:qb + 2 * sb + 16] = np.array([1, layer, kind, bits], np.int32).view(np.uint8)
    return pkt


def np_codec_decode(packet: np.ndarray, heads: int, dim: int, bits: int, kind: int) -> np.ndarray:
    """Independent NumPy restatement of optimized_decode.decode_into for one record."""
    e = 128 * heads * dim
    qb = e * bits // 8
    sb = 2 * heads * dim * 4
    pk = np.asarray(packet, dtype=np.uint8)
    if bits == 8:
        full = pk[:qb].astype(np.float32)
    else:
        p = pk[:qb].astype(np.float32)
        hi = np.floor(p / 16)
        full = np.stack((p - 16 * hi, hi), axis=-1).reshape(-1)
    params = pk[:qb + 2 * sb].view(np.float32)
    if kind == 0:
        shape, pshape = (2, 64, heads, dim), (2, 1, heads, dim)
    else:
        shape, pshape = (128, heads, dim // 64, 64), (128, heads, dim // 64, 1)
    scale = params[qb // 4:(qb + sb) // 4].reshape(pshape)
    off = params[(qb + sb) // 4:(qb + 2 * sb) // 4].reshape(pshape)
    with np.errstate(invalid="ignore", over="ignore"):  # 0 * inf, inf - inf -> NaN, as in torch
        v = (full.reshape(shape) * scale).astype(np.float32)
        v = (v + off).astype(np.float32)
    return f32_to_bf16(v.reshape(128, heads, dim))


# ---------------------------------------------------------------- OpenSSL

def ossl_gcm_encrypt(key: bytes, iv12: bytes, aad, pt):
    a, p = _b(aad), _b(pt)
    c = np.zeros_like(p)
    tag = np.zeros(16, np.uint8)
    rc = ossl().si_ossl_gcm_encrypt(_ptr(_b(key)), _ptr(_b(iv12)), _ptr(a), a.size, _ptr(p),
                                    p.size, _ptr(c), _ptr(tag))
    assert rc == 0
    return c, tag.tobytes()


def ossl_gcm_decrypt(key: bytes, iv12: bytes, aad, ct_, tag: bytes):
    a, c = _b(aad), _b(ct_)
    p = np.zeros_like(c)
    ok = ossl().si_ossl_gcm_decrypt(_ptr(_b(key)), _ptr(_b(iv12)), _ptr(a), a.size, _ptr(c),
                                    c.size, _ptr(_b(tag)), _ptr(p))
    return int(ok), p


def iv12_from_words(words) -> bytes:
    return b"".join(int(w).to_bytes(4, "big") for w in list(words)[:3])


def cpu_threads() -> int:
    return len(os.sched_getaffinity(0))
