"""CPU restatement of the session key agreement (test infrastructure only).

The reference's experimental device session (secure_infer.cpp:447-521, with
the device half in kernels/aicpu/key_agreement.aicpu:9-49) agrees on the
AES-128 session key and the 4-byte IV salt without sending either across
PCIe:

* the host draws an X25519 secret and a 32-byte challenge and sends its
  public value and the challenge;
* the device draws its own X25519 secret, computes its public value and the
  shared secret, and derives
  key   = BLAKE2b(key=shared, size 16)(info || host_public || device_public || challenge)
  proof = BLAKE2b(key=key,    size 32)(challenge)
  (info = "SecureInfer X25519 BLAKE2b test v1"), and returns its public value
  and the proof; the key stays in device memory;
* the host computes the same shared secret and key, checks the proof, and
  derives salt = BLAKE2b(key=shared, size 4)("SecureInfer IV salt v1").

X25519 is restated from RFC 7748 (section 5: the Montgomery ladder over
GF(2^255 - 19), with scalar clamping and the top bit of u masked); it is
pinned by the RFC's test vectors in tests/test_agreement.py.  BLAKE2b is
Python's hashlib.blake2b (RFC 7693, keyed mode).  Only tests/ import this
module.
"""
from __future__ import annotations

import hashlib

P = 2 ** 255 - 19
A24 = 121665
INFO = b"SecureInfer X25519 BLAKE2b test v1"
SALT_INFO = b"SecureInfer IV salt v1"


def _clamp(k: bytes) -> int:
    b = bytearray(k)
    b[0] &= 248
    b[31] &= 127
    b[31] |= 64
    return int.from_bytes(b, "little")


def x25519(scalar: bytes, u: bytes) -> bytes:
    """RFC 7748 X25519(k, u): 32-byte little-endian strings."""
    assert len(scalar) == 32 and len(u) == 32
    k = _clamp(scalar)
    x1 = int.from_bytes(u, "little") & ((1 << 255) - 1)
    x2, z2, x3, z3, swap = 1, 0, x1, 1, 0
    for t in range(254, -1, -1):
        kt = (k >> t) & 1
        swap ^= kt
        if swap:
            x2, x3, z2, z3 = x3, x2, z3, z2
        swap = kt
        a, b = (x2 + z2) % P, (x2 - z2) % P
        aa, bb = a * a % P, b * b % P
        e = (aa - bb) % P
        c, d = (x3 + z3) % P, (x3 - z3) % P
        da, cb = d * a % P, c * b % P
        x3 = (da + cb) ** 2 % P
        z3 = x1 * (da - cb) ** 2 % P
        x2 = aa * bb % P
        z2 = e * (aa + A24 * e) % P
    if swap:
        x2, z2 = x3, z3
    return (x2 * pow(z2, P - 2, P) % P).to_bytes(32, "little")


def public_key(secret: bytes) -> bytes:
    return x25519(secret, (9).to_bytes(32, "little"))


def blake2b(key: bytes, size: int, *parts: bytes) -> bytes:
    return hashlib.blake2b(b"".join(parts), key=key, digest_size=size).digest()


def device_half(host_public: bytes, challenge: bytes, device_secret: bytes):
    """(device_public, key, proof) of key_agreement.aicpu:29-44."""
    device_public = public_key(device_secret)
    shared = x25519(device_secret, host_public)
    key = blake2b(shared, 16, INFO, host_public, device_public, challenge)
    return device_public, key, blake2b(key, 32, challenge)


def host_half(host_secret: bytes, device_public: bytes, challenge: bytes):
    """(key, expected proof, salt) of secure_infer.cpp:487-499."""
    host_public = public_key(host_secret)
    shared = x25519(host_secret, device_public)
    key = blake2b(shared, 16, INFO, host_public, device_public, challenge)
    return key, blake2b(key, 32, challenge), blake2b(shared, 4, SALT_INFO)
