"""The session key agreement's restatement (oracle/agreement.py), pinned
before it is used to check the device code:

* X25519 against RFC 7748's test vectors (section 5.2, including the
  1- and 1000-fold iterations, and the section 6.1 Diffie-Hellman example);
  the section 5.2 second vector's output was taken from OpenSSL's X25519,
  which the test also runs;
* X25519 and keyed BLAKE2b against OpenSSL (EVP_PKEY_X25519, the BLAKE2BMAC
  EVP_MAC) on random inputs, BLAKE2b also against hashlib;
* the two halves of the exchange (key_agreement.aicpu:29-44,
  secure_infer.cpp:487-499) derive the same key and the proof checks.
"""
import ctypes as ct
import hashlib
import os

import pytest

from oracle import agreement as A
from oracle import oracle as O

h = bytes.fromhex
RFC_5_2 = [
    ("a546e36bf0527c9d3b16154b82465edd62144c0ac1fc5a18506a2244ba449ac4",
     "e6db6867583030db3594c1a424b15f7c726624ec26b3353b10a903a6d0ab1c4c",
     "c3da55379de9c6908e94ea4df28d084f32eccf03491c71f754b4075577a28552"),
    ("4b66e9d4d1b4673c5ad22691957d6af5c11b6421e0ea01d42ca4169e7918ba0d",
     "e5210f12786811d3f4b7959d0538ae2c31dbe7106fc03c3efc4cd549c715a493",
     "95cbde9476e8907d7aade45cb4b873f88b595a68799fa152e6f8f7647aac7957"),
]
ALICE = ("77076d0a7318a57d3c16c17251b26645df4c2f87ebc0992ab177fba51db92c2a",
         "8520f0098930a754748b7ddcb43ef75a0dbf3a0d26381af4eba4a98eaa9b4e6a")
BOB = ("5dab087e624a8a4b79e17f8b83800ee66f3bb1292618b6fd1c2f8b27ff88e0eb",
       "de9edb7d7b7dc1b4d35b61c2ece435373f8343c85b78674dadfc7e146f882b4f")
SHARED = "4a5d9d5ba4ce2de1728e3bf480350f25e07e21c947d19e3376f09b3c1e161742"


def ossl_x25519(k: bytes, u: bytes) -> bytes:
    out = ct.create_string_buffer(32)
    assert O.ossl().si_ossl_x25519(k, u, out) == 0
    return out.raw


def ossl_blake2b(key: bytes, msg: bytes, n: int) -> bytes:
    out = ct.create_string_buffer(n)
    assert O.ossl().si_ossl_blake2b_keyed(key, len(key), msg, len(msg), out, n) == 0
    return out.raw


@pytest.mark.parametrize("k,u,want", RFC_5_2)
def test_x25519_rfc7748_vectors(k, u, want):
    assert A.x25519(h(k), h(u)).hex() == want
    assert ossl_x25519(h(k), h(u)).hex() == want


def test_x25519_rfc7748_iterations():
    k = u = (9).to_bytes(32, "little")
    for i in range(1000):
        k, u = A.x25519(k, u), k
        if i == 0:
            assert k.hex() == "422c8e7a6227d7bca1350b3e2bb7279f7897b87bb6854b783c60e80311ae3079"
    assert k.hex() == "684cf59ba83309552800ef566f2f4d3c1c3887c49360e3875f2eb94d99532c51"


def test_x25519_rfc7748_diffie_hellman():
    assert A.public_key(h(ALICE[0])).hex() == ALICE[1]
    assert A.public_key(h(BOB[0])).hex() == BOB[1]
    assert A.x25519(h(ALICE[0]), h(BOB[1])).hex() == SHARED
    assert A.x25519(h(BOB[0]), h(ALICE[1])).hex() == SHARED


def test_restatement_matches_openssl():
    for _ in range(8):
        k, u = os.urandom(32), os.urandom(32)
        assert A.x25519(k, u) == ossl_x25519(k, u)
    for klen in (0, 16, 32, 64):
        for mlen in (0, 1, 127, 128, 129, 300):
            key, msg = os.urandom(klen), os.urandom(mlen)
            for n in (4, 16, 32, 64):
                want = hashlib.blake2b(msg, key=key, digest_size=n).digest()
                assert A.blake2b(key, n, msg) == want
                if klen:  # the MAC needs a key
                    assert ossl_blake2b(key, msg, n) == want


def test_exchange_halves_derive_one_key():
    host_secret, device_secret, challenge = os.urandom(32), os.urandom(32), os.urandom(32)
    host_public = A.public_key(host_secret)
    device_public, key, proof = A.device_half(host_public, challenge, device_secret)
    key_h, expected, salt = A.host_half(host_secret, device_public, challenge)
    assert key == key_h and proof == expected and len(salt) == 4
    # a different challenge changes the key and fails the proof
    _, key2, proof2 = A.device_half(host_public, os.urandom(32), device_secret)
    assert key2 != key and proof2 != expected
