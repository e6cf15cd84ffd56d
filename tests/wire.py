"""Test helpers: build reference-format wire records with OpenSSL (the
reference's host crypto) and the oracle's IV / AAD builders."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

AAD = 64


def align32(n: int) -> int:
    return (n + 31) & ~31


def stride(n: int) -> int:
    return align32(n) + 96


def record_iv(salt: bytes, ticket: int, session_nonce: int = 0) -> tuple:
    return O.pack_iv_words(O.derive_transfer_iv(salt + bytes(12), ticket, 0, session_nonce))


def build_wire(key: bytes, salt: bytes, payloads: list[np.ndarray], kinds: list[int],
               layer: int, block_ids: list[int], ticket_base: int, direction: int = 1,
               session_nonce: int = 0, use_openssl: bool = True) -> np.ndarray:
    """Encrypted wire records [ct pad32][tag][status 0][aad] for `payloads`."""
    n = payloads[0].size
    st = stride(n)
    wire = np.zeros(len(payloads) * st, np.uint8)
    h = O.hash_subkey(key)
    for r, (pt, kind, bid) in enumerate(zip(payloads, kinds, block_ids)):
        ticket = ticket_base + r
        ivw = record_iv(salt, ticket, session_nonce)
        aad = O.build_gcm_aad(direction, kind, layer, bid, 0, n, ticket, 0, session_nonce)
        if use_openssl:
            c, tag = O.ossl_gcm_encrypt(key, O.iv12_from_words(ivw), aad, pt)
        else:
            c, tag = O.gcm_encrypt_tag(key, h, ivw, aad, pt)
        o = r * st
        wire[o:o + n] = c
        wire[o + align32(n):o + align32(n) + 16] = np.frombuffer(tag, np.uint8)
        wire[o + align32(n) + 32:o + align32(n) + 96] = np.frombuffer(aad, np.uint8)
    return wire


def wire_aads(key_unused, salt, n: int, kinds, layer, block_ids, ticket_base, direction=2,
              session_nonce: int = 0) -> np.ndarray:
    """Wire records with only the AAD filled (writeback input)."""
    st = stride(n)
    wire = np.zeros(len(kinds) * st, np.uint8)
    for r, (kind, bid) in enumerate(zip(kinds, block_ids)):
        aad = O.build_gcm_aad(direction, kind, layer, bid, 0, n, ticket_base + r, 0, session_nonce)
        o = r * st + align32(n) + 32
        wire[o:o + 64] = np.frombuffer(aad, np.uint8)
    return wire


def bf16_blocks(rng: np.random.Generator, nblocks: int, heads: int, dim: int) -> np.ndarray:
    """~N(0,1) float32 rounded to bf16 (RNE), as uint16 [nblocks, 128, h, d]."""
    x = rng.standard_normal((nblocks, 128, heads, dim), dtype=np.float32)
    return O.f32_to_bf16(x)
