"""Writes tests/golden/gcm_openssl_vectors.json with OpenSSL (libcrypto, the
reference's host AES-128-GCM, secure_infer.cpp:6486-6550).

Each vector: key, 12-B IV, 64-B AAD, the seed of a PCG64 plaintext stream,
the byte count, SHA-256 of the ciphertext and the tag.  Sizes are the
crypto_smoke.py:39 sizes plus the codec packet widths.
Run: python tests/golden/make_gcm_vectors.py
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as O  # noqa: E402

SIZES = [16, 31, 64, 1000, 32768, 40976, 81936, 147472, 262144]


def plaintext(seed: int, n: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


def main():
    rng = np.random.default_rng(20261201)
    out = []
    for i, n in enumerate(SIZES):
        key = rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
        iv = rng.integers(0, 256, 12, dtype=np.uint8).tobytes()
        aad = rng.integers(0, 256, 64, dtype=np.uint8).tobytes()
        seed = 1000 + i
        pt = plaintext(seed, n)
        c, tag = O.ossl_gcm_encrypt(key, iv, aad, pt)
        out.append(dict(bytes=n, key=key.hex(), iv=iv.hex(), aad=aad.hex(), pt_seed=seed,
                        ct_sha256=hashlib.sha256(c.tobytes()).hexdigest(), tag=tag.hex(),
                        ct_head=c[:32].tobytes().hex()))
    meta = dict(generator="OpenSSL EVP_aes_128_gcm", version=O.ossl().si_ossl_version().decode(),
                plaintext="numpy PCG64(pt_seed).integers(0,256,bytes,uint8)")
    path = Path(__file__).with_name("gcm_openssl_vectors.json")
    path.write_text(json.dumps(dict(meta=meta, vectors=out), indent=1) + "\n")
    print(path)


if __name__ == "__main__":
    main()
