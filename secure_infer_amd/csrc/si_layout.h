// Host-visible layouts shared by the kernels and the host code: the record
// kernel's unit geometry, the per-key context in device memory and the
// cross-workgroup GHASH accumulator.  No device code: the host library
// includes this header alone.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SI_T 256            // threads per unit = blocks per row
#define SI_U 3              // units per workgroup of the record kernel
#define SI_NT (SI_T * SI_U) // threads per workgroup of the record kernel

namespace si {

// Per-key context in device memory, built on the host.
struct GcmCtx {
    uint32_t rk[44];      // AES-128 round keys, LE column words
    uint32_t rk16[44];    // rotl16(rk)
    uint32_t te0[256];    // Te0
    uint32_t h[4];        // H, memory byte order
    uint32_t npow;        // entries of the power table that follows
    uint32_t reserved[3];
    uint4 gh4[32 * 16];   // 4-bit tables of H^SI_T
    uint4 gh4b[32 * 16];  // 4-bit tables of H^(2*SI_T)
    uint4 gh4u[32 * 16];  // 4-bit tables of H^(SI_U*SI_T)
    uint4 gh4u2[32 * 16]; // 4-bit tables of H^(2*SI_U*SI_T)
    // followed by uint4 hpow[npow]: hpow[e] = H^e in memory byte order
};

// One record's cross-workgroup GHASH accumulator; zero between launches
// (the finalising workgroup resets it).
struct RecAcc {
    uint32_t w[4];
    uint32_t count;
    uint32_t reserved[3];
};

}  // namespace si
