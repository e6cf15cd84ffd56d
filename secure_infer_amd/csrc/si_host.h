// Internal interface between the session / control-plane code (si_api.cpp)
// and the host transfer runtime (si_host.cpp).  Not part of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "secure_infer_gpu.h"

namespace si_internal {

struct SessionKeys {
    uint8_t key[16];
    uint8_t salt[4];  // IV salt, big-endian bytes
    uint64_t nonce;   // session nonce added to every ticket
    uint64_t max_record_bytes;
};

SessionKeys session_keys(const si_session* s);

// n consecutive fresh transfer tickets (process-monotonic, never 0).
uint64_t reserve_tickets(uint32_t n);

// Registers a reload issued on `stream` with the calling thread's open layer
// group; false when no group is open.
bool group_note(hipStream_t stream, uint32_t layer, uint32_t* fail_count);

}  // namespace si_internal
