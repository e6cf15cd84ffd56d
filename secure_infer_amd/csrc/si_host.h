// Internal interface between the session / control-plane code (si_api.cpp)
// and the host transfer runtime (si_host.cpp).  Not part of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <openssl/crypto.h>
#include <stdint.h>

#include "secure_infer_gpu.h"

namespace si_internal {

// A copy of a session's host key material; every copy (launch records,
// prefetches, D2H jobs, locals) wipes itself when it goes.
struct SessionKeys {
    uint8_t key[16];
    uint8_t salt[4];  // IV salt, big-endian bytes
    uint64_t nonce;   // session nonce added to every ticket
    uint64_t max_record_bytes;
    SessionKeys() = default;
    SessionKeys(const SessionKeys&) = default;
    SessionKeys& operator=(const SessionKeys&) = default;
    ~SessionKeys() { OPENSSL_cleanse(key, sizeof(key)); }
};

SessionKeys session_keys(const si_session* s);

// Work not yet issued that names a session (a thread's pending H2D launch or
// D2H job) holds it: secure_infer_gpu_session_destroy refuses while any
// hold remains, so no thread is left with a pointer to a freed session.
void session_hold(si_session* s);
void session_release(si_session* s);
uint32_t session_holds(const si_session* s);

class SessionHold {
public:
    SessionHold() = default;
    SessionHold(const SessionHold&) = delete;
    SessionHold& operator=(const SessionHold&) = delete;
    ~SessionHold() { reset(); }
    void take(si_session* s)
    {
        reset();
        session_hold(s);
        s_ = s;
    }
    void reset()
    {
        if (s_) session_release(s_);
        s_ = nullptr;
    }

private:
    si_session* s_ = nullptr;
};

// n consecutive fresh transfer tickets (process-monotonic, never 0).
uint64_t reserve_tickets(uint32_t n);

// Marks tickets [t0, t0 + n) as used; false if any of them was used before
// (the replay set of secure_infer_gcm_replay_reserve).
bool replay_reserve_range(uint64_t t0, uint64_t n);

// True while the calling thread is inside secure_infer_h2d_layer_group_begin/end.
bool group_open();

// The record count the calling thread's open layer group announced (-1: none).
int64_t group_expected();

// Issues the H2D swaps the calling thread's layer group has accumulated
// (copies, then one reload launch); 0 on success.
int flush_pending_h2d();

// The job id set by secure_infer_recovery_set_job_id.
uint64_t current_job_id();

// Observed H2D swaps of job `job_id` on every layer, waited for without
// retries: 1 if every record authenticated, 0 otherwise; *found is set when
// the job had observed swaps (left unchanged otherwise).
int wait_observed_job(uint64_t job_id, bool* found);

// Observed H2D swaps of `layer` (host-sealed records): waits for their
// status words, re-seals every record that failed once under a fresh ticket
// and checks it again.  0 if every record authenticated, -1 otherwise;
// *found tells whether the layer had observed swaps.
int wait_observed_layer(uint32_t layer, bool* found);

// Called when a session is destroyed: issues the calling thread's pending
// launches; if another thread still holds the session (work not issued),
// returns false and changes nothing else.  Otherwise drops the session's
// unconsumed prefetches (after their sealing tasks end), marks its observed
// swaps as not retryable (a failed record then fails its layer) and returns
// true.
bool forget_session(si_session* s);

}  // namespace si_internal
