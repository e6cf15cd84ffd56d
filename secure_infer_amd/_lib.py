"""ctypes binding of libsecure_infer.so (the HIP library built for gfx950).

Raises at import of the binding when the library is missing: there is no
CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as ct
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libsecure_infer.so"

_v, _u8, _u32, _u64, _sz, _i = (ct.c_void_p, ct.c_uint8, ct.c_uint32, ct.c_uint64, ct.c_size_t,
                                ct.c_int)


class SiReloadDesc(ct.Structure):
    """si_reload_desc (include/secure_infer_gpu.h)."""
    _fields_ = [
        ("wire", _v), ("wire_stride", _u64), ("bytes", _u64), ("nrec", _u32), ("n_k", _u32),
        ("iv_words", _v), ("ticket_base", _u64), ("cache_k", _v), ("cache_v", _v),
        ("slot_bytes", _u64), ("nslots", _u64), ("slots", _v), ("codec_bits", _u32),
        ("heads", _u32), ("head_dim", _u32), ("layer", _u32), ("staging", _v),
        ("fail_count", _v), ("status_out", _v), ("flags", _u32),
    ]


class SiWritebackDesc(ct.Structure):
    """si_writeback_desc (include/secure_infer_gpu.h)."""
    _fields_ = [
        ("wire", _v), ("wire_stride", _u64), ("bytes", _u64), ("nrec", _u32), ("n_k", _u32),
        ("iv_words", _v), ("ticket_base", _u64), ("cache_k", _v), ("cache_v", _v),
        ("slot_bytes", _u64), ("nslots", _u64), ("slots", _v), ("codec_bits", _u32),
        ("heads", _u32), ("head_dim", _u32), ("layer", _u32), ("staging", _v),
        ("fail_count", _v),
    ]


# name -> (argtypes, restype); every symbol declared in include/secure_infer_gpu.h
SIGNATURES = {
    "secure_infer_gpu_gcm_decrypt_verify_do": ([_v] * 7 + [_u64] + [_u32] * 4, _i),
    "secure_infer_gpu_gcm_decrypt_verify_aad_do": ([_v] * 7 + [_u64] + [_u32] * 4 + [_v, _u64], _i),
    "secure_infer_gpu_gcm_encrypt_tag_do": ([_v] * 6 + [_u64] + [_u32] * 4 + [_v, _u64], _i),
    "secure_infer_gpu_gcm_verify_only_aad_do": ([_v] * 6 + [_u64] + [_u32] * 4 + [_v, _u64], _i),
    "secure_infer_gpu_gcm_verify_xor_aad_do": ([_v] * 8 + [_u64] + [_u32] * 4 + [_v, _u64], _i),
    "secure_infer_gpu_aes_ctr_do": ([_v] * 4 + [_u64] + [_u32] * 4, _i),
    "secure_infer_gpu_keystream_do": ([_v] * 3 + [_u64] + [_u32] * 4, _i),
    "secure_infer_gpu_auth_gate_do": ([_v, _v, _v, _u64], _i),
    "secure_infer_gpu_gcm_verify_xor_do": ([_v] * 8 + [_u64] + [_u32] * 4, _i),
    "secure_infer_gpu_gcm_verify_only_do": ([_v] * 6 + [_u64] + [_u32] * 4, _i),
    "secure_infer_gpu_gcm_verify_xor_batch_do": ([_v] * 9 + [_u64, _u64, _v, _u32], _i),
    "secure_infer_gpu_keystream_batch_do": ([_v, _v, _v, _v, _u64, _u32], _i),
    "secure_infer_gpu_ghash_do": ([_v] * 10 + [_u64, _u64, _u32], _i),
    "secure_infer_gpu_key_agreement_do": ([_v] * 7, _i),
    "secure_infer_gpu_session_create": ([_v, _v, _u64, _u64, ct.POINTER(_v)], _i),
    "secure_infer_gpu_session_destroy": ([_v], _i),
    "secure_infer_gpu_session_agree": ([_u64, _u64, ct.POINTER(_v)], _i),
    "secure_infer_test_x25519": ([_v, _v, _v], _i),
    "secure_infer_test_blake2b": ([_v, _u32, _v, _u64, _v, _u32], _i),
    "secure_infer_test_context_image": ([_v, _u64, _i, _v, _u64], ct.c_int64),
    "secure_infer_gpu_session_hash_subkey": ([_v, _v], _i),
    "secure_infer_gpu_reload_layer": ([_v, _v, ct.POINTER(SiReloadDesc)], _i),
    "secure_infer_gpu_reload_layer_noalloc": ([_v, _v, ct.POINTER(SiReloadDesc)], _i),
    "secure_infer_gpu_writeback_layer": ([_v, _v, ct.POINTER(SiWritebackDesc)], _i),
    "secure_infer_gpu_time_next_layer": ([_v, _v], _i),
    "secure_infer_gpu_clock_next_layers": ([_v, _u64, _u32], _i),
    "secure_infer_gpu_clock_layers_used": ([_v, _u32], _i),
    "secure_infer_gpu_clock_rate_khz": ([_v], _i),
    "secure_infer_codec_width": ([_u32, _u32, _u32], _u64),
    "secure_infer_wire_stride": ([_u64], _u64),
    "secure_infer_new_transfer_ticket": ([], _u64),
    "secure_infer_derive_transfer_iv": ([_v, _u64, _u64, _u64, _v], _i),
    "secure_infer_register_host_range_ex": ([_v, _sz, _u32, _u32, _sz], None),
    "secure_infer_register_host_range": ([_v, _sz], None),
    "secure_infer_clear_host_ranges": ([], None),
    "secure_infer_build_gcm_aad": ([_v, _sz, _u8, _u64, _u64, _u64, _v], _i),
    "secure_infer_gcm_replay_reserve": ([_u64], _i),
    "secure_infer_h2d_layer_group_begin": ([_sz], _i),
    "secure_infer_h2d_layer_group_end": ([], _i),
    "secure_infer_recovery_wait_layer_authentication": ([_u32], _i),
    "secure_infer_recovery_track_layer": ([_u32, _v, _v], _i),
    "secure_infer_host_threads": ([], _i),
    "secure_infer_h2d_swap": ([_v, _v, _v, _u64, _u64, _v, _u64, _u64, _v, _u32, _u32, _u32, _u32,
                               _u32, _u32, _v], _i),
    "secure_infer_test_tamper_h2d": ([ct.c_int32, ct.c_int32, ct.c_int64, _u32], _i),
    "secure_infer_test_tamper_d2h": ([_u32], _i),
    "secure_infer_test_tamper_agree": ([_u32], _i),
    "secure_infer_test_noalloc_hold": ([_v, _i], _i),
    "secure_infer_test_strict_phases": ([_i], _i),
    "secure_infer_retire_transfer_prefetches": ([], None),
    "secure_infer_invalidate_transfer_prefetches": ([], None),
    "secure_infer_get_transfer_prefetch_stats": ([ct.POINTER(_u64)] * 3, None),
    "secure_infer_count_ready_unconsumed_gcm_tickets": ([], _u64),
    "secure_infer_h2d_prefetch": ([_v, _v, _u64, _u64, _v, _u32, _u32, _u32, _u32, _u32, _u32], _i),
    "secure_infer_h2d_prefetch_group": ([_v, _v, _v, _u64, _u64, _v, _u32, _u32, _u32, _u32, _u32], _i),
    "secure_infer_h2d_prefetch_layer": ([_v, _v, _v, _u64, _u64, _v, _v, _v, _u32, _u32, _u32, _u32, _u32], _i),
    "secure_infer_flush_completed_h2d_profile": ([], None),
    "secure_infer_drain_h2d_profile_after_job": ([], None),
    "secure_infer_pause_h2d_profile": ([ct.c_int], None),
    "secure_infer_recovery_set_job_id": ([_u64], None),
    "secure_infer_recovery_wait_job_authentication": ([_u64], _i),
    "secure_infer_d2h_batch_begin": ([_sz], _i),
    "secure_infer_d2h_group_begin": ([_sz], _i),
    "secure_infer_d2h_group_end": ([], _i),
    "secure_infer_d2h_batch_device_barrier": ([], _i),
    "secure_infer_d2h_batch_end": ([], _i),
    "secure_infer_d2h_swap": ([_v, _v, _v, _u64, _u64, _v, _u64, _u64, _v, _u32, _u32, _u32, _u32,
                               _u32, _u32], _i),
    "secure_infer_gpu_version": ([], ct.c_char_p),
    "secure_infer_gpu_set_chunk_rows": ([_i], _i),
    "secure_infer_gpu_set_straddle_rows": ([_i], _i),
    "secure_infer_gpu_layout": ([_u32, _u64, _u64, _u32, _v, _v, _u32], _i),
}

_lib: ct.CDLL | None = None


def load() -> ct.CDLL:
    """Returns the bound library; raises if libsecure_infer.so was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m secure_infer_amd.build` "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback")
    lib = ct.CDLL(str(LIB_PATH))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib
