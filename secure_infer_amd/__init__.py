"""secure_infer for MI355X: authenticated KV reload / writeback on gfx950.

The hot path is libsecure_infer.so (hand-written HIP for gfx950 behind a
C-ABI, include/secure_infer_gpu.h); this package binds it for PyTorch-ROCm
tensors.  See ``secure_infer_amd.gcm``.
"""
from .gcm import (  # noqa: F401
    AAD_BYTES, CODEC_MODES, SI_CODEC_INT4, SI_CODEC_INT8, SI_CODEC_NONE, D2HTransfer, GcmSession,
    LayerShape, NativeTransfer, PreparedLayer, aes_ctr, auth_gate, build_gcm_aad, clear_host_ranges, codec_width,
    derive_transfer_iv, drain_h2d_profile_after_job, flush_completed_h2d_profile, pause_h2d_profile, gcm_decrypt_verify,
    gcm_encrypt_tag, gcm_verify_only, gcm_verify_xor, gcm_verify_xor_batch, ghash, GHASH_FINALIZE_TAG,
    GHASH_VERIFY_TAG, GHASH_XOR_ON_SUCCESS, key_agreement, keystream_batch,
    inject_d2h_tamper, inject_h2d_tamper, iv_words, keystream, layer_bits, new_transfer_ticket,
    reference_ticket_order, register_host_range, replay_reserve, retire_transfer_prefetches,
    set_chunk_rows, set_job_id, set_straddle_rows, transfer_prefetch_stats, wait_job_authentication,
    wire_stride, wire_tag_offset)
