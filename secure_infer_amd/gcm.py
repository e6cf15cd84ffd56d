"""Python face of libsecure_infer.so on PyTorch-ROCm tensors.

* Kernel-level calls mirror the reference's device launchers
  (secure_infer/native/kernels/aicpu/launcher.asc) one record at a time.
* ``GcmSession`` owns a device-resident AES-128 key with its GHASH tables and
  runs the fused per-layer reload / writeback kernels.
* ``NativeTransfer`` mirrors ``native_layerwise.NativeTransfer`` (per-layer
  authenticated reload into the paged cache, native_layerwise.py:85-130) and
  the per-layer authentication wait the reuse schedulers block on
  (``secure_infer_recovery_wait_layer_authentication``, secure_infer.cpp:7303).

All tensors handed to the library are CUDA (HIP) tensors; every call is
asynchronous on the given (default: current) stream.
"""
from __future__ import annotations

import ctypes as ct
import math
import struct
from dataclasses import dataclass

import torch

from . import _lib

AAD_BYTES = 64
SI_CODEC_NONE, SI_CODEC_INT8, SI_CODEC_INT4 = 0, 8, 4
SI_RELOAD_VERIFY_BEFORE_RELEASE = 1  # si_reload_desc.flags (include/secure_infer_gpu.h)


def lib():
    return _lib.load()


def _p(t: torch.Tensor | None):
    return None if t is None else ct.c_void_p(t.data_ptr())


def _stream(stream) -> ct.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return ct.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed (rc={rc})")


def _dev(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ------------------------------------------------------------------ wire layout

def wire_tag_offset(nbytes: int) -> int:
    """Ciphertext area of a wire record is padded to 32 B (secure_infer.cpp:6319-6320)."""
    return (nbytes + 31) & ~31


def wire_stride(nbytes: int) -> int:
    """[ct pad32][tag 16][status 16][AAD 64] (secure_infer.cpp:6379-6388)."""
    return int(lib().secure_infer_wire_stride(nbytes))


def codec_width(bits: int, heads: int, head_dim: int) -> int:
    return int(lib().secure_infer_codec_width(bits, heads, head_dim))


# ------------------------------------------------------------------ control plane

def new_transfer_ticket() -> int:
    return int(lib().secure_infer_new_transfer_ticket())


def derive_transfer_iv(base_iv: bytes, ticket: int, block_offset: int = 0,
                       session_nonce: int = 0) -> bytes:
    out = (ct.c_uint8 * 16)()
    base = (ct.c_uint8 * 16).from_buffer_copy(bytes(base_iv).ljust(16, b"\0"))
    _check(lib().secure_infer_derive_transfer_iv(base, session_nonce, ticket, block_offset, out),
           "derive_transfer_iv")
    return bytes(out)


def iv_words(iv: bytes) -> tuple[int, int, int, int]:
    """pack_inline_iv: four big-endian words (secure_infer.cpp:2083-2093)."""
    return struct.unpack(">IIII", bytes(iv[:16]))


def register_host_range(tensor: torch.Tensor, layer_id: int, tensor_kind: int) -> None:
    """_register_host_range (npu_predict.py:384-408)."""
    block_bytes = tensor[0].numel() * tensor.element_size() if tensor.ndim and tensor.shape[0] else 0
    lib().secure_infer_register_host_range_ex(ct.c_void_p(tensor.data_ptr()),
                                              tensor.numel() * tensor.element_size(),
                                              layer_id, tensor_kind, block_bytes)


def clear_host_ranges() -> None:
    lib().secure_infer_clear_host_ranges()


def build_gcm_aad(host_ptr: int, nbytes: int, direction: int, ticket: int,
                  transfer_offset: int = 0, session_nonce: int = 0) -> bytes:
    out = (ct.c_uint8 * 64)()
    ok = lib().secure_infer_build_gcm_aad(ct.c_void_p(host_ptr), nbytes, direction, ticket,
                                          transfer_offset, session_nonce, out)
    if ok != 1:
        raise ValueError("invalid AAD request")
    return bytes(out)


def replay_reserve(ticket: int) -> bool:
    return lib().secure_infer_gcm_replay_reserve(ticket) == 1


# ------------------------------------------------------------------ kernel-level mirrors

def gcm_decrypt_verify(ciphertext, key, hash_subkey, expected_tag, plaintext_out, status_out,
                       iv, aad=None, nbytes=None, stream=None) -> None:
    """secure_infer_aicpu_gcm_decrypt_verify[_aad]_do (launcher.asc:214-275)."""
    n = ciphertext.numel() if nbytes is None else nbytes
    a = 0 if aad is None else aad.numel()
    _check(lib().secure_infer_gpu_gcm_decrypt_verify_aad_do(
        _stream(stream), _p(ciphertext), _p(key), _p(hash_subkey), _p(expected_tag),
        _p(plaintext_out), _p(status_out), n, *iv, _p(aad), a), "gcm_decrypt_verify")


def gcm_encrypt_tag(plaintext, key, hash_subkey, ciphertext_out, tag_out, iv, aad=None,
                    nbytes=None, stream=None) -> None:
    """secure_infer_aicpu_gcm_encrypt_tag_do (launcher.asc:279-308)."""
    n = plaintext.numel() if nbytes is None else nbytes
    a = 0 if aad is None else aad.numel()
    _check(lib().secure_infer_gpu_gcm_encrypt_tag_do(
        _stream(stream), _p(plaintext), _p(key), _p(hash_subkey), _p(ciphertext_out), _p(tag_out),
        n, *iv, _p(aad), a), "gcm_encrypt_tag")


def gcm_verify_only(ciphertext, key, hash_subkey, expected_tag, status_out, iv, aad=None,
                    stream=None) -> None:
    """secure_infer_aicpu_gcm_verify_only[_aad]_do (launcher.asc:378-435): the
    AAD-less launcher when aad is None."""
    if aad is None:
        _check(lib().secure_infer_gpu_gcm_verify_only_do(
            _stream(stream), _p(ciphertext), _p(key), _p(hash_subkey), _p(expected_tag),
            _p(status_out), ciphertext.numel(), *iv), "gcm_verify_only")
        return
    _check(lib().secure_infer_gpu_gcm_verify_only_aad_do(
        _stream(stream), _p(ciphertext), _p(key), _p(hash_subkey), _p(expected_tag),
        _p(status_out), ciphertext.numel(), *iv, _p(aad), aad.numel()), "gcm_verify_only")


def gcm_verify_xor(ciphertext, key, hash_subkey, expected_tag, keystream, plaintext_out,
                   status_out, iv, aad=None, stream=None) -> None:
    """secure_infer_aicpu_gcm_verify_xor[_aad]_do (launcher.asc:312-376): the
    AAD-less launcher when aad is None."""
    if aad is None:
        _check(lib().secure_infer_gpu_gcm_verify_xor_do(
            _stream(stream), _p(ciphertext), _p(key), _p(hash_subkey), _p(expected_tag),
            _p(keystream), _p(plaintext_out), _p(status_out), ciphertext.numel(), *iv),
            "gcm_verify_xor")
        return
    _check(lib().secure_infer_gpu_gcm_verify_xor_aad_do(
        _stream(stream), _p(ciphertext), _p(key), _p(hash_subkey), _p(expected_tag),
        _p(keystream), _p(plaintext_out), _p(status_out), ciphertext.numel(), *iv, _p(aad),
        aad.numel()), "gcm_verify_xor")


def _ptrs(tensors):
    return (ct.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


def _iv_array(ivs):
    return (ct.c_uint32 * (4 * len(ivs)))(*[w for iv in ivs for w in iv])


def gcm_verify_xor_batch(key, hash_subkey, ciphertexts, expected_tags, keystreams, plaintext_outs,
                         status_outs, ivs, aads=None, stream=None) -> None:
    """secure_infer_aicpu_gcm_verify_xor_batch_do (launcher.asc:440-486): up to
    four same-size records under one key, each verified and released."""
    n = ciphertexts[0].numel()
    a = 0 if aads is None else aads[0].numel()
    _check(lib().secure_infer_gpu_gcm_verify_xor_batch_do(
        _stream(stream), _p(key), _p(hash_subkey), _ptrs(ciphertexts), _ptrs(expected_tags),
        _ptrs(keystreams), _ptrs(plaintext_outs), _ptrs(status_outs),
        None if aads is None else _ptrs(aads), n, a, _iv_array(ivs), len(ciphertexts)),
        "gcm_verify_xor_batch")


def keystream_batch(key, outs, ivs, stream=None) -> None:
    """secure_infer_aicpu_keystream_batch_do (launcher.asc:184-210)."""
    _check(lib().secure_infer_gpu_keystream_batch_do(
        _stream(stream), _p(key), _ptrs(outs), _iv_array(ivs), outs[0].numel(), len(outs)),
        "keystream_batch")


GHASH_FINALIZE_TAG, GHASH_VERIFY_TAG, GHASH_XOR_ON_SUCCESS = 1, 2, 4


def ghash(inp, hash_subkey, out, aad=None, tag_mask=None, expected_tag=None, keystream=None,
          plaintext_out=None, status_out=None, flags=0, nbytes=None, stream=None) -> None:
    """secure_infer_aicpu_ghash_do (launcher.asc:75-114, ghash.aicpu:978-1045)."""
    n = inp.numel() if nbytes is None else nbytes
    a = 0 if aad is None else aad.numel()
    _check(lib().secure_infer_gpu_ghash_do(
        _stream(stream), _p(inp), _p(hash_subkey), _p(out), _p(aad), _p(tag_mask), _p(expected_tag),
        _p(keystream), _p(plaintext_out), _p(status_out), n, a, flags), "ghash")


def key_agreement(host_public, challenge, device_key, device_public, proof, status,
                  stream=None) -> None:
    """secure_infer_aicpu_key_agreement_do (launcher.asc:19-32): the device half
    of the session agreement on device buffers."""
    _check(lib().secure_infer_gpu_key_agreement_do(
        _stream(stream), _p(host_public), _p(challenge), _p(device_key), _p(device_public),
        _p(proof), _p(status)), "key_agreement")


def aes_ctr(inp, key, out, iv, stream=None) -> None:
    """secure_infer_aicpu_aes_ctr_do (launcher.asc:134-155)."""
    _check(lib().secure_infer_gpu_aes_ctr_do(_stream(stream), _p(inp), _p(key), _p(out),
                                             inp.numel(), *iv), "aes_ctr")


def keystream(key, out, iv, stream=None) -> None:
    """secure_infer_aicpu_keystream_do (launcher.asc:160-179)."""
    _check(lib().secure_infer_gpu_keystream_do(_stream(stream), _p(key), _p(out), out.numel(), *iv),
           "keystream")


def auth_gate(data, status, stream=None) -> None:
    """secure_infer_aicpu_auth_gate_do (launcher.asc:116-132)."""
    _check(lib().secure_infer_gpu_auth_gate_do(_stream(stream), _p(data), _p(status),
                                               data.numel() * data.element_size()), "auth_gate")


# ------------------------------------------------------------------ sessions

CODEC_MODES = ("none", "int8", "int4", "mixed")


def layer_bits(mode: str, layer: int, layers: int) -> int:
    """Codec bits of one layer (transport_codec.layer_bits, transport_codec.py:18-19):
    ``mixed`` keeps int8 for the first ceil(L/3) layers and int4 after them."""
    if mode not in CODEC_MODES:
        raise ValueError(f"codec mode {mode!r} not in {CODEC_MODES}")
    if mode == "none":
        return SI_CODEC_NONE
    return SI_CODEC_INT8 if mode == "int8" or (mode == "mixed" and layer < math.ceil(layers / 3)) \
        else SI_CODEC_INT4


@dataclass
class LayerShape:
    """Geometry of one layer's records: kv heads x head_dim per token, and the
    transport codec -- either fixed bits for every layer (``codec_bits``) or a
    reference codec mode (``codec`` in none / int8 / int4 / mixed) over
    ``layers`` layers."""
    heads: int
    head_dim: int
    codec_bits: int = SI_CODEC_NONE
    codec: str | None = None
    layers: int | None = None

    def __post_init__(self):
        if self.codec is not None:
            if self.codec not in CODEC_MODES:
                raise ValueError(f"codec mode {self.codec!r} not in {CODEC_MODES}")
            if self.codec == "mixed" and not self.layers:
                raise ValueError("the mixed codec needs the layer count")

    def bits_for(self, layer: int) -> int:
        if self.codec is None:
            return self.codec_bits
        return layer_bits(self.codec, layer, self.layers or 1)

    @property
    def block_bytes(self) -> int:
        return 128 * self.heads * self.head_dim * 2

    def record_bytes_for(self, layer: int) -> int:
        bits = self.bits_for(layer)
        if bits == SI_CODEC_NONE:
            return self.block_bytes
        return codec_width(bits, self.heads, self.head_dim)

    @property
    def record_bytes(self) -> int:
        if self.codec == "mixed":
            raise ValueError("record size depends on the layer under the mixed codec: use record_bytes_for")
        return self.record_bytes_for(0)


class GcmSession:
    """One AES-128-GCM session: key and GHASH tables resident on the device.

    IV of the record with ticket t: salt[4] || BE64(session_nonce + t) || BE32(2)
    (secure_infer_derive_transfer_iv, secure_infer.cpp:274-300).
    """

    def __init__(self, key: bytes, iv_salt: bytes, session_nonce: int = 0,
                 max_record_bytes: int = 1 << 20):
        if len(key) < 16 or len(iv_salt) < 4:
            raise ValueError("key needs 16 bytes and iv_salt 4 bytes")
        self.key = bytes(key[:16])
        self.iv_salt = bytes(iv_salt[:4])
        self.session_nonce = int(session_nonce)
        self.max_record_bytes = int(max_record_bytes)
        h = ct.c_void_p()
        kb = (ct.c_uint8 * 16).from_buffer_copy(self.key)
        sb = (ct.c_uint8 * 4).from_buffer_copy(self.iv_salt)
        _check(lib().secure_infer_gpu_session_create(kb, sb, self.session_nonce,
                                                     self.max_record_bytes, ct.byref(h)),
               "session_create")
        self._h = h
        out = (ct.c_uint8 * 16)()
        _check(lib().secure_infer_gpu_session_hash_subkey(self._h, out), "hash_subkey")
        self.hash_subkey = bytes(out)

    @classmethod
    def agree(cls, session_nonce: int = 0, max_record_bytes: int = 1 << 20) -> "GcmSession":
        """A session whose key and IV salt are agreed with the device by an
        X25519 + BLAKE2b exchange (the reference's device session,
        secure_infer.cpp:447-521, key_agreement.aicpu:9-49): the key is
        derived on the device and never crosses PCIe; the library's host
        runtime keeps its own copy for OpenSSL.  ``key`` and ``iv_salt`` are
        None: nothing outside the library learns them."""
        self = cls.__new__(cls)
        self.key = None
        self.iv_salt = None
        self.session_nonce = int(session_nonce)
        self.max_record_bytes = int(max_record_bytes)
        h = ct.c_void_p()
        self._h = ct.c_void_p()
        _check(lib().secure_infer_gpu_session_agree(self.session_nonce, self.max_record_bytes, ct.byref(h)),
               "session_agree")
        self._h = h
        out = (ct.c_uint8 * 16)()
        _check(lib().secure_infer_gpu_session_hash_subkey(self._h, out), "hash_subkey")
        self.hash_subkey = bytes(out)
        return self

    def close(self) -> None:
        """Destroys the session; raises (and keeps it) while another thread
        still has swaps of it that were not issued (an open layer group or
        D2H batch)."""
        if self._h:
            _check(lib().secure_infer_gpu_session_destroy(self._h), "session_destroy (session still in use)")
            self._h = ct.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def base_iv(self) -> bytes:
        return self.iv_salt + bytes(12)

    def record_iv(self, ticket: int) -> tuple[int, int, int, int]:
        return iv_words(derive_transfer_iv(self.base_iv(), ticket, 0, self.session_nonce))

    def prepare_reload_layer(self, wire: torch.Tensor, nbytes: int, nrec: int, n_k: int,
                             cache_k: torch.Tensor, cache_v: torch.Tensor, slots: torch.Tensor,
                             ticket_base: int = 0, iv_words_dev: torch.Tensor | None = None,
                             codec_bits: int = SI_CODEC_NONE, heads: int = 0, head_dim: int = 0,
                             layer: int = 0, staging: torch.Tensor | None = None,
                             fail_count: torch.Tensor | None = None,
                             verify_before_release: bool = False) -> "PreparedLayer":
        """The checked descriptor of one reload layer, launched by
        ``.launch(stream)`` as often as needed (buffers with fixed addresses, as
        a serving loop keeps them); the tensors are kept alive with it.
        ``verify_before_release`` selects SI_RELOAD_VERIFY_BEFORE_RELEASE: every
        tag is checked before any plaintext reaches the cache (two launches)."""
        for t, name in ((wire, "wire"), (cache_k, "cache_k"), (cache_v, "cache_v"),
                        (slots, "slots")):
            _dev(t, name)
        if slots.dtype != torch.int64 or slots.numel() < nrec:
            raise ValueError("slots must be int64 with one entry per record")
        stride = wire_stride(nbytes)
        if wire.numel() * wire.element_size() < nrec * stride:
            raise ValueError("wire buffer too small")
        if codec_bits and (staging is None or staging.numel() * staging.element_size()
                           < nrec * wire_tag_offset(nbytes)):
            raise ValueError("codec reload needs a staging buffer of nrec*align32(bytes)")
        d = _lib.SiReloadDesc(
            wire=wire.data_ptr(), wire_stride=stride, bytes=nbytes, nrec=nrec, n_k=n_k,
            iv_words=None if iv_words_dev is None else iv_words_dev.data_ptr(),
            ticket_base=ticket_base, cache_k=cache_k.data_ptr(), cache_v=cache_v.data_ptr(),
            slot_bytes=cache_k[0].numel() * cache_k.element_size(),
            nslots=min(cache_k.shape[0], cache_v.shape[0]), slots=slots.data_ptr(),
            codec_bits=codec_bits, heads=heads, head_dim=head_dim, layer=layer,
            staging=None if staging is None else staging.data_ptr(),
            fail_count=None if fail_count is None else fail_count.data_ptr(),
            flags=SI_RELOAD_VERIFY_BEFORE_RELEASE if verify_before_release else 0)
        return PreparedLayer(lib().secure_infer_gpu_reload_layer, self, d,
                             (wire, cache_k, cache_v, slots, iv_words_dev, staging, fail_count), "reload_layer")

    def reload_layer(self, wire: torch.Tensor, nbytes: int, nrec: int, n_k: int,
                     cache_k: torch.Tensor, cache_v: torch.Tensor, slots: torch.Tensor,
                     ticket_base: int = 0, iv_words_dev: torch.Tensor | None = None,
                     codec_bits: int = SI_CODEC_NONE, heads: int = 0, head_dim: int = 0,
                     layer: int = 0, staging: torch.Tensor | None = None,
                     fail_count: torch.Tensor | None = None, stream=None,
                     verify_before_release: bool = False) -> None:
        """One layer of authenticated reload of device-resident wire records
        (secure_infer_gpu_reload_layer); arguments as prepare_reload_layer."""
        self.prepare_reload_layer(wire, nbytes, nrec, n_k, cache_k, cache_v, slots, ticket_base, iv_words_dev,
                                  codec_bits, heads, head_dim, layer, staging, fail_count,
                                  verify_before_release).launch(stream)

    def prepare_writeback_layer(self, wire: torch.Tensor, nbytes: int, nrec: int, n_k: int,
                                cache_k: torch.Tensor, cache_v: torch.Tensor, slots: torch.Tensor,
                                ticket_base: int = 0, iv_words_dev: torch.Tensor | None = None,
                                codec_bits: int = SI_CODEC_NONE, heads: int = 0, head_dim: int = 0,
                                layer: int = 0, staging: torch.Tensor | None = None,
                                fail_count: torch.Tensor | None = None) -> "PreparedLayer":
        """The checked descriptor of one writeback layer (see prepare_reload_layer)."""
        for t, name in ((wire, "wire"), (cache_k, "cache_k"), (cache_v, "cache_v"),
                        (slots, "slots")):
            _dev(t, name)
        stride = wire_stride(nbytes)
        if wire.numel() * wire.element_size() < nrec * stride:
            raise ValueError("wire buffer too small")
        if codec_bits and staging is None:
            raise ValueError("codec writeback needs a staging buffer")
        d = _lib.SiWritebackDesc(
            wire=wire.data_ptr(), wire_stride=stride, bytes=nbytes, nrec=nrec, n_k=n_k,
            iv_words=None if iv_words_dev is None else iv_words_dev.data_ptr(),
            ticket_base=ticket_base, cache_k=cache_k.data_ptr(), cache_v=cache_v.data_ptr(),
            slot_bytes=cache_k[0].numel() * cache_k.element_size(),
            nslots=min(cache_k.shape[0], cache_v.shape[0]), slots=slots.data_ptr(),
            codec_bits=codec_bits, heads=heads, head_dim=head_dim, layer=layer,
            staging=None if staging is None else staging.data_ptr(),
            fail_count=None if fail_count is None else fail_count.data_ptr())
        return PreparedLayer(lib().secure_infer_gpu_writeback_layer, self, d,
                             (wire, cache_k, cache_v, slots, iv_words_dev, staging, fail_count), "writeback_layer")

    def writeback_layer(self, wire: torch.Tensor, nbytes: int, nrec: int, n_k: int,
                        cache_k: torch.Tensor, cache_v: torch.Tensor, slots: torch.Tensor,
                        ticket_base: int = 0, iv_words_dev: torch.Tensor | None = None,
                        codec_bits: int = SI_CODEC_NONE, heads: int = 0, head_dim: int = 0,
                        layer: int = 0, staging: torch.Tensor | None = None,
                        fail_count: torch.Tensor | None = None, stream=None) -> None:
        """One layer of gather (+ quantise) + seal into device wire records
        (secure_infer_gpu_writeback_layer); arguments as prepare_writeback_layer."""
        self.prepare_writeback_layer(wire, nbytes, nrec, n_k, cache_k, cache_v, slots, ticket_base,
                                     iv_words_dev, codec_bits, heads, head_dim, layer, staging,
                                     fail_count).launch(stream)


class PreparedLayer:
    """A layer launch whose descriptor was built and checked once: launch()
    only calls the library, where reload_layer() / writeback_layer() rebuild
    and re-check the descriptor on every call."""

    def __init__(self, fn, session: GcmSession, desc, keep, what: str):
        self._fn = fn
        self._session = session
        self._desc = desc
        self._ref = ct.byref(desc)
        self._keep = keep
        self._what = what

    def launch(self, stream=None) -> None:
        """On `stream` (a torch stream, a raw handle, a ct.c_void_p, or None
        for the current stream)."""
        h = stream if isinstance(stream, ct.c_void_p) else _stream(stream)
        _check(self._fn(h, self._session._h, self._ref), self._what)


DEFAULT_CHUNK_ROWS = 3
DEFAULT_STRADDLE_ROWS = 6


def set_chunk_rows(jmax: int) -> None:
    """Minimum rows (of 256 blocks) per workgroup share of a layer (1..256)."""
    _check(lib().secure_infer_gpu_set_chunk_rows(jmax), "set_chunk_rows")


def set_straddle_rows(rows: int) -> None:
    """Cost, in rows, charged to a share that straddles two records (0..256)."""
    _check(lib().secure_infer_gpu_set_straddle_rows(rows), "set_straddle_rows")


def reference_ticket_order(nblocks: int, group_blocks: int) -> list[tuple[int, int]]:
    """(kind, block) of a layer's records in the order NativeTransfer submits
    them, i.e. the order their tickets follow: groups of ``group_blocks``
    (0: one group) from the tail, K then V within a group, blocks ascending
    (native_layerwise.py:96-129 with one slice stream)."""
    order = []
    end = nblocks
    g = group_blocks if group_blocks and nblocks > group_blocks else nblocks
    while end > 0:
        start = max(0, end - g)
        for kind in (0, 1):
            order.extend((kind, b) for b in range(start, end))
        end = start
    return order


def _torch_stream(stream):
    return stream if stream is not None else torch.cuda.current_stream()


class NativeTransfer:
    """Per-layer authenticated reload driver (native_layerwise.py:85-130).

    ``single_layer_kv_transfer((host, mapping), destination)`` has the
    reference's contract: ``host`` = (cpu_k, cpu_v) host pools of this layer
    ([num_cpu_blocks, 128, h, d] bf16, or packet arrays [num_cpu_blocks,
    width] uint8 with a codec), ``mapping`` = the [N, 2] int64 (cpu_block,
    gpu_slot) table of swap_blocks, ``destination`` = (cache_k, cache_v) device
    paged caches [num_slots, 128, h, d].

    * With ``causal_group_blocks`` = G (the reference sets RUNTIME_LOAD_CHUNK /
      128, connector.py:288) a layer's mapping is cut into groups of G blocks
      submitted tail first, each inside its own layer-group brackets
      (native_layerwise.py:96-112); records therefore take tickets in
      (layer, group, kind, slice, block) order.
    * With ``stripe`` each group stripes its rows over the slice ``streams``
      (native_layerwise.py:113-129): every slice stream first waits for the
      caller's stream, and the caller's stream waits for all of them after
      the submission, so attention on the caller's stream is ordered after
      the reload.  Without it (the default) a group's rows all go to the
      first slice stream in the same order, so records take the same
      tickets, and the group stays one launch: the reference stripes to run
      several AICPU GHASH chains at once, where one launch here already
      spans every CU (MI355X, int4 Qwen2.5-7B records, three slice streams:
      24 launches per layer instead of 4, 1,037-1,099 instead of 174-180 us
      per layer end to end sealed ahead of demand).
    * Each (kind, slice) is sealed on the host (OpenSSL, worker pool), copied
      through the slice stream's pinned ring and verified / decrypted /
      scattered on the device; a group's K and V swaps of one stream go out
      as one copy sequence and one launch at the group's end.  The call
      returns once the work is queued.  With ``pipeline_seal`` (default) the
      layer's seals are queued on the worker pool first, so later parts seal
      while earlier parts are copied (the reference's CPU ciphertext
      prefetch, secure_infer.cpp:3264-3710; one MI355X, 16 host CPUs, groups
      of 16 blocks: 41-KB int4 records 545 -> 406 us per 28-layer-model layer
      end to end, 256-KB bf16 records 831 -> 553 us).  A layer already sealed
      with ``prefetch_kv_transfer`` is not sealed again.
      ``wait_layer`` returns the layer's authentication result after at most
      one strict retry per failed record (wait_for_layer_load,
      connector.py:378-410; secure_infer.cpp:7303-7333).
    * With ``codec_auth_wait`` a codec layer's transfer returns only once the
      layer has authenticated (``wait_layer``, strict retries included) and
      raises ``RuntimeError('Packed KV authentication failed')`` otherwise:
      the reference's codec transfer asserts ``wait_auth(layer) == 0`` before
      it decodes a layer (transport_codec.py:168-174, pipelined_codec.py:118).
      Here the device decodes in the same launch sequence, stream-ordered
      after the verification (a failed record decodes to zeros); with
      SECURE_INFER_VERIFY_BEFORE_RELEASE=1 it also releases no record's
      plaintext before that record's tag has been checked.  The transfer is
      then synchronous per codec layer, as the reference's is.

    ``single_layer_wire_transfer((wire, mapping), destination, ticket_base)``
    reloads records already resident on the device (K blocks then V blocks,
    tickets ticket_base .. ticket_base+2N-1, or explicit per-record IV words);
    a failure among them is final (there is no host copy to retry from).
    """

    def __init__(self, session: GcmSession, shape: LayerShape, stream=None, streams=None,
                 causal_group_blocks: int = 0, pipeline_seal: bool = True, stripe: bool = False,
                 merge_groups: bool = False, codec_auth_wait: bool = False):
        self.session = session
        self.shape = shape
        self.stream = stream
        self.streams = list(streams) if streams else [stream]
        self.stripe = bool(stripe)
        self.merge_groups = bool(merge_groups)
        self.codec_auth_wait = bool(codec_auth_wait)
        self.causal_group_blocks = int(causal_group_blocks)
        self.pipeline_seal = pipeline_seal
        self.layer = 0
        self._keep = {}
        self._staging = None
        self._prefetched = set()

    def _plan(self, mapping: torch.Tensor):
        """Groups of (kind, slice index, address of the mapping part, rows) in
        submission order: causal groups of ``causal_group_blocks`` from the
        tail, then K / V, then the slice streams' stripes.  A part is a row
        range of the contiguous [N, 2] int64 mapping, passed by address (a
        torch slice and copy per part cost ~25 us per layer in Python)."""
        n = int(mapping.shape[0])
        base = mapping.data_ptr()
        group = self.causal_group_blocks
        g = group if group and n > group else n
        nsl = len(self.streams) if self.stripe else 1
        plan, end = [], n
        while end > 0:
            start = max(0, end - g)
            k = end - start
            parts = []
            for kind in (0, 1):
                for j in range(nsl):
                    r0, r1 = start + k * j // nsl, start + k * (j + 1) // nsl
                    if r1 > r0:
                        parts.append((kind, j, ct.c_void_p(base + 16 * r0), r1 - r0))
            plan.append((k, parts))
            end = start
        return plan

    @staticmethod
    def _check_mapping(host, mapping: torch.Tensor, destination) -> None:
        """The swaps refuse ids outside either pool before sealing anything;
        sealing ahead must not spend tickets on a mapping they refuse.
        (numpy: a torch reduction would wake torch's CPU thread pool, whose
        spinning threads then compete with the sealing workers.)"""
        m = mapping.numpy()
        lo, hi = m.min(0), m.max(0)
        if (lo[0] < 0 or hi[0] >= min(host[0].shape[0], host[1].shape[0]) or lo[1] < 0
                or hi[1] >= min(destination[0].shape[0], destination[1].shape[0])):
            raise RuntimeError("h2d_swap refused: a mapping entry lies outside its pool")

    @staticmethod
    def _host_pool(src: torch.Tensor) -> torch.Tensor:
        if src.is_cuda or not src.is_contiguous():
            raise ValueError("host pools must be contiguous CPU tensors")
        return src

    def single_layer_kv_transfer(self, payload, destination, *unused) -> None:
        host, mapping = payload
        mapping = mapping.to(device="cpu", dtype=torch.int64).contiguous()
        plan = self._plan(mapping)
        if not plan:
            self.layer += 1
            return
        if self.layer in self._prefetched:
            self._prefetched.discard(self.layer)
        elif self.pipeline_seal and (len(plan) > 1 or len(plan[0][1]) > 1):
            self._check_mapping(host, mapping, destination)
            self.prefetch_kv_transfer(payload, self.layer)
            self._prefetched.discard(self.layer)
        bits = self.shape.bits_for(self.layer)
        parent = torch.cuda.current_stream()
        streams = [_torch_stream(s) for s in (self.streams if self.stripe else self.streams[:1])]
        for st in streams:
            if st != parent:
                st.wait_stream(parent)
        # Per-kind pool arguments and stream handles, computed once per layer.
        pools = []
        for kind in (0, 1):
            src, dst = self._host_pool(host[kind]), destination[kind]
            _dev(dst, "destination cache")
            pools.append((ct.c_void_p(src.data_ptr()), src.stride(0) * src.element_size(), src.shape[0],
                          ct.c_void_p(dst.data_ptr()), dst.stride(0) * dst.element_size(), dst.shape[0]))
        handles = [_stream(st) for st in streams]
        L = lib()
        swap, h = L.secure_infer_h2d_swap, self.session._h
        heads, dim, layer = self.shape.heads, self.shape.head_dim, self.layer
        # merge_groups: one layer group around every causal group of the layer
        # (same swaps, same order, same tickets), so the layer goes to the
        # device as one launch; otherwise one per causal group, the
        # reference's grouping (native_layerwise.py:96-112).
        brackets = [(sum(k for k, _ in plan), [p for _, parts in plan for p in parts])] if self.merge_groups \
            else plan
        for k, parts in brackets:
            _check(L.secure_infer_h2d_layer_group_begin(2 * k), "h2d_layer_group_begin")
            try:
                for kind, j, part, rows in parts:
                    sp, sbb, sn, dp, dbb, dn = pools[kind]
                    _check(swap(handles[j], h, sp, sbb, sn, dp, dbb, dn, part, rows, kind, layer, bits, heads,
                                dim, None), "h2d_swap")
            finally:
                _check(L.secure_infer_h2d_layer_group_end(), "h2d_layer_group_end")
        for st in streams:
            if st != parent:
                parent.wait_stream(st)
        self.layer += 1
        self._codec_auth(layer, bits)

    def _codec_auth(self, layer: int, bits: int) -> None:
        if self.codec_auth_wait and bits and self.wait_layer(layer) != 0:
            raise RuntimeError("Packed KV authentication failed")

    def prefetch_kv_transfer(self, payload, layer: int) -> bool:
        """Seal `layer`'s records on the host worker pool ahead of demand
        (the reference's CPU ciphertext prefetch, secure_infer.cpp:3264-3710),
        in the decomposition single_layer_kv_transfer will submit, so that
        transfer only copies them.  Returns False if the prefetch budget is
        spent (the transfer then seals on demand)."""
        host, mapping = payload
        mapping = mapping.to(device="cpu", dtype=torch.int64).contiguous()
        bits = self.shape.bits_for(layer)
        ok = True
        pools = []
        for kind in (0, 1):
            src = self._host_pool(host[kind])
            pools.append((ct.c_void_p(src.data_ptr()), src.stride(0) * src.element_size(), src.shape[0]))
        L, h = lib(), self.session._h
        prefetch = L.secure_infer_h2d_prefetch
        heads, dim = self.shape.heads, self.shape.head_dim
        # One stream and K / V pools of one geometry: a group's K and V swaps
        # are sealed together into one buffer, which the group's launch
        # copies in one DMA (same tickets as two prefetches: K, then V).
        paired = (len(self.streams) == 1 or not self.stripe) and pools[0][1:] == pools[1][1:]
        plan = self._plan(mapping)
        if paired and self.merge_groups and len(plan) > 1:
            # The whole layer in one buffer, in the device layout of its one
            # launch: one DMA per layer.
            base = mapping.data_ptr()
            starts = (ct.c_uint32 * len(plan))(*[(parts[0][2].value - base) // 16 for _, parts in plan])
            rows = (ct.c_uint32 * len(plan))(*[parts[0][3] for _, parts in plan])
            sp, sbb, sn = pools[0]
            ok = L.secure_infer_h2d_prefetch_layer(h, sp, pools[1][0], sbb, sn, ct.c_void_p(base), starts, rows,
                                                   len(plan), layer, bits, heads, dim) == 0
            self._prefetched.add(layer)
            return ok
        for _, parts in plan:
            if paired:
                (_, _, part, rows), _ = parts
                sp, sbb, sn = pools[0]
                ok &= L.secure_infer_h2d_prefetch_group(h, sp, pools[1][0], sbb, sn, part, rows, layer, bits, heads,
                                                        dim) == 0
                continue
            for kind, _, part, rows in parts:
                sp, sbb, sn = pools[kind]
                ok &= prefetch(h, sp, sbb, sn, part, rows, kind, layer, bits, heads, dim) == 0
        self._prefetched.add(layer)
        return ok

    def single_layer_wire_transfer(self, payload, destination, ticket_base: int = 0,
                                   iv_words_dev: torch.Tensor | None = None) -> None:
        wire, mapping = payload
        cache_k, cache_v = destination
        n = int(mapping.shape[0])
        bits = self.shape.bits_for(self.layer)
        nbytes = self.shape.record_bytes_for(self.layer)
        parent = torch.cuda.current_stream()
        launch = _torch_stream(self.stream)
        if launch != parent:
            launch.wait_stream(parent)
        # Everything the kernel reads or counts into is made on the launch
        # stream, so its initialisation is ordered before the kernel, and kept
        # until the layer is observed.
        with torch.cuda.stream(launch):
            slots = mapping[:, 1].to(device=cache_k.device, dtype=torch.int64)
            slots = torch.cat([slots, slots]).contiguous()
            fail = torch.zeros(1, dtype=torch.int32, device=cache_k.device)
            staging = None
            if bits:
                need = 2 * n * wire_tag_offset(nbytes)
                if self._staging is None or self._staging.numel() < need:
                    self._staging = torch.empty(need, dtype=torch.uint8, device=cache_k.device)
                staging = self._staging
        self.session.reload_layer(wire, nbytes, 2 * n, n, cache_k, cache_v, slots,
                                  ticket_base=ticket_base, iv_words_dev=iv_words_dev,
                                  codec_bits=bits, heads=self.shape.heads,
                                  head_dim=self.shape.head_dim, layer=self.layer,
                                  staging=staging, fail_count=fail, stream=launch)
        ev = torch.cuda.Event()
        ev.record(launch)
        if launch != parent:
            parent.wait_stream(launch)
        self._keep[self.layer] = (ev, fail, slots)
        _check(lib().secure_infer_recovery_track_layer(self.layer, ct.c_void_p(ev.cuda_event),
                                                       ct.c_void_p(fail.data_ptr())),
               "recovery_track_layer")
        self.layer += 1
        self._codec_auth(self.layer - 1, bits)

    def reload_layers(self, payloads, destinations, lookahead: int = 1) -> None:
        """Every layer of a stored prefix in order, through
        single_layer_kv_transfer, with the host sealing ahead: before layer
        l's swaps the records of layers l .. l + lookahead are queued for
        sealing (prefetch_kv_transfer, in layer order, so tickets keep the
        reference's (layer, group, kind, block) order), so layer l + 1 seals
        while layer l copies.  The reference keeps a window of predicted
        records sealing ahead of the swaps (schedule_linear_prefetches,
        secure_infer.cpp:1696-1740); here the window is `lookahead` whole
        layers, named by the caller instead of predicted from addresses.  A
        prefetch over the SECURE_INFER_PREFETCH_MB budget leaves that layer
        to seal on demand.  Layers are numbered from the driver's current
        layer."""
        n = len(payloads)
        if len(destinations) != n:
            raise ValueError("one destination per payload")
        base = self.layer
        maps = [m.to(device="cpu", dtype=torch.int64).contiguous() for _, m in payloads]
        for (host, _), m, dst in zip(payloads, maps, destinations):
            if m.shape[0]:
                self._check_mapping(host, m, dst)
        for l in range(n):
            for a in range(l, min(n, l + 1 + max(0, int(lookahead)))):
                if base + a not in self._prefetched and maps[a].shape[0]:
                    self.prefetch_kv_transfer((payloads[a][0], maps[a]), base + a)
            self.single_layer_kv_transfer((payloads[l][0], maps[l]), destinations[l])

    def wait_layer(self, layer: int) -> int:
        """0 if every record of `layer` authenticated, -1 otherwise."""
        rc = int(lib().secure_infer_recovery_wait_layer_authentication(layer))
        self._keep.pop(layer, None)
        return rc


class D2HTransfer:
    """Sealed writeback of device KV blocks into host pools: the D2H branch of
    _submit_transfer (npu_predict.py:874-916) with the same batch / group
    brackets (secure_infer_d2h_batch_begin ... batch_end).

    ``store(src_tensors, dst_tensors, src_to_dst)``: per layer, src = (k_cache,
    v_cache) device caches, dst = (cpu_k, cpu_v) host pools, and src_to_dst the
    [N, 2] int64 (gpu_slot, cpu_block) table.  Blocks are sealed on the device
    (gather, codec quantise, AES-GCM), copied to pinned memory on the library's
    D2H stream and authenticated + decrypted into the host pools by the worker
    pool.  Raises if any record fails host verification (it is zeroed), or if
    a mapping entry lies outside its pool (nothing is then queued for it).
    """

    def __init__(self, session: GcmSession, shape: LayerShape, group_blocks: int = 16,
                 stream=None):
        self.session = session
        self.shape = shape
        self.group_blocks = max(1, int(group_blocks))
        self.stream = stream

    def store(self, src_tensors, dst_tensors, src_to_dst, layers=None) -> None:
        mapping = src_to_dst.to(device="cpu", dtype=torch.int64).contiguous()
        n = int(mapping.shape[0])
        layers = list(range(len(src_tensors))) if layers is None else list(layers)
        stream = _stream(self.stream)
        L = lib()
        if L.secure_infer_d2h_batch_begin(n * len(src_tensors) * 2) <= 0:
            raise RuntimeError("d2h_batch_begin failed")
        try:
            for layer, src, dst in zip(layers, src_tensors, dst_tensors):
                bits = self.shape.bits_for(layer)
                for kind in (0, 1):
                    s_cache, d_pool = src[kind], dst[kind]
                    _dev(s_cache, "source cache")
                    if d_pool.is_cuda or not d_pool.is_contiguous():
                        raise ValueError("host pools must be contiguous CPU tensors")
                    for b0 in range(0, n, self.group_blocks):
                        part = mapping[b0:b0 + self.group_blocks].contiguous()
                        if L.secure_infer_d2h_group_begin(part.shape[0]) <= 0:
                            raise RuntimeError("d2h_group_begin failed")
                        try:
                            _check(L.secure_infer_d2h_swap(
                                stream, self.session._h, ct.c_void_p(s_cache.data_ptr()),
                                s_cache[0].numel() * s_cache.element_size(), s_cache.shape[0],
                                ct.c_void_p(d_pool.data_ptr()), d_pool[0].numel() * d_pool.element_size(),
                                d_pool.shape[0], ct.c_void_p(part.data_ptr()), part.shape[0], kind, layer,
                                bits, self.shape.heads, self.shape.head_dim),
                                "d2h_swap")
                        finally:
                            _check(L.secure_infer_d2h_group_end(), "d2h_group_end")
            _check(L.secure_infer_d2h_batch_device_barrier(), "d2h_batch_device_barrier")
        finally:
            rc = L.secure_infer_d2h_batch_end()
        if rc != 0:
            raise RuntimeError("d2h batch: host authentication failed")


def retire_transfer_prefetches() -> None:
    """Drops records sealed ahead of demand that no swap consumed
    (secure_infer.cpp:1137-1148; EncodedStore binds it, transport_codec.py:50)."""
    lib().secure_infer_retire_transfer_prefetches()


def transfer_prefetch_stats() -> dict:
    """Swaps served from ready prefetches / after waiting for one / sealed on
    demand (secure_infer_get_transfer_prefetch_stats, secure_infer.cpp:817-830)."""
    v = [ct.c_uint64() for _ in range(3)]
    lib().secure_infer_get_transfer_prefetch_stats(*[ct.byref(x) for x in v])
    return {"ready": v[0].value, "busy_fallback": v[1].value, "missing_fallback": v[2].value}


def set_job_id(job_id: int) -> None:
    """secure_infer_recovery_set_job_id (secure_infer.cpp:5311)."""
    lib().secure_infer_recovery_set_job_id(job_id)


def wait_job_authentication(job_id: int) -> int:
    """1 if every record of the job authenticated, 0 if not, -1 if it has none
    (secure_infer_recovery_wait_job_authentication, secure_infer.cpp:7336-7372)."""
    return int(lib().secure_infer_recovery_wait_job_authentication(job_id))


def flush_completed_h2d_profile() -> None:
    lib().secure_infer_flush_completed_h2d_profile()


def drain_h2d_profile_after_job() -> None:
    lib().secure_infer_drain_h2d_profile_after_job()


def pause_h2d_profile(paused: bool) -> None:
    """Stops (True) or resumes (False) recording ledger rows and their timing events."""
    lib().secure_infer_pause_h2d_profile(int(bool(paused)))


def inject_h2d_tamper(layer: int = -1, kind: int = -1, host_block: int = -1, shots: int = 1) -> None:
    """Test-only: flip the first ciphertext byte of the next `shots` H2D records
    sealed from (layer, kind, host_block) (-1 = any) after sealing
    (PIPE_GCM_TAMPER_H2D*, secure_infer.cpp:6139-6250)."""
    _check(lib().secure_infer_test_tamper_h2d(layer, kind, host_block, shots), "test_tamper_h2d")


def inject_d2h_tamper(shots: int = 1) -> None:
    """Test-only: flip the first ciphertext byte of the next `shots` D2H records
    before host authentication (PIPE_GCM_TAMPER_D2H, secure_infer.cpp:2451-2467)."""
    _check(lib().secure_infer_test_tamper_d2h(shots), "test_tamper_d2h")
