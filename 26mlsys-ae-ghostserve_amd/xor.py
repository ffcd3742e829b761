"""XOR single parity, signature-compatible with benchmark/xor/main.py.

``xor_kernel`` stands in for the reference's JIT-built pybind module
(benchmark/xor/kernel.cu:225-244): same function names, positional argument
order and in-place semantics, backed by libkvec's HIP kernels.

Differences from the reference, none of which changes an output byte:
  * K/V may be any 2-byte dtype (fp16, bf16, ...) or a 1-byte one (fp8); the
    bytes are coded as raw bits and come back in the input dtype.
  * forward_encode_kv writes K||V into the shard tensor's data rows and P in
    one pass over K and V (kvec_xor_encode_kv), instead of the reference's
    pack, staging copy and encode (the shards are identical).
  * Every call is stream-ordered on torch's current stream; unpack does not
    block the host.
"""
from __future__ import annotations

import torch

from . import _lib


def _stream(t: torch.Tensor) -> int:
    return _lib.stream_handle(t.device)


class _XorKernel:
    """The reference module ``xor_kernel`` (benchmark/xor/kernel.cu:225-244)."""

    @staticmethod
    def encode_xor(data_padded, shards, data_shards, shard_size):
        _lib.require_cuda(data_padded, shards, what="encode_xor tensor")
        _lib.call("kvec_xor_encode", data_padded.data_ptr(), shards.data_ptr(), int(data_shards),
                  int(shard_size), _stream(shards))

    @staticmethod
    def reconstruct_xor(encoded_data, recovered_data, recovered_missing_shards, shard_size,
                        data_shards, missing_indices):
        _lib.require_cuda(encoded_data, recovered_data, recovered_missing_shards,
                          what="reconstruct_xor tensor")
        if missing_indices.dtype != torch.int32 or not missing_indices.is_cuda:
            raise TypeError("missing_indices must be an int32 GPU tensor")
        _lib.call("kvec_xor_reconstruct", encoded_data.data_ptr(), recovered_data.data_ptr(),
                  recovered_missing_shards.data_ptr(), int(shard_size), int(data_shards),
                  missing_indices.data_ptr(), int(missing_indices.numel()), _stream(encoded_data))

    @staticmethod
    def pack_kv(key_input, value_input, kv_bytes, n, seq_len):
        _lib.require_cuda(key_input, value_input, kv_bytes, what="pack_kv tensor")
        _lib.call("kvec_pack_kv", key_input.data_ptr(), value_input.data_ptr(),
                  kv_bytes.data_ptr(), int(n), int(seq_len), _stream(kv_bytes))

    @staticmethod
    def unpack_kv(kv_bytes, dequant_KV, n, seq_len):
        _lib.require_cuda(kv_bytes, dequant_KV, what="unpack_kv tensor")
        _lib.call("kvec_unpack_kv", kv_bytes.data_ptr(), dequant_KV.data_ptr(), int(n),
                  int(seq_len), _stream(kv_bytes))


xor_kernel = _XorKernel()


def determine_shard_size(num_bytes: int, num_data_shards: int):
    """benchmark/xor/main.py:39-43."""
    pad = (num_data_shards - (num_bytes % num_data_shards)) % num_data_shards
    padded_total = num_bytes + pad
    shard_size = padded_total // num_data_shards
    return shard_size, pad


def _check_kv(keys, values):
    if not (keys.is_cuda and values.is_cuda):
        raise AssertionError("Run on CUDA for GPU timing.")
    if keys.dtype != values.dtype or keys.element_size() not in (1, 2):
        raise AssertionError("keys/values must share a 1- or 2-byte dtype")
    if keys.shape != values.shape:
        raise AssertionError("keys and values must have the same shape")


def forward_encode_kv(keys, values, num_data_shards, num_parity_shards):
    """benchmark/xor/main.py:47-133: K||V bytes -> (num_data_shards + 1) shards."""
    if num_parity_shards != 1:
        raise ValueError("XOR parity supports exactly 1 parity shard.")
    _check_kv(keys, values)
    keys = keys.contiguous()
    values = values.contiguous()
    device = keys.device
    B, H, T, D = keys.shape
    n = B * H * D
    es = keys.element_size()
    total_bytes = 2 * es * T * n

    shard_size, pad = determine_shard_size(total_bytes, num_data_shards)
    data_bytes = num_data_shards * shard_size
    shards_KV = torch.empty((num_data_shards + num_parity_shards, shard_size), dtype=torch.uint8,
                            device=device)
    # the pack (K bytes then V bytes, zero padding) and the encode in one call:
    # one pass over K and V when the layouts allow it
    _lib.call("kvec_xor_encode_kv", keys.data_ptr(), values.data_ptr(), total_bytes // 2,
              shards_KV.data_ptr(), int(num_data_shards), int(shard_size), _stream(shards_KV))

    pack_io = 2 * total_bytes
    encode_io = data_bytes + data_bytes + shard_size
    return {
        "shards_KV": shards_KV,
        "seq_len": T,
        "n": n,
        "shard_size": shard_size,
        "device": device,
        "shape_BHTD": (B, H, T, D),
        "pack_io": pack_io,
        "encode_io": encode_io,
        "num_data_shards": num_data_shards,
        "num_parity_shards": num_parity_shards,
        "pad": pad,
        "total_bytes": total_bytes,
        "orig_keys": keys,
        "orig_vals": values,
    }


def backwards_decode_kv(pkg, missing_shards):
    """benchmark/xor/main.py:137-212: rebuild the missing shard in place (one
    missing shard at most), unpack K, V.  Returns (keys, values, stats)."""
    shards_KV = pkg["shards_KV"]
    T = pkg["seq_len"]
    n = pkg["n"]
    shard_size = pkg["shard_size"]
    device = pkg["device"]
    B, H, _, D = pkg["shape_BHTD"]
    num_data_shards = pkg["num_data_shards"]
    num_parity_shards = pkg["num_parity_shards"]
    total_shards = num_data_shards + num_parity_shards
    dtype = pkg["orig_keys"].dtype if "orig_keys" in pkg else torch.float16

    if num_parity_shards != 1:
        raise ValueError("XOR parity supports exactly 1 parity shard.")
    if len(missing_shards) > 1:
        raise ValueError("XOR parity can recover only a single missing shard.")
    for idx in missing_shards:
        if idx < 0 or idx >= total_shards:
            raise ValueError(f"Missing shard {idx} out of range 0..{total_shards-1}")

    # The missing shard is rebuilt in place and the data rows copied out in one
    # call (one pass over the rows when a data row is lost).  The reference
    # zeroes the missing shard first; that row is rewritten in full and never
    # read, so the zeroing is left out.
    es = torch.empty((), dtype=dtype).element_size()
    de_bytes_needed = 2 * es * T * n
    if num_data_shards * shard_size < de_bytes_needed:
        raise RuntimeError("Not enough bytes in reconstructed data region.")
    dequant_KV = torch.empty(2 * T * n, dtype=dtype, device=device)
    missing = int(missing_shards[0]) if len(missing_shards) == 1 else -1
    _lib.call("kvec_xor_recover_kv", shards_KV.data_ptr(), dequant_KV.data_ptr(),
              int(num_data_shards), int(shard_size), de_bytes_needed, missing, _stream(shards_KV))
    r_ms = 0.0

    keys_out = dequant_KV[:T * n].view(B, H, T, D)
    values_out = dequant_KV[T * n: 2 * T * n].view(B, H, T, D)
    return keys_out, values_out, {
        "reconstruct_ms": r_ms,
        "reconstruct_io": ((num_data_shards + 1) * shard_size + 2 * shard_size) if r_ms > 0 else 0,
        "unpack_io": 2 * de_bytes_needed,
    }
