"""The reference's star-diagonal "RDP" code, signature-compatible with
benchmark/rdp/main.py.

``rdp_kernel`` stands in for the pybind module ``rdp_kernel_rdp_parallel``
(benchmark/rdp/kernel.cu:525-538).  The P/Q bytes are those of the reference.
Its two-row "recovery" is reproduced as the reference observably behaves: the
lower row is rebuilt from P and the other row keeps its input bytes (the
reference's ring walk is overwritten by its final rebuild-from-P kernels), so
it recovers nothing when two data rows are really lost.  True double-erasure
recovery is :func:`spec.rdp_decode` (textbook RDP).

K/V may be any 2-byte dtype (coded as raw bits; results come back in the input
dtype).
"""
from __future__ import annotations

import torch

from . import _lib


def _stream(t: torch.Tensor) -> int:
    return _lib.stream_handle(t.device)


class _RdpKernel:
    """The reference module ``rdp_kernel_rdp_parallel``."""

    @staticmethod
    def fused_backup_full_kv(K_TN, V_TN, shards, num_data_shards, shard_size, T, n, star_base):
        _lib.require_cuda(K_TN, V_TN, shards, what="fused_backup_full_kv tensor")
        _lib.call("kvec_gs_rdp_backup", K_TN.data_ptr(), V_TN.data_ptr(), shards.data_ptr(),
                  int(num_data_shards), int(shard_size), int(T), int(n), int(star_base),
                  _stream(shards))

    @staticmethod
    def fused_recovery_full_kv(shards, out_half_TN, num_data_shards, shard_size, T, n, star_base,
                               missing_a, missing_b):
        _lib.require_cuda(shards, out_half_TN, what="fused_recovery_full_kv tensor")
        _lib.call("kvec_gs_rdp_recover", shards.data_ptr(), out_half_TN.data_ptr(),
                  int(num_data_shards), int(shard_size), int(T), int(n), int(star_base),
                  int(missing_a), int(missing_b), _stream(shards))


rdp_kernel = _RdpKernel()


def determine_shard_size_words(total_words: int, num_data_shards: int):
    """benchmark/rdp/main.py:21-27."""
    if num_data_shards <= 0:
        raise ValueError("num_data_shards must be > 0")
    pad = (num_data_shards - (total_words % num_data_shards)) % num_data_shards
    padded_total = total_words + pad
    shard_size = padded_total // num_data_shards
    return shard_size, pad


def fused_backup_full_kv(keys_bhtd: torch.Tensor, values_bhtd: torch.Tensor,
                         num_data_shards: int, star_base: int = 0):
    """benchmark/rdp/main.py:44-92: token-major pack + P/Q in one call."""
    if not (keys_bhtd.is_cuda and values_bhtd.is_cuda):
        raise ValueError("keys/values must be CUDA tensors.")
    if keys_bhtd.dtype != values_bhtd.dtype or keys_bhtd.element_size() != 2:
        raise ValueError("keys/values must be fp16 (or another 2-byte dtype).")
    if keys_bhtd.shape != values_bhtd.shape:
        raise ValueError("K and V shapes must match [B,H,T,D].")
    if num_data_shards <= 0:
        raise ValueError("num_data_shards must be > 0")

    B, H, T, D = keys_bhtd.shape
    n = B * H * D
    total_words = 2 * T * n
    K_TN = keys_bhtd.permute(2, 0, 1, 3).contiguous().view(T, n)
    V_TN = values_bhtd.permute(2, 0, 1, 3).contiguous().view(T, n)

    shard_size, pad_words = determine_shard_size_words(total_words, num_data_shards)
    nd = int(num_data_shards)
    shards = torch.empty((nd + 2, shard_size), dtype=torch.uint16, device=K_TN.device)
    # the reference zero-fills everything; only the padding words are read
    # before being written
    shards.view(-1).view(torch.int16)[total_words:nd * shard_size].zero_()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    rdp_kernel.fused_backup_full_kv(K_TN, V_TN, shards, nd, int(shard_size), int(T), int(n),
                                    int(star_base))
    t1.record()
    torch.cuda.synchronize()
    backup_ms = t0.elapsed_time(t1)
    return {
        "shards_KV": shards,
        "shard_size": int(shard_size),
        "seq_len": int(T),
        "n": int(n),
        "num_data_shards": nd,
        "star_base": int(star_base),
        "shape_BHTD": (B, H, T, D),
        "backup_ms": backup_ms,
        "pad_words": int(pad_words),
        "dtype": keys_bhtd.dtype,
    }


def fused_recovery_full_kv(pkg: dict, missing_a: int, missing_b: int = -1):
    """benchmark/rdp/main.py:95-126: returns (keys_bhtd, values_bhtd, stats)."""
    shards = pkg["shards_KV"]
    shard_size = pkg["shard_size"]
    T = pkg["seq_len"]
    n = pkg["n"]
    nd = pkg["num_data_shards"]
    star_base = pkg["star_base"]
    B, H, _, D = pkg["shape_BHTD"]
    dtype = pkg.get("dtype", torch.float16)

    packed_TN = torch.empty(2 * T * n, dtype=dtype, device=shards.device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    rdp_kernel.fused_recovery_full_kv(shards, packed_TN, int(nd), int(shard_size), int(T), int(n),
                                      int(star_base), int(missing_a), int(missing_b))
    t1.record()
    torch.cuda.synchronize()
    recover_ms = t0.elapsed_time(t1)

    dK = packed_TN[:T * n].view(T, n)
    dV = packed_TN[T * n:].view(T, n)
    keys = dK.view(T, B, H, D).permute(1, 2, 0, 3).contiguous()
    values = dV.view(T, B, H, D).permute(1, 2, 0, 3).contiguous()
    return keys, values, {"recover_ms": recover_ms}
