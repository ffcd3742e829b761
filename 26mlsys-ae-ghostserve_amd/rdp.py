"""The reference's star-diagonal "RDP" code, signature-compatible with
benchmark/rdp/main.py.

``rdp_kernel`` stands in for the pybind module ``rdp_kernel_rdp_parallel``
(benchmark/rdp/kernel.cu:525-538).  The P/Q bytes are those of the reference.
Its two-row "recovery" is reproduced as the reference observably behaves: the
lower row is rebuilt from P and the other row keeps its input bytes (the
reference's ring walk is overwritten by its final rebuild-from-P kernels), so
it recovers nothing when two data rows are really lost.

``scheme="spec"`` keeps the same functions, arguments and returned dicts but
codes the shard tensor with textbook RDP (Corbett et al., FAST 2004) over the
smallest prime p > num_data_shards (p = 7 for six data shards): the data rows
are shards, row nd is P and row nd+1 is Q, and fused_recovery_full_kv then
rebuilds any two lost rows (data, P or Q) byte-exact.  Its shard size is the
reference's rounded up so that every shard row splits into p-1 RDP rows of a
whole number of 16-byte cells.

K/V may be any 2-byte dtype (coded as raw bits; results come back in the input
dtype).
"""
from __future__ import annotations

import torch

from . import _lib, spec


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


SCHEMES = ("ghostserve", "spec")


def spec_prime(num_data_shards: int) -> int:
    """Smallest odd prime p with p - 1 >= num_data_shards."""
    p = max(3, int(num_data_shards) + 1)
    while any(p % q == 0 for q in range(2, int(p ** 0.5) + 1)):
        p += 1
    return p


def spec_shard_size_words(total_words: int, num_data_shards: int, p: int):
    """The reference's shard size rounded up so that a shard row splits into
    p-1 RDP rows of a multiple of 16 bytes (8 words) each.  Returns
    (shard_size, pad_words)."""
    S, _ = determine_shard_size_words(total_words, num_data_shards)
    q = 8 * (p - 1)
    S = -(-S // q) * q
    return S, num_data_shards * S - total_words


def _rows_u8(shards: torch.Tensor):
    """The rows of a [(rows), S] uint16 shard tensor as byte tensors."""
    b = shards.view(torch.uint8).view(shards.shape[0], -1)
    return [b[i] for i in range(shards.shape[0])]


def _check_scheme(scheme: str):
    if scheme not in SCHEMES:
        raise ValueError(f"scheme must be one of {SCHEMES}, not {scheme!r}")


def fused_backup_full_kv(keys_bhtd: torch.Tensor, values_bhtd: torch.Tensor,
                         num_data_shards: int, star_base: int = 0, scheme: str = "ghostserve"):
    """benchmark/rdp/main.py:44-92: token-major pack + P/Q in one call.
    scheme="spec": textbook RDP P/Q instead of the star-diagonal code."""
    _check_scheme(scheme)
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

    nd = int(num_data_shards)
    p = spec_prime(nd) if scheme == "spec" else 0
    if scheme == "spec":
        shard_size, pad_words = spec_shard_size_words(total_words, nd, p)
    else:
        shard_size, pad_words = determine_shard_size_words(total_words, nd)
    shards = torch.empty((nd + 2, shard_size), dtype=torch.uint16, device=K_TN.device)
    # the reference zero-fills everything; only the padding words are read
    # before being written
    shards.view(-1).view(torch.int16)[total_words:nd * shard_size].zero_()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    if scheme == "spec":
        # K_TN || V_TN into the data rows, then textbook RDP over the rows
        _lib.call("kvec_rs16_pack", K_TN.data_ptr(), V_TN.data_ptr(), shards.data_ptr(),
                  T * n, T * n, _stream(shards))
        rows = _rows_u8(shards)
        spec.rdp_encode(rows[:nd], rows[nd], rows[nd + 1], p, unit_bytes=spec.RDP_UNIT)
    else:
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
        "scheme": scheme,
        "p": p,
    }


def fused_recovery_full_kv(pkg: dict, missing_a: int, missing_b: int = -1):
    """benchmark/rdp/main.py:95-126: returns (keys_bhtd, values_bhtd, stats).
    For a pkg of scheme "spec" the lost rows (data 0..nd-1, P = nd, Q = nd+1;
    other indices are ignored) are rebuilt by the textbook RDP decode first."""
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
    if pkg.get("scheme", "ghostserve") == "spec":
        lost = [int(e) for e in (missing_a, missing_b) if 0 <= int(e) < nd + 2]
        spec.rdp_decode(_rows_u8(shards), int(pkg["p"]), lost, unit_bytes=spec.RDP_UNIT)
        _lib.call("kvec_rs16_split", shards.data_ptr(), packed_TN.data_ptr(),
                  packed_TN[T * n:].data_ptr(), T * n, T * n, _stream(shards))
    else:
        rdp_kernel.fused_recovery_full_kv(shards, packed_TN, int(nd), int(shard_size), int(T),
                                          int(n), int(star_base), int(missing_a), int(missing_b))
    t1.record()
    torch.cuda.synchronize()
    recover_ms = t0.elapsed_time(t1)

    dK = packed_TN[:T * n].view(T, n)
    dV = packed_TN[T * n:].view(T, n)
    keys = dK.view(T, B, H, D).permute(1, 2, 0, 3).contiguous()
    values = dV.view(T, B, H, D).permute(1, 2, 0, 3).contiguous()
    return keys, values, {"recover_ms": recover_ms}
