"""spec family: textbook RDP over a prime p and Reed-Solomon over GF(2^8).

These codes have no counterpart in the reference (whose "RDP" is the
star-diagonal code in :mod:`.rdp`); they are the codes the KV-cache stripe
configurations are defined with.  Shards are separate HBM buffers: a stripe
set is k data tensors plus its parity tensors, each a contiguous byte tensor.

RDP stripe geometry: every shard holds (p-1)*row_bytes bytes, cut into
stripes of (p-1)*unit_bytes bytes (the last one shorter when unit_bytes does
not divide row_bytes).  Stripe s has p-1 rows of g_s = min(unit_bytes,
row_bytes - s*unit_bytes) bytes, row r at s*(p-1)*unit_bytes + r*g_s, and every
byte offset of its rows is one RDP instance; unit_bytes = 0 is a single stripe
of p-1 row planes.  Column p-1 of the code is the row parity P and Q holds the
diagonals 0..p-2 (Corbett et al., FAST 2004).  A byte stream is cut into k
consecutive shards of (p-1)*row_bytes bytes, zero-padded at the end.

``RDP_UNIT`` (64 KiB) is the stripe unit the KV chunk stripes use: with it each
wave's loads of a shard stay inside one 384 KiB stripe (p = 7), which MI355X's
HBM serves markedly faster than p-1 row planes far apart.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np
import torch

from . import _lib


RDP_UNIT = 65536


def rdp_unit_for(record_bytes: int = 16) -> int:
    """The stripe unit for streams of ``record_bytes`` records: the largest
    common multiple of 1024 and the record size up to RDP_UNIT (or that
    common multiple itself when it is larger)."""
    import math
    lcm = 1024 * int(record_bytes) // math.gcd(1024, int(record_bytes))
    return max(lcm, RDP_UNIT // lcm * lcm)


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def rdp_row_bytes(stream_bytes: int, k: int, p: int, granule: int = 16) -> int:
    """Smallest row plane (multiple of ``granule``) holding ``stream_bytes``."""
    r = _lib.lib().kvec_rdp_row_bytes(int(stream_bytes), int(k), int(p), int(granule))
    if r < 0:
        raise ValueError("bad RDP geometry arguments")
    return int(r)


def _row_bytes_of(shards: Sequence[torch.Tensor], p: int, row_bytes: int | None) -> int:
    nb = {_nbytes(t) for t in shards}
    if len(nb) != 1:
        raise ValueError("all shards of a stripe set must have the same size")
    size = nb.pop()
    if row_bytes is None:
        if size % (p - 1):
            raise ValueError(f"shard size {size} is not a multiple of p-1={p - 1}")
        row_bytes = size // (p - 1)
    elif size < (p - 1) * row_bytes:
        raise ValueError("shard smaller than (p-1)*row_bytes")
    return int(row_bytes)


def rdp_encode(data: Sequence[torch.Tensor], P: torch.Tensor, Q: torch.Tensor, p: int = 7,
               row_bytes: int | None = None, unit_bytes: int = 0) -> None:
    """Write the row parity P and diagonal parity Q of ``data`` (k <= p-1 shards)."""
    _lib.require_cuda(*data, P, Q, what="RDP shard")
    R = _row_bytes_of(list(data) + [P, Q], p, row_bytes)
    _lib.call("kvec_rdp_encode", _lib.ptr_array(data), len(data), P.data_ptr(), Q.data_ptr(),
              int(p), R, int(unit_bytes), _lib.stream_handle(P.device))


def rdp_decode(shards: Sequence[torch.Tensor], p: int, erased: Sequence[int],
               row_bytes: int | None = None, unit_bytes: int = 0) -> None:
    """Rebuild up to two erased shards in place; ``shards`` = data..., P, Q."""
    # distinct indices, in order, before the count check and the padding: a
    # repeated index must not push a third erasure out of the list
    er = list(dict.fromkeys(int(e) for e in erased if e is not None and int(e) >= 0))
    if len(er) > 2:
        raise ValueError("RDP recovers at most two erased shards")
    er = (er + [-1, -1])[:2]
    _lib.require_cuda(*shards, what="RDP shard")
    R = _row_bytes_of(shards, p, row_bytes)
    k = len(shards) - 2
    _lib.call("kvec_rdp_decode", _lib.ptr_array(shards), k, int(p), R, int(unit_bytes), er[0],
              er[1], _lib.stream_handle(shards[0].device))


def alloc_rdp_stripe(k: int, p: int, row_bytes: int, device, parity: bool = True):
    """k data + (P, Q) byte tensors for one stripe set, each its own allocation."""
    n = (p - 1) * row_bytes
    data = [torch.empty(n, dtype=torch.uint8, device=device) for _ in range(k)]
    if not parity:
        return data
    return data, torch.empty(n, dtype=torch.uint8, device=device), \
        torch.empty(n, dtype=torch.uint8, device=device)


def split_stream(stream: torch.Tensor, k: int, shard_bytes: int):
    """Copy a byte stream into k zero-padded shard tensors (device copies)."""
    flat = stream.reshape(-1).view(torch.uint8)
    out = []
    for i in range(k):
        t = torch.zeros(shard_bytes, dtype=torch.uint8, device=flat.device)
        lo = i * shard_bytes
        hi = min(flat.numel(), lo + shard_bytes)
        if hi > lo:
            t[: hi - lo].copy_(flat[lo:hi])
        out.append(t)
    return out


# ------------------------------------------------------------------ RS GF(2^8)
def rs8_cauchy(k: int, m: int) -> np.ndarray:
    """The m x k Cauchy parity block C[i][j] = 1 / ((k+i) ^ j) over GF(2^8)/0x11D."""
    C = np.zeros((m, k), np.uint8)
    _lib.call("kvec_rs8_cauchy", int(k), int(m), C.ctypes.data)
    return C


def rs8_encode(data: Sequence[torch.Tensor], parity: Sequence[torch.Tensor]) -> None:
    """parity[i] = XOR_j C[i][j] * data[j] (separate equally sized byte shards)."""
    _lib.require_cuda(*data, *parity, what="RS shard")
    nb = {_nbytes(t) for t in list(data) + list(parity)}
    if len(nb) != 1:
        raise ValueError("all shards must have the same size")
    _lib.call("kvec_rs8_encode", _lib.ptr_array(data), len(data), _lib.ptr_array(parity),
              len(parity), nb.pop(), _lib.stream_handle(data[0].device))


def rs8_decode(shards: Sequence[torch.Tensor], k: int, erased: Sequence[int]) -> None:
    """Rebuild the erased shards (data..., parity...) in place; at most m = len(shards)-k."""
    _lib.require_cuda(*shards, what="RS shard")
    nb = {_nbytes(t) for t in shards}
    if len(nb) != 1:
        raise ValueError("all shards must have the same size")
    er = np.ascontiguousarray(sorted({int(e) for e in erased}), dtype=np.int32)
    _lib.call("kvec_rs8_decode", _lib.ptr_array(shards), int(k), len(shards) - int(k), nb.pop(),
              er.ctypes.data_as(ctypes.c_void_p) if er.size else None, int(er.size),
              _lib.stream_handle(shards[0].device))
