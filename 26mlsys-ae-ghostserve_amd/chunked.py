"""Chunked coding of a paged KV cache as prefill chunks arrive.

The reference codes each prefill step's KV on the serving path after an fp16
conversion (bench_ghostserve_rdp.py:334-392, :445-458).  Here the cache bytes
themselves are coded (any dtype, e.g. fp8 e4m3 with a per-layer scale), one
chunk at a time, straight out of the paged pool:

  * textbook RDP(p) row + diagonal parity and systematic RS(k, m) over
    GF(2^8)/0x11D (Cauchy) share the same k data shards;
  * chunk c owns the region of (p-1)*width bytes at c*(p-1)*width of every
    shard of a whole-sequence stripe set; its stream (its token records in
    order, see :mod:`.paged`), zero padded, is cut into k pieces of
    (p-1)*width bytes, piece j being data shard j's region;
  * a region is a spec RDP stripe set with rows of ``width`` bytes cut into
    stripes of ``unit_bytes`` rows (see :mod:`.spec`), so each chunk is coded
    once, into its own region, with no parity read back, and each region's
    parity is one contiguous range of every parity shard;
  * the data shards are optional: the pool is the primary copy of the data, and
    decode reads the surviving data cells from the pool and writes rebuilt ones
    back into the pool pages.

Shard indices of decode: data 0..k-1, P = k, Q = k+1, RS parity i = k+2+i.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np
import torch

from . import _lib
from .paged import PagedKV
from .spec import rdp_unit_for


def chunk_width(chunk_stream_bytes: int, k: int, p: int, record_bytes: int) -> int:
    """Smallest cell width (a multiple of one token record) holding a chunk."""
    w = _lib.lib().kvec_chunk_width(int(chunk_stream_bytes), int(k), int(p), int(record_bytes))
    if w < 0:
        raise ValueError("bad chunk geometry arguments")
    return int(w)


class ChunkedStripes:
    """Whole-sequence stripe set for ``n_chunks`` equally sized chunks.

    Holds P, Q, the m RS parity shards and (with ``keep_data``) the k data
    shards, each (p-1)*row_bytes bytes with row_bytes = n_chunks * width, so
    chunk c's region is bytes [region(c), region(c) + region_bytes) of each.
    ``unit_bytes`` is the stripe unit of a region (by default the largest
    multiple of 1024 and of the record size up to 64 KiB).  ``scales`` (e.g.
    the per-layer fp32 scales of an fp8 cache) are carried alongside as a
    copy; they are per-layer constants, not coded.
    """

    def __init__(self, chunk_stream_bytes: int, record_bytes: int, n_chunks: int, device,
                 k: int = 5, p: int = 7, m: int = 3, keep_data: bool = False,
                 scales: torch.Tensor | None = None, unit_bytes: int | None = None):
        if n_chunks < 1:
            raise ValueError("n_chunks must be >= 1")
        self.k, self.p, self.m, self.n_chunks = int(k), int(p), int(m), int(n_chunks)
        self.width = chunk_width(chunk_stream_bytes, k, p, record_bytes)
        self.unit_bytes = rdp_unit_for(record_bytes) if unit_bytes is None else int(unit_bytes)
        self.region_bytes = (self.p - 1) * self.width
        self.row_bytes = self.n_chunks * self.width
        n = (p - 1) * self.row_bytes
        mk = lambda: torch.empty(n, dtype=torch.uint8, device=device)  # noqa: E731
        self.data = [mk() for _ in range(k)] if keep_data else None
        self.P, self.Q = mk(), mk()
        self.rs = [mk() for _ in range(m)]
        self.scales = None if scales is None else scales.detach().clone()

    def shards(self):
        """data (if kept), P, Q, RS parity -- in decode index order."""
        return (list(self.data) if self.data else []) + [self.P, self.Q] + list(self.rs)

    def region(self, c: int) -> int:
        """Byte offset of chunk ``c``'s region in every shard."""
        return int(c) * self.region_bytes

    def _struct(self, c: int):
        if not 0 <= c < self.n_chunks:
            raise ValueError(f"chunk {c} not in [0, {self.n_chunks})")
        keep = []
        data = None
        if self.data is not None:
            data = _lib.ptr_array(self.data)
            keep.append(data)
        rs = _lib.ptr_array(self.rs) if self.rs else None
        keep.append(rs)
        st = _lib.ChunkStripe(
            ctypes.cast(data, ctypes.POINTER(ctypes.c_void_p)) if data is not None else None,
            self.k, self.P.data_ptr(), self.Q.data_ptr(), self.p,
            ctypes.cast(rs, ctypes.POINTER(ctypes.c_void_p)) if rs is not None else None,
            self.m, self.row_bytes, self.region(c), self.width, self.unit_bytes)
        return st, keep

    def encode(self, kv: PagedKV, c: int) -> None:
        """Code chunk ``c`` (the descriptor ``kv``) into its region."""
        st, keep = self._struct(c)
        _lib.call("kvec_chunk_encode_paged", kv.c, ctypes.byref(st),
                  _lib.stream_handle(self.P.device))
        del keep

    def decode(self, kv: PagedKV, c: int, erased: Sequence[int]) -> None:
        """Rebuild chunk ``c``'s region of the erased shards; lost data goes
        back into the pool pages of ``kv`` (and into the data shards if kept)."""
        st, keep = self._struct(c)
        er = np.ascontiguousarray(sorted({int(e) for e in erased}), dtype=np.int32)
        _lib.call("kvec_chunk_decode_paged", kv.c, kv.pool.data_ptr(), ctypes.byref(st),
                  er.ctypes.data_as(ctypes.c_void_p) if er.size else None, int(er.size),
                  _lib.stream_handle(self.P.device))
        del keep


def chunk_kv(pool: torch.Tensor, page_table: torch.Tensor, c: int, chunk_tokens: int) -> PagedKV:
    """Descriptor of prefill chunk ``c`` (positions c*chunk_tokens ..) of every sequence."""
    return PagedKV(pool, page_table, c * chunk_tokens, chunk_tokens)
