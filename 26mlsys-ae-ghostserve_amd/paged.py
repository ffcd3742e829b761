"""Paged KV pool <-> coding stream (the serving plugin's delta gather,
bench_ghostserve_rdp.py:440-458, over a paged pool), and the fused
gather + RDP encode that codes a prefill chunk straight out of the pool.

Pool tensor: [layers, pool_pages, page_tokens, 2 (K,V), kv_heads, head_dim] of
any dtype (coded as raw bytes).  Page table: int32 [batch, pages_per_seq] of
pool page indices.  Stream of a chunk of ``tokens`` positions starting at
``tok_off``: the chunk's token records in order,
[layers, batch, tokens, 2 (K,V), kv_heads, head_dim], so each pool page
contributes contiguous runs of records.
"""
from __future__ import annotations

from typing import Sequence

import torch

from . import _lib


class PagedKV:
    """A chunk of a paged KV pool: the descriptor the kernels take."""

    def __init__(self, pool: torch.Tensor, page_table: torch.Tensor, tok_off: int = 0,
                 tokens: int | None = None):
        if pool.dim() != 6 or pool.shape[3] != 2:
            raise ValueError("pool must be [layers, pool_pages, page_tokens, 2, heads, dim]")
        if page_table.dtype != torch.int32 or page_table.dim() != 2:
            raise ValueError("page_table must be int32 [batch, pages_per_seq]")
        _lib.require_cuda(pool, page_table, what="paged KV tensor")
        L, npages, pt, _, H, D = pool.shape
        B, pps = page_table.shape
        if tokens is None:
            tokens = pps * pt - tok_off
        self.pool, self.page_table = pool, page_table
        self.layers, self.pool_pages, self.page_tokens = L, npages, pt
        self.batch, self.pages_per_seq = B, pps
        self.tok_off, self.tokens = int(tok_off), int(tokens)
        self.token_bytes = H * D * pool.element_size()
        self.heads, self.dim = H, D
        self._c = _lib.PagedKV(pool.data_ptr(), npages, L, self.token_bytes, pt,
                               page_table.data_ptr(), B, pps, self.tok_off, self.tokens)

    @property
    def c(self):
        return self._c

    def stream_bytes(self) -> int:
        return int(_lib.lib().kvec_kv_stream_bytes(self._c))

    def stream_shape(self):
        return (self.layers, self.batch, self.tokens, 2, self.heads, self.dim)

    def gather(self, out: torch.Tensor | None = None) -> torch.Tensor:
        """The chunk's stream, as a uint8 tensor of stream_bytes() bytes."""
        n = self.stream_bytes()
        if out is None:
            out = torch.empty(n, dtype=torch.uint8, device=self.pool.device)
        elif out.numel() * out.element_size() < n:
            raise ValueError("output smaller than the stream")
        _lib.require_cuda(out, what="gather output")
        _lib.call("kvec_kv_gather", self._c, out.data_ptr(), _lib.stream_handle(out.device))
        return out

    def gather_split(self, out_k: torch.Tensor, out_v: torch.Tensor) -> None:
        """The chunk's K halves into out_k and V halves into out_v, each in
        record order (stream_bytes() / 2 bytes each, 16-byte aligned)."""
        half = self.stream_bytes() // 2
        for t in (out_k, out_v):
            if t.numel() * t.element_size() < half:
                raise ValueError("output smaller than half the stream")
        _lib.require_cuda(out_k, out_v, what="gather output")
        _lib.call("kvec_kv_gather_split", self._c, out_k.data_ptr(), out_v.data_ptr(),
                  _lib.stream_handle(out_k.device))

    def scatter(self, stream: torch.Tensor) -> None:
        """Write a stream (e.g. a recovered one) back into the pool pages."""
        if stream.numel() * stream.element_size() < self.stream_bytes():
            raise ValueError("stream smaller than the chunk")
        _lib.require_cuda(stream, what="scatter input")
        _lib.call("kvec_kv_scatter", self._c, self.pool.data_ptr(), stream.data_ptr(),
                  _lib.stream_handle(stream.device))


def rdp_row_bytes_for(kv: PagedKV, k: int, p: int) -> int:
    """RDP row size R (each shard is (p-1)*R bytes) for kv's stream: a
    multiple of one token record (K and V)."""
    from .spec import rdp_row_bytes
    return rdp_row_bytes(kv.stream_bytes(), k, p, 2 * kv.token_bytes)


def rdp_encode_paged(kv: PagedKV, data: Sequence[torch.Tensor], P: torch.Tensor, Q: torch.Tensor,
                     p: int = 7, row_bytes: int | None = None, unit_bytes: int = 0) -> int:
    """Gather kv's chunk into the k data shards and write their RDP parity, in
    one pass over the pool (stripe geometry of ``spec``; unit_bytes a multiple
    of 1024 and of the token record).  Returns the row size used."""
    if row_bytes is None:
        row_bytes = rdp_row_bytes_for(kv, len(data), p)
    _lib.require_cuda(*data, P, Q, what="RDP shard")
    for t in list(data) + [P, Q]:
        if t.numel() * t.element_size() < (p - 1) * row_bytes:
            raise ValueError("shard smaller than (p-1)*row_bytes")
    _lib.call("kvec_rdp_encode_paged", kv.c, _lib.ptr_array(data), len(data), P.data_ptr(),
              Q.data_ptr(), int(p), int(row_bytes), int(unit_bytes), _lib.stream_handle(P.device))
    return int(row_bytes)


def rdp_decode_paged(kv: PagedKV, P: torch.Tensor, Q: torch.Tensor, erased: Sequence[int], k: int,
                     p: int = 7, row_bytes: int | None = None, unit_bytes: int = 0,
                     data: Sequence[torch.Tensor] | None = None) -> None:
    """Rebuild up to two lost shards of kv's stripe set (data 0..k-1, P = k,
    Q = k+1): lost data straight into the pool pages (and into ``data`` when
    the data shard buffers are given), lost parity into P / Q.  Surviving data
    is read from ``data`` when given, else from the pool."""
    er = list(dict.fromkeys(int(e) for e in erased if e is not None and int(e) >= 0))
    if len(er) > 2:
        raise ValueError("RDP recovers at most two erased shards")
    er = (er + [-1, -1])[:2]
    if row_bytes is None:
        row_bytes = rdp_row_bytes_for(kv, k, p)
    shards = [P, Q] + (list(data) if data is not None else [])
    _lib.require_cuda(*shards, what="RDP shard")
    for t in shards:
        if t.numel() * t.element_size() < (p - 1) * row_bytes:
            raise ValueError("shard smaller than (p-1)*row_bytes")
    if data is not None and len(data) != k:
        raise ValueError(f"expected {k} data shards")
    _lib.call("kvec_rdp_decode_paged", kv.c, kv.pool.data_ptr(),
              _lib.ptr_array(data) if data is not None else None, int(k), P.data_ptr(),
              Q.data_ptr(), int(p), int(row_bytes), int(unit_bytes), er[0], er[1],
              _lib.stream_handle(P.device))
