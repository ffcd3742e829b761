"""The serving plugin's inline extension ``rdp_kv_ops``
(bench_ghostserve_rdp.py:92-207), same names and keyword arguments.

pack_row_from_block  row r of the stripe = K words || V words of one rank
compute_rdp_parity   P and Q of the first nd rows (the gs star-diagonal code)

Both run on torch's current stream, as the reference's do.  The reference
converts the KV to fp16 before packing (bench_ghostserve_rdp.py:345-346), which
is lossy for a bf16 cache; here any 2-byte dtype is packed as raw bits, so the
parity protects the bytes actually stored.
"""
from __future__ import annotations

import torch

from . import _lib


def pack_row_from_block(k_blk: torch.Tensor, v_blk: torch.Tensor, shards: torch.Tensor, row: int):
    """bench_ghostserve_rdp.py:152-175."""
    if not (k_blk.is_cuda and v_blk.is_cuda and shards.is_cuda):
        raise RuntimeError("CUDA tensors required.")
    if k_blk.element_size() != 2 or v_blk.element_size() != 2:
        raise RuntimeError("KV must be fp16.")
    if shards.dtype != torch.uint16:
        raise RuntimeError("shards must be uint16.")
    if not (k_blk.is_contiguous() and v_blk.is_contiguous()):
        raise RuntimeError("KV must be contiguous.")
    if shards.dim() != 2:
        raise RuntimeError("shards must be [rows, S].")
    # the reference leaves this unchecked (an out-of-range row writes past
    # the tensor); here it is an error like the other argument checks
    if not 0 <= int(row) < shards.size(0):
        raise RuntimeError("row must be in [0, shards.size(0)).")
    words = k_blk.numel()
    S = shards.size(1)
    if S < 2 * words:
        raise RuntimeError("shard_size must be >= 2 * words.")
    if not shards.is_contiguous():
        raise RuntimeError("shards must be contiguous.")
    _lib.call("kvec_gs_pack_row", k_blk.data_ptr(), v_blk.data_ptr(), shards.data_ptr(),
              int(words), int(row), int(S), _lib.stream_handle(shards.device))


def compute_rdp_parity(rows: torch.Tensor, nd: int, S: int, star_base: int):
    """bench_ghostserve_rdp.py:177-199."""
    if not rows.is_cuda:
        raise RuntimeError("rows must be CUDA")
    if rows.dtype != torch.uint16:
        raise RuntimeError("rows must be uint16")
    if not (rows.dim() == 2 and rows.size(0) >= nd + 2 and rows.size(1) >= S):
        raise RuntimeError("bad shapes")
    if not rows.is_contiguous():
        raise RuntimeError("rows must be contiguous")
    _lib.call("kvec_gs_rdp_parity", rows.data_ptr(), int(nd), int(S), int(star_base),
              _lib.stream_handle(rows.device))
