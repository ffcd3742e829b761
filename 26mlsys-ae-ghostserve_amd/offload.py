"""Parity offload to host memory, overlapped with coding.

The reference's parity driver copies P and Q of each prefill step to pageable
host memory with ``.to("cpu", non_blocking=True)`` followed by a device-wide
synchronize, then times a host-to-device "probe" copy back
(bench_ghostserve_rdp.py:362-374): the copy is synchronous and blocks the
serving loop.

Here the copies run on a side stream (default priority) into pinned host
buffers, ordered after the encode through an event, so the next chunk's
encode runs while the previous chunk's parity crosses PCIe.  A chunk's parity
lives in its own columns of the whole-sequence stripes (``chunked``), so
offloading chunk c never races with encoding chunk c+1; the host copy of each
shard keeps the same [p-1, row_bytes] layout, so a restore is the same copies
in the other direction.
"""
from __future__ import annotations

from typing import Sequence

import torch


class ParityOffload:
    """Pinned host mirrors of parity shards plus a copy stream.

    ``shards`` are the device parity tensors (each ``rows * row_bytes`` bytes,
    row-major [rows, row_bytes]); the host mirrors have the same shape.
    """

    def __init__(self, shards: Sequence[torch.Tensor], rows: int, row_bytes: int):
        if not shards:
            raise ValueError("no parity shards")
        for t in shards:
            if t.numel() * t.element_size() != rows * row_bytes or not t.is_contiguous():
                raise ValueError("each parity shard must be a contiguous rows*row_bytes buffer")
        self.device = shards[0].device
        self.rows, self.row_bytes = int(rows), int(row_bytes)
        self.dev = [t.view(torch.uint8).view(rows, row_bytes) for t in shards]
        self.host = [torch.empty((rows, row_bytes), dtype=torch.uint8, pin_memory=True)
                     for _ in shards]
        self.stream = torch.cuda.Stream(device=self.device)

    def _copy(self, col_off: int, width: int, to_host: bool, after: torch.cuda.Event | None):
        if col_off < 0 or width <= 0 or col_off + width > self.row_bytes:
            raise ValueError("column range outside the row planes")
        done = torch.cuda.Event()
        with torch.cuda.stream(self.stream):
            if after is not None:
                self.stream.wait_event(after)
            for d, h in zip(self.dev, self.host):
                for r in range(self.rows):
                    src, dst = (d, h) if to_host else (h, d)
                    dst[r, col_off:col_off + width].copy_(src[r, col_off:col_off + width],
                                                          non_blocking=True)
            done.record(self.stream)
        return done

    def to_host(self, col_off: int, width: int) -> torch.cuda.Event:
        """Copy columns [col_off, col_off+width) of every parity row plane to
        the host mirrors, after the work already queued on the current stream.
        Returns the event that marks the copies done."""
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(self.device))
        return self._copy(col_off, width, True, ready)

    def to_device(self, col_off: int, width: int) -> torch.cuda.Event:
        """Restore those columns from the host mirrors (e.g. after the device
        copy of the parity was lost).  The copies start after the work already
        queued on the current stream (an encode or decode that still reads or
        writes those columns), and the current stream is made to wait for
        them."""
        cur = torch.cuda.current_stream(self.device)
        ready = torch.cuda.Event()
        ready.record(cur)
        done = self._copy(col_off, width, False, ready)
        cur.wait_event(done)
        return done
