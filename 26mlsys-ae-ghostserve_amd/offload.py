"""Parity offload to host memory, overlapped with coding.

The reference's parity driver copies P and Q of each prefill step to pageable
host memory with ``.to("cpu", non_blocking=True)`` followed by a device-wide
synchronize, then times a host-to-device "probe" copy back
(bench_ghostserve_rdp.py:362-374): the copy is synchronous and blocks the
serving loop.

Here the copies run on a side stream (default priority) into pinned host
buffers, ordered after the encode through an event, so the next chunk's
encode runs while the previous chunk's parity crosses PCIe.  Device-to-host
copies into pinned memory go to the DMA engines, which leave the compute
units and the L2 write path to the encodes (measured beside a 16-chunk fp8
encode: 103 us per encode against 100 alone).  Copies by compute units
stretch those encodes instead: the runtime's blit kernels (the path with
HSA_ENABLE_SDMA=0, and under a kernel-tracing profiler) 12-20x, and a copy
kernel of as few as 8 workgroups storing to host memory 1.7x.  A chunk's parity
is one contiguous region of every parity shard (``chunked``), so offloading
chunk c is one copy per shard and never races with encoding chunk c+1; the
host copy of each shard has the shard's own layout, so a restore is the same
copies in the other direction.
"""
from __future__ import annotations

from typing import Sequence

import torch


class ParityOffload:
    """Pinned host mirrors of parity shards plus a copy stream.

    ``shards`` are the device parity tensors (contiguous, equally sized); the
    host mirrors are byte tensors of the same size.
    """

    def __init__(self, shards: Sequence[torch.Tensor]):
        if not shards:
            raise ValueError("no parity shards")
        sizes = {t.numel() * t.element_size() for t in shards}
        if len(sizes) != 1 or not all(t.is_contiguous() for t in shards):
            raise ValueError("parity shards must be contiguous and of one size")
        self.device = shards[0].device
        self.nbytes = sizes.pop()
        self.dev = [t.view(torch.uint8).view(-1) for t in shards]
        self.host = [torch.empty(self.nbytes, dtype=torch.uint8, pin_memory=True) for _ in shards]
        self.stream = torch.cuda.Stream(device=self.device)

    def _copy(self, off: int, nbytes: int, to_host: bool, after: torch.cuda.Event):
        if off < 0 or nbytes <= 0 or off + nbytes > self.nbytes:
            raise ValueError("byte range outside the parity shards")
        done = torch.cuda.Event()
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(after)
            for d, h in zip(self.dev, self.host):
                src, dst = (d, h) if to_host else (h, d)
                dst[off:off + nbytes].copy_(src[off:off + nbytes], non_blocking=True)
            done.record(self.stream)
        return done

    def to_host(self, off: int, nbytes: int) -> torch.cuda.Event:
        """Copy bytes [off, off+nbytes) of every parity shard (a chunk's
        region) to the host mirrors, after the work already queued on the
        current stream.  Returns the event that marks the copies done."""
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(self.device))
        return self._copy(off, nbytes, True, ready)

    def to_device(self, off: int, nbytes: int) -> torch.cuda.Event:
        """Restore those bytes from the host mirrors (e.g. after the device
        copy of the parity was lost).  The copies start after the work already
        queued on the current stream (an encode or decode that still reads or
        writes those bytes), and the current stream is made to wait for
        them."""
        cur = torch.cuda.current_stream(self.device)
        ready = torch.cuda.Event()
        ready.record(cur)
        done = self._copy(off, nbytes, False, ready)
        cur.wait_event(done)
        return done
