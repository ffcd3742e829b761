"""Serving hook: parity of every prefill step's KV delta, with JSONL metrics.

The counterpart of the reference's serving plugin (bench_ghostserve_rdp.py:
211-481, a sitecustomize module patched into SGLang's FlashInfer backend).
After the attention backend's ``forward_extend``, the KV slots that step wrote
(``batch.slot_mapping``, -1 = no slot) are the chunk's delta.  Per chunk:

  * the chunk counter advances: rank 0 counts and broadcasts, and the parity
    owner rotates, dst = (chunk_id - 1) % world (:285-300);
  * each rank's delta becomes one parity row, all K words then all V words
    (pack_row_from_block, :105-118), and the rows go to dst (:302-332);
  * dst computes the star-diagonal P/Q of the rows (compute_rdp_parity,
    :121-150) and copies them to host memory (:362-374);
  * one JSONL record per chunk goes to FT_METRICS_FILE with the reference's
    fields (chunk_id, dst_rank, first_chunk_wall_ms, timings{rdp_encode_ms,
    rdp_decode_ms, gpu_to_cpu_ms, cpu_to_gpu_ms, parity_bytes}; :376-389).

Environment (as the reference reads it): RDP_STAR_BASE, FT_METRICS_FILE,
FT_PROG_START_MONO.

What differs:
  * the delta is gathered by the paged-gather kernel straight into the row,
    K half and V half (one pass; the reference indexes the pool twice, copies
    to fp16 and packs).  KV of any 2-byte dtype is coded as raw bits.  For an
    fp16 pool the parity bytes are the reference's; for a bf16 pool they are
    on purpose not, since the reference's .to(torch.float16) before packing
    (bench_ghostserve_rdp.py:345-346) is lossy and its parity cannot rebuild
    the bf16 cache;
  * the host copy of P/Q runs on a side stream into pinned buffers and the
    record is written once that copy has finished (checked at the next step
    or at ``flush()``), instead of a device-wide synchronize per chunk; its
    gpu_to_cpu_ms is the copy's own duration on the GPU;
  * the H2D "probe" copy is made only when asked for (``probe_h2d=True``);
  * any backend with ``forward_extend`` is hooked, not only FlashInfer's
    (ROCm serving backends are not FlashInfer).
The gather of rows to dst is the reference's, and kept: dst receives one row
per other rank, each over its own link of a fully connected node, whereas
XOR-reducing per-rank parity contributions would bring it two rows (P's and
Q's share) per rank.
"""
from __future__ import annotations

import functools
import json
import math
import os
import time
from typing import Callable, Optional

import torch

from . import paged, rdp_kv_ops


def _dist():
    import torch.distributed as dist
    if dist.is_available() and dist.is_initialized():
        return dist
    return None


class ChunkCounter:
    """Global chunk ids (bench_ghostserve_rdp.py:285-300): rank 0 counts, every
    rank receives the id by broadcast; dst = (chunk_id - 1) % world.  The
    broadcast tensor lives on the device for a GPU process group and in host
    memory for gloo."""

    def __init__(self):
        self.count = 0

    def next(self, device: torch.device):
        dist = _dist()
        if dist is None:
            self.count += 1
            return self.count, 0
        if dist.get_rank() == 0:
            self.count += 1
        dev = torch.device("cpu") if dist.get_backend() == "gloo" else device
        t = torch.tensor([self.count], dtype=torch.int64, device=dev)
        dist.broadcast(t, src=0)
        cid = int(t.item())
        self.count = cid
        return cid, (cid - 1) % dist.get_world_size()


class MetricsLog:
    """Append-only JSONL file (bench_ghostserve_rdp.py:232-244); no file, no
    output."""

    def __init__(self, path: Optional[str]):
        self.path = path

    def append(self, entry: dict) -> None:
        if not self.path:
            return
        with open(self.path, "a", encoding="utf-8") as f:
            f.write(json.dumps(entry) + "\n")


class KVParityHook:
    """Per-step parity of the KV delta; call :meth:`on_extend` after each
    ``forward_extend`` (or let :func:`install` do it)."""

    def __init__(self, star_base: Optional[int] = None, metrics_file: Optional[str] = None,
                 prog_start_mono: Optional[float] = None, probe_h2d: bool = False):
        env = os.environ
        self.star_base = int(env.get("RDP_STAR_BASE", "0")) if star_base is None else int(star_base)
        self.metrics = MetricsLog(env.get("FT_METRICS_FILE") if metrics_file is None else metrics_file)
        if prog_start_mono is None:
            prog_start_mono = float(env.get("FT_PROG_START_MONO", "nan"))
        self.prog_start_mono = prog_start_mono
        self.probe_h2d = probe_h2d
        self.counter = ChunkCounter()
        self.first_chunk_wall_ms: Optional[float] = None
        self._stream: Optional[torch.cuda.Stream] = None
        self._pending: list = []
        self.last_parity = None   # (P, Q) host tensors of the newest finished chunk

    # ------------------------------------------------------------ per step
    def on_extend(self, kv_pool: torch.Tensor, slot_mapping) -> Optional[int]:
        """Code this step's delta.  ``kv_pool``: [max_tokens, 2, kv_heads,
        head_dim] of a 2-byte dtype; ``slot_mapping``: the slots written this
        step, -1 for none.  Returns the chunk id, or None for an empty step."""
        self.poll()
        if kv_pool.dim() != 4 or kv_pool.shape[1] != 2 or kv_pool.element_size() != 2:
            raise ValueError("kv_pool must be [max_tokens, 2, kv_heads, head_dim] of a 2-byte dtype")
        if not kv_pool.is_contiguous():
            raise ValueError("kv_pool must be contiguous")
        dev = kv_pool.device
        slots = torch.as_tensor(slot_mapping, device=dev).reshape(-1)
        active = slots[slots != -1].to(torch.int32)
        n = int(active.numel())
        if n == 0:
            return None
        cid, dst = self.counter.next(dev)
        if self.first_chunk_wall_ms is None and not math.isnan(self.prog_start_mono):
            self.first_chunk_wall_ms = (time.perf_counter() - self.prog_start_mono) * 1000.0

        T, _, H, D = kv_pool.shape
        elems = n * H * D            # words of K (and of V) in this rank's delta
        S = 2 * elems                # words per row: K then V
        dist = _dist()
        world = dist.get_world_size() if dist is not None else 1
        rank = dist.get_rank() if dist is not None else 0
        rows = torch.empty((world + 2, S), dtype=torch.int16, device=dev) if rank == dst else None
        mine = rows[rank] if rows is not None else torch.empty(S, dtype=torch.int16, device=dev)
        kv = paged.PagedKV(kv_pool.view(1, T, 1, 2, H, D), active.view(1, n), 0, n)
        kv.gather_split(mine[:elems], mine[elems:])
        if world > 1:
            self._gather_rows(dist, mine, rows, dst, dev)
        if rank != dst:
            return cid

        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        rdp_kv_ops.compute_rdp_parity(rows.view(torch.uint16), world, S, self.star_base)
        t1.record()
        # P/Q to pinned host memory on a side stream, after the parity kernel
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=dev)
        P_h = torch.empty(S, dtype=torch.int16, pin_memory=True)
        Q_h = torch.empty(S, dtype=torch.int16, pin_memory=True)
        c0 = torch.cuda.Event(enable_timing=True)
        c1 = torch.cuda.Event(enable_timing=True)
        self._stream.wait_event(t1)
        with torch.cuda.stream(self._stream):
            c0.record(self._stream)
            P_h.copy_(rows[world], non_blocking=True)
            Q_h.copy_(rows[world + 1], non_blocking=True)
            c1.record(self._stream)
            rows.record_stream(self._stream)
            h0 = h1 = None
            if self.probe_h2d:
                h0 = torch.cuda.Event(enable_timing=True)
                h1 = torch.cuda.Event(enable_timing=True)
                probe = torch.empty((2, S), dtype=torch.int16, device=dev)
                h0.record(self._stream)
                probe[0].copy_(P_h, non_blocking=True)
                probe[1].copy_(Q_h, non_blocking=True)
                h1.record(self._stream)
        self._pending.append((cid, dst, (t0, t1), (c0, c1), (h0, h1), P_h, Q_h))
        return cid

    def _gather_rows(self, dist, mine, rows, dst, dev):
        """Every rank's row to dst (bench_ghostserve_rdp.py:302-332).  gloo
        collectives take host tensors, copied synchronously both ways."""
        world = dist.get_world_size()
        if dist.get_backend() == "gloo":
            h = mine.cpu()
            glist = [torch.empty_like(h) for _ in range(world)] if rows is not None else None
            dist.gather(h, gather_list=glist, dst=dst)
            if rows is not None:
                for r in range(world):
                    rows[r].copy_(glist[r].to(dev))
        else:
            glist = [rows[r] for r in range(world)] if rows is not None else None
            dist.gather(mine, gather_list=glist, dst=dst)

    # ------------------------------------------------------------ records
    def poll(self, wait: bool = False) -> int:
        """Write the records of chunks whose host copies have finished (all of
        them with ``wait``); returns how many were written."""
        done = 0
        while self._pending:
            cid, dst, enc, d2h, h2d, P_h, Q_h = self._pending[0]
            last = h2d[1] if h2d[1] is not None else d2h[1]
            if wait:
                last.synchronize()
            elif not last.query():
                break
            self._pending.pop(0)
            self.last_parity = (P_h, Q_h)
            self.metrics.append({
                "chunk_id": int(cid),
                "dst_rank": int(dst),
                "first_chunk_wall_ms": self.first_chunk_wall_ms,
                "timings": {
                    "rdp_encode_ms": float(enc[0].elapsed_time(enc[1])),
                    "rdp_decode_ms": None,
                    "gpu_to_cpu_ms": float(d2h[0].elapsed_time(d2h[1])),
                    "cpu_to_gpu_ms": (float(h2d[0].elapsed_time(h2d[1]))
                                      if h2d[0] is not None else None),
                    "parity_bytes": int(2 * P_h.numel() * 2),
                },
            })
            done += 1
        return done

    def flush(self) -> int:
        return self.poll(wait=True)


_KV_POOL_ATTRS = ("kv_buffer", "kv_pool", "kv_cache")


def install(model_runner, hook: Optional[KVParityHook] = None,
            on_error: Optional[Callable[[Exception], None]] = None) -> KVParityHook:
    """Wrap the runner's attention backend ``forward_extend`` like the
    reference's patch (bench_ghostserve_rdp.py:396-481): the original call
    runs first with every argument passed through; then the batch (keyword
    ``batch`` or the first positional argument), the backend's KV pool
    (``kv_buffer``, ``kv_pool`` or ``kv_cache``) and ``batch.slot_mapping``
    feed :meth:`KVParityHook.on_extend`.  A failure in the hook is reported to
    ``on_error`` (default: printed) and never fails the forward pass."""
    backend = getattr(model_runner, "attn_backend", None) or getattr(model_runner, "attention_backend", None)
    if backend is None or not hasattr(backend, "forward_extend"):
        raise ValueError("model runner has no attention backend with forward_extend")
    if getattr(backend, "_kvec_hooked", None) is not None:
        return backend._kvec_hooked
    hook = hook or KVParityHook()
    orig = backend.forward_extend

    @functools.wraps(orig)
    def forward_extend(*args, **kwargs):
        res = orig(*args, **kwargs)
        try:
            batch = kwargs.get("batch", None)
            if batch is None and args:
                batch = args[0]
            pool = next((getattr(backend, a) for a in _KV_POOL_ATTRS
                         if getattr(backend, a, None) is not None), None)
            slots = getattr(batch, "slot_mapping", None) if batch is not None else None
            if pool is not None and slots is not None:
                hook.on_extend(pool, slots)
        except Exception as e:  # the serving loop must not fail on parity
            (on_error or (lambda x: print(f"[kvec] parity hook error: {x}", flush=True)))(e)
        return res

    backend.forward_extend = forward_extend
    backend._kvec_hooked = hook
    return hook
