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
  * the step's device work (slot upload, gather, P/Q, the copy and the
    events that time them) is enqueued by one native call, kvec_hook_step,
    over buffers and events made once per step shape;
  * the H2D "probe" copy is made only when asked for (``probe_h2d=True``);
  * any backend with ``forward_extend`` is hooked, not only FlashInfer's
    (ROCm serving backends are not FlashInfer).
The gather of rows to dst is the reference's, and kept: dst receives one row
per other rank, each over its own link of a fully connected node, whereas
XOR-reducing per-rank parity contributions would bring it two rows (P's and
Q's share) per rank.
"""
from __future__ import annotations

import ctypes
import functools
import json
import math
import os
import time
from typing import Callable, Optional

import numpy as np
import torch

from . import _lib, paged


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
    output.  The reference opens the file for every record; here it stays
    open in append mode and each line is flushed as it is written, so a
    reader sees the same file, without an open and a close per chunk."""

    def __init__(self, path: Optional[str]):
        self.path = path
        self._f = None

    def append(self, entry: dict) -> None:
        if not self.path:
            return
        if self._f is None:
            self._f = open(self.path, "a", encoding="utf-8")
        self._f.write(json.dumps(entry) + "\n")
        self._f.flush()

    def close(self) -> None:
        if self._f is not None:
            self._f.close()
            self._f = None

    def __del__(self):
        self.close()


class _StepPlan:
    """Resources of one step shape (active slots, heads, head_dim, dtype,
    pool, group size, rank, star_base), made once and reused while the shape
    repeats:

      * two row buffers [world + 2, S], used in turn;
      * the device slot buffer, the paged-gather descriptor over it, and two
        pinned staging buffers for slot maps given on the host;
      * a ring of pinned [2, S] buffers for the copies of P and Q, each with
        the four events of its step (P/Q start and end, copy start and end).

    A step's P/Q rows are read by its copy on the side stream, so before a row
    buffer is written again (two steps later) the current stream waits, on the
    device, for the event that marks that copy done; and a step's slots are
    uploaded from a staging buffer that is refilled only after that upload."""

    RING = 4

    def __init__(self, kv_pool: torch.Tensor, n: int, world: int, rank: int, star_base: int):
        dev = kv_pool.device
        T, _, H, D = kv_pool.shape
        self.world, self.rank, self.star_base, self.n = world, rank, star_base, n
        self.elems = n * H * D          # words of K (and of V) in one rank's delta
        self.S = 2 * self.elems         # words per row: K then V
        self.rows = [torch.empty((world + 2, self.S), dtype=torch.int16, device=dev) for _ in range(2)]
        self.slots = torch.empty(n, dtype=torch.int32, device=dev)
        self.kv = paged.PagedKV(kv_pool.view(1, T, 1, 2, H, D), self.slots.view(1, n), 0, n)
        self.staging = [torch.empty(n, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self.staging_np = [t.numpy() for t in self.staging]
        self.staged = [None, None]      # event after the upload out of staging[i]
        self.pq = [torch.empty((2, self.S), dtype=torch.int16, pin_memory=True) for _ in range(self.RING)]
        self.events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(self.RING)]
        self.stage_ev = [torch.cuda.Event() for _ in range(2)]
        for e in [x for ev in self.events for x in ev] + self.stage_ev:
            e.record()                  # the HIP events exist from here on: the step records them by handle
        self.ev_args = [(ctypes.c_void_p * 4)(*[e.cuda_event for e in ev]) for ev in self.events]
        self.busy = [False] * self.RING  # ring slot of a step whose record is not written yet
        self.slot = 0
        self.freed = [None, None]       # copy-done event of each row buffer's last step
        self.turn = 0


class KVParityHook:
    """Per-step parity of the KV delta; call :meth:`on_extend` after each
    ``forward_extend`` (or let :func:`install` do it).

    A step is one native call (kvec_hook_step) that enqueues the slot upload,
    the gather of this rank's delta into its row, P/Q and the copy of P and Q
    to pinned host memory, with the events the JSONL timings come from; the
    plan of a step shape (buffers, descriptor, events) is made once.
    ``last_parity`` holds (P, Q) of the newest chunk whose record was written:
    host tensors that stay valid for the next RING - 1 steps of that shape."""

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
        self._plans: dict = {}
        self.last_parity = None   # (P, Q) host tensors of the newest finished chunk

    # ------------------------------------------------------------ per step
    @staticmethod
    def _check_pool(kv_pool: torch.Tensor) -> None:
        if kv_pool.dim() != 4 or kv_pool.shape[1] != 2 or kv_pool.element_size() != 2:
            raise ValueError("kv_pool must be [max_tokens, 2, kv_heads, head_dim] of a 2-byte dtype")
        if not kv_pool.is_contiguous():
            raise ValueError("kv_pool must be contiguous")

    @staticmethod
    def _active(slot_mapping):
        """The slots written this step (-1 entries dropped): an int32 device
        tensor for a device slot_mapping, an int32 numpy array otherwise.  The
        count is needed on the host (it sizes the rows), so a device
        slot_mapping costs one synchronization here, as in the reference
        (bench_ghostserve_rdp.py:449-451); a host one costs none."""
        if isinstance(slot_mapping, torch.Tensor) and slot_mapping.device.type != "cpu":
            slots = slot_mapping.reshape(-1)
            return slots[slots != -1].to(torch.int32)
        a = slot_mapping.numpy() if isinstance(slot_mapping, torch.Tensor) else np.asarray(slot_mapping)
        a = a.reshape(-1)
        return a[a != -1].astype(np.int32, copy=False)

    MAX_PLANS = 8   # step shapes kept (prefill chunks of a few sizes repeat)

    def _plan(self, kv_pool: torch.Tensor, n: int, world: int, rank: int) -> _StepPlan:
        key = (kv_pool.data_ptr(), tuple(kv_pool.shape), kv_pool.dtype, n, world, rank, self.star_base)
        plan = self._plans.pop(key, None)
        if plan is None:
            if len(self._plans) >= self.MAX_PLANS:
                # the least recently used shape: its rows go back to the
                # allocator only once the copies queued on the side stream
                # have read them (its host buffers stay referenced by the
                # pending records)
                old = self._plans.pop(next(iter(self._plans)))
                if self._stream is not None:
                    for r in old.rows:
                        r.record_stream(self._stream)
                # its staging buffers go back to torch's pinned-memory cache,
                # which does not know of the uploads kvec_hook_step queued
                # from them: those must have run first
                for e in old.staged:
                    if e is not None:
                        e.synchronize()
            plan = _StepPlan(kv_pool, n, world, rank, self.star_base)
        self._plans[key] = plan   # most recently used last
        return plan

    def _begin(self, plan: _StepPlan, act):
        """Take the next row buffer and stage this step's slots: a host array
        goes to a pinned staging buffer (refilled only once its last upload
        has run), a device tensor straight into the plan's slot buffer.
        Returns the row buffer and the staging buffer's address (None)."""
        b = plan.turn
        plan.turn ^= 1
        if isinstance(act, np.ndarray):
            if plan.staged[b] is not None:
                plan.staged[b].synchronize()
            plan.staging_np[b][:] = act
            return b, plan.staging[b].data_ptr()
        plan.slots.copy_(act)
        return b, None

    def _issue(self, plan: _StepPlan, b: int, staging, gather: bool, code: bool, cid: int, dst: int):
        """One kvec_hook_step: [the wait for the row buffer, the slot upload
        and the gather of this rank's row] and/or [P/Q and their copy to the
        next pinned ring buffer on the side stream]."""
        dev = plan.rows[b].device
        stream = torch.cuda.current_stream(dev).cuda_stream
        pq = side = evs = None
        if code:
            if self._stream is None:
                self._stream = torch.cuda.Stream(device=dev)
            s = plan.slot
            plan.slot = (s + 1) % plan.RING
            if plan.busy[s]:
                # the ring came round to a step whose record is not written:
                # wait for that step's last copy (its probe's, if it made
                # one); the records before it finished earlier on the same
                # side stream, so the poll writes them all
                for ent in self._pending:
                    if ent[2] is plan and ent[3] == s:
                        (ent[4][1] if ent[4] is not None else plan.events[s][3]).synchronize()
                        break
                self.poll()
            pq, side, evs = plan.pq[s].data_ptr(), self._stream.cuda_stream, plan.ev_args[s]
        freed = plan.freed[b] if gather else None
        _lib.call("kvec_hook_step", plan.kv.c if gather else None, staging, plan.rows[b].data_ptr(), plan.rank,
                  plan.world, plan.S, plan.star_base, pq, stream, side,
                  freed.cuda_event if freed is not None else None, evs)
        if staging is not None:
            plan.stage_ev[b].record()
            plan.staged[b] = plan.stage_ev[b]
        if not code:
            return
        plan.busy[s] = True
        plan.freed[b] = plan.events[s][3]
        h = None
        if self.probe_h2d:
            # the reference's device-host-device round trip of P/Q (:370-374)
            h = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            with torch.cuda.stream(self._stream):
                probe = torch.empty((2, plan.S), dtype=torch.int16, device=dev)
                h[0].record(self._stream)
                probe.copy_(plan.pq[s], non_blocking=True)
                h[1].record(self._stream)
        self._pending.append((cid, dst, plan, s, h))

    def on_extend(self, kv_pool: torch.Tensor, slot_mapping) -> Optional[int]:
        """Code this step's delta.  ``kv_pool``: [max_tokens, 2, kv_heads,
        head_dim] of a 2-byte dtype; ``slot_mapping``: the slots written this
        step, -1 for none.  Returns the chunk id, or None for an empty step."""
        self.poll()
        self._check_pool(kv_pool)
        dev = kv_pool.device
        act = self._active(slot_mapping)
        n = int(act.shape[0])
        if n == 0:
            return None
        cid, dst = self.counter.next(dev)
        if self.first_chunk_wall_ms is None and not math.isnan(self.prog_start_mono):
            self.first_chunk_wall_ms = (time.perf_counter() - self.prog_start_mono) * 1000.0
        dist = _dist()
        world = dist.get_world_size() if dist is not None else 1
        rank = dist.get_rank() if dist is not None else 0
        plan = self._plan(kv_pool, n, world, rank)
        b, staging = self._begin(plan, act)
        if world == 1:
            self._issue(plan, b, staging, True, True, cid, dst)
            return cid
        self._issue(plan, b, staging, True, False, cid, dst)
        self._gather_rows(dist, plan.rows[b][rank], plan.rows[b] if rank == dst else None, dst, dev)
        if rank == dst:
            self._issue(plan, b, None, False, True, cid, dst)
        return cid

    def step_as_owner(self, kv_pool: torch.Tensor, slot_mapping, world: int) -> Optional[int]:
        """The parity owner's work of one step in a group of ``world`` ranks,
        in one process: this rank's delta gathered into row 0, P/Q of the
        ``world`` rows and their copies to host memory.  The other ranks'
        rows are whatever the row buffer holds (the exchange that would
        bring them is not part of it): a single-GPU measurement of the
        owner's step at a real group size."""
        self.poll()
        self._check_pool(kv_pool)
        act = self._active(slot_mapping)
        n = int(act.shape[0])
        if n == 0:
            return None
        self.counter.count += 1
        plan = self._plan(kv_pool, n, int(world), 0)
        b, staging = self._begin(plan, act)
        self._issue(plan, b, staging, True, True, self.counter.count, 0)
        return self.counter.count

    def _gather_rows(self, dist, mine, rows, dst, dev):
        """Every rank's row to dst (bench_ghostserve_rdp.py:302-332), as bytes:
        neither gloo nor NCCL/RCCL has a 16-bit integer type.  gloo
        collectives take host tensors, copied synchronously both ways."""
        world = dist.get_world_size()
        mine = mine.view(torch.uint8)
        if dist.get_backend() == "gloo":
            h = mine.cpu()
            glist = [torch.empty_like(h) for _ in range(world)] if rows is not None else None
            dist.gather(h, gather_list=glist, dst=dst)
            if rows is not None:
                for r in range(world):
                    rows[r].view(torch.uint8).copy_(glist[r].to(dev))
        else:
            glist = [rows[r].view(torch.uint8) for r in range(world)] if rows is not None else None
            dist.gather(mine, gather_list=glist, dst=dst)

    # ------------------------------------------------------------ records
    def poll(self, wait: bool = False) -> int:
        """Write the records of chunks whose host copies have finished (all of
        them with ``wait``); returns how many were written."""
        done = 0
        while self._pending:
            cid, dst, plan, s, h = self._pending[0]
            ev = plan.events[s]
            last = h[1] if h is not None else ev[3]
            if wait:
                last.synchronize()
            elif not last.query():
                break
            self._pending.pop(0)
            plan.busy[s] = False
            self.last_parity = (plan.pq[s][0], plan.pq[s][1])
            if self.metrics.path:
                self.metrics.append({
                    "chunk_id": int(cid),
                    "dst_rank": int(dst),
                    "first_chunk_wall_ms": self.first_chunk_wall_ms,
                    "timings": {
                        "rdp_encode_ms": float(ev[0].elapsed_time(ev[1])),
                        "rdp_decode_ms": None,
                        "gpu_to_cpu_ms": float(ev[2].elapsed_time(ev[3])),
                        "cpu_to_gpu_ms": float(h[0].elapsed_time(h[1])) if h is not None else None,
                        "parity_bytes": int(2 * plan.S * 2),
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
