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


class _StepPlan:
    """Resources of one step shape (active slots, heads, head_dim, dtype,
    pool, group size, star_base), reused while the shape repeats: two row
    buffers [world + 2, S] used in turn and, with graphs, a static slot
    buffer, the paged-gather descriptor over it and one HIP graph per row
    buffer for the gather of this rank's delta and one for P/Q.

    A step's P/Q rows are read by its host copies on the side stream, so
    before a buffer is written again (two steps later) the current stream
    waits, on the device, for the event that marks those copies done."""

    def __init__(self, kv_pool: torch.Tensor, n: int, world: int, rank: int, star_base: int,
                 graphs: bool):
        dev = kv_pool.device
        T, _, H, D = kv_pool.shape
        self.world, self.rank, self.star_base = world, rank, star_base
        self.elems = n * H * D          # words of K (and of V) in one rank's delta
        self.S = 2 * self.elems         # words per row: K then V
        self.rows = [torch.empty((world + 2, self.S), dtype=torch.int16, device=dev) for _ in range(2)]
        self.pool6 = kv_pool.view(1, T, 1, 2, H, D)
        self.n = n
        if graphs:
            self.slots = torch.empty(n, dtype=torch.int32, device=dev)
            self.kv = paged.PagedKV(self.pool6, self.slots.view(1, n), 0, n)
        self.freed = [None, None]
        self.graphs = graphs
        self.g_gather = [None, None]
        self.g_parity = [None, None]
        self.turn = 0

    def _gather(self, b: int, kv: paged.PagedKV):
        mine = self.rows[b][self.rank]
        kv.gather_split(mine[:self.elems], mine[self.elems:])

    def _parity(self, b: int):
        rdp_kv_ops.compute_rdp_parity(self.rows[b].view(torch.uint16), self.world, self.S, self.star_base)

    def _replay(self, which: list, fn, b: int):
        if which[b] is None:
            # captured on torch.cuda.graph's side stream; replays are ordered
            # on the current one
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn(b)
            which[b] = g
        which[b].replay()

    def begin(self, active: torch.Tensor) -> int:
        """Take the next row buffer (after the host copies that last read
        it) and, with graphs, load this step's slots; returns the buffer."""
        b = self.turn
        self.turn ^= 1
        if self.freed[b] is not None:
            torch.cuda.current_stream(active.device).wait_event(self.freed[b])
        self.active = active
        if self.graphs:
            self.slots.copy_(active, non_blocking=True)
        return b

    def gather(self, b: int):
        if self.graphs:
            self._replay(self.g_gather, lambda bb: self._gather(bb, self.kv), b)
        else:
            self._gather(b, paged.PagedKV(self.pool6, self.active.view(1, self.n), 0, self.n))

    def parity(self, b: int):
        if self.graphs:
            self._replay(self.g_parity, self._parity, b)
        else:
            self._parity(b)


class KVParityHook:
    """Per-step parity of the KV delta; call :meth:`on_extend` after each
    ``forward_extend`` (or let :func:`install` do it).

    ``graphs``: replay each step's gather and P/Q kernels from HIP graphs
    captured once per step shape (the first step of a shape captures them)
    instead of launching them through the C calls.  Off by default: on
    MI355X with torch 2.10 a graph replay costs the host about as much as
    the two launches it replaces, plus a device copy of the slots, and the
    owner's step at TP8 took 219 against 203 us per step."""

    def __init__(self, star_base: Optional[int] = None, metrics_file: Optional[str] = None,
                 prog_start_mono: Optional[float] = None, probe_h2d: bool = False,
                 graphs: bool = False):
        env = os.environ
        self.star_base = int(env.get("RDP_STAR_BASE", "0")) if star_base is None else int(star_base)
        self.metrics = MetricsLog(env.get("FT_METRICS_FILE") if metrics_file is None else metrics_file)
        if prog_start_mono is None:
            prog_start_mono = float(env.get("FT_PROG_START_MONO", "nan"))
        self.prog_start_mono = prog_start_mono
        self.probe_h2d = probe_h2d
        self.graphs = graphs
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
    def _active(slot_mapping, dev) -> torch.Tensor:
        """The slots written this step (-1 entries dropped), int32 on the
        device.  The count is needed on the host (it sizes the rows), so a
        device slot_mapping costs one synchronization here, as in the
        reference (bench_ghostserve_rdp.py:449-451); a host one costs none."""
        slots = torch.as_tensor(slot_mapping).reshape(-1)
        if slots.device.type == "cpu":
            # pinned, so the upload is queued behind the device's work
            # instead of waiting for it
            return slots[slots != -1].to(torch.int32).pin_memory().to(dev, non_blocking=True)
        slots = slots.to(dev)
        return slots[slots != -1].to(torch.int32)

    MAX_PLANS = 8   # step shapes kept (prefill chunks of a few sizes repeat)

    def _plan(self, kv_pool: torch.Tensor, n: int, world: int, rank: int) -> _StepPlan:
        key = (kv_pool.data_ptr(), tuple(kv_pool.shape), kv_pool.dtype, n, world, rank, self.star_base)
        plan = self._plans.pop(key, None)
        if plan is None:
            if len(self._plans) >= self.MAX_PLANS:
                # the least recently used shape: its rows go back to the
                # allocator only once the copies queued on the side stream
                # have read them
                old = self._plans.pop(next(iter(self._plans)))
                if self._stream is not None:
                    for r in old.rows:
                        r.record_stream(self._stream)
            plan = _StepPlan(kv_pool, n, world, rank, self.star_base, self.graphs)
        self._plans[key] = plan   # most recently used last
        return plan

    def on_extend(self, kv_pool: torch.Tensor, slot_mapping) -> Optional[int]:
        """Code this step's delta.  ``kv_pool``: [max_tokens, 2, kv_heads,
        head_dim] of a 2-byte dtype; ``slot_mapping``: the slots written this
        step, -1 for none.  Returns the chunk id, or None for an empty step."""
        self.poll()
        self._check_pool(kv_pool)
        dev = kv_pool.device
        active = self._active(slot_mapping, dev)
        n = int(active.numel())
        if n == 0:
            return None
        cid, dst = self.counter.next(dev)
        if self.first_chunk_wall_ms is None and not math.isnan(self.prog_start_mono):
            self.first_chunk_wall_ms = (time.perf_counter() - self.prog_start_mono) * 1000.0
        dist = _dist()
        world = dist.get_world_size() if dist is not None else 1
        rank = dist.get_rank() if dist is not None else 0
        plan = self._plan(kv_pool, n, world, rank)
        b = plan.begin(active)
        plan.gather(b)
        if world > 1:
            self._gather_rows(dist, plan.rows[b][rank], plan.rows[b] if rank == dst else None, dst, dev)
        if rank == dst:
            self._code_owner(plan, b, cid, dst)
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
        active = self._active(slot_mapping, kv_pool.device)
        n = int(active.numel())
        if n == 0:
            return None
        self.counter.count += 1
        plan = self._plan(kv_pool, n, int(world), 0)
        b = plan.begin(active)
        plan.gather(b)
        self._code_owner(plan, b, self.counter.count, 0)
        return self.counter.count

    def _code_owner(self, plan: _StepPlan, b: int, cid: int, dst: int) -> None:
        """P/Q of the row buffer and their copy to pinned host memory on a
        side stream (the two rows are adjacent: one copy); the JSONL record
        waits for that copy."""
        dev = plan.rows[b].device
        rows, world, S = plan.rows[b], plan.world, plan.S
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        plan.parity(b)
        t1.record()
        # P/Q to pinned host memory on a side stream, after the parity kernel
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=dev)
        PQ_h = torch.empty((2, S), dtype=torch.int16, pin_memory=True)
        P_h, Q_h = PQ_h[0], PQ_h[1]
        c0 = torch.cuda.Event(enable_timing=True)
        c1 = torch.cuda.Event(enable_timing=True)
        self._stream.wait_event(t1)
        with torch.cuda.stream(self._stream):
            c0.record(self._stream)
            PQ_h.copy_(rows[world:world + 2], non_blocking=True)
            c1.record(self._stream)
            h0 = h1 = None
            if self.probe_h2d:
                h0 = torch.cuda.Event(enable_timing=True)
                h1 = torch.cuda.Event(enable_timing=True)
                probe = torch.empty((2, S), dtype=torch.int16, device=dev)
                h0.record(self._stream)
                probe.copy_(PQ_h, non_blocking=True)
                h1.record(self._stream)
        plan.freed[b] = c1
        self._pending.append((cid, dst, (t0, t1), (c0, c1), (h0, h1), P_h, Q_h))

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
