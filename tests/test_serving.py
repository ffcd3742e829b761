"""Serving hook host logic on the CPU: the JSONL writer, the chunk counter
(alone, and across two gloo ranks), and the forward_extend wrapper
(bench_ghostserve_rdp.py:232-244, :285-300, :396-481)."""
import json
import os
import socket

import pytest
import torch
import torch.multiprocessing as mp

from conftest import load_pkg


def test_metrics_log_appends_json_lines(tmp_path):
    serving = load_pkg().serving
    path = tmp_path / "m.jsonl"
    log = serving.MetricsLog(str(path))
    log.append({"chunk_id": 1, "timings": {"rdp_encode_ms": 0.5}})
    log.append({"chunk_id": 2})
    lines = path.read_text().splitlines()
    assert [json.loads(x)["chunk_id"] for x in lines] == [1, 2]
    serving.MetricsLog(None).append({"x": 1})   # no file: no output, no error


def test_chunk_counter_single_process():
    c = load_pkg().serving.ChunkCounter()
    assert [c.next(torch.device("cpu")) for _ in range(3)] == [(1, 0), (2, 0), (3, 0)]


def _counter_rank(rank, world, port, out):
    import torch.distributed as dist
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank,
                            world_size=world)
    try:
        c = load_pkg().serving.ChunkCounter()
        if rank == 1:
            c.count = 100   # only rank 0's count is authoritative
        out[rank] = [c.next(torch.device("cpu")) for _ in range(5)]
    finally:
        dist.destroy_process_group()


def test_chunk_counter_two_ranks_agree_and_rotate():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    ctx = mp.get_context("spawn")
    with ctx.Manager() as m:
        out = m.dict()
        procs = [ctx.Process(target=_counter_rank, args=(r, 2, port, out)) for r in range(2)]
        for p in procs:
            p.start()
        for p in procs:
            p.join(120)
            assert p.exitcode == 0
        want = [(i, (i - 1) % 2) for i in range(1, 6)]
        assert out[0] == want and out[1] == want


def _rows_rank(rank, world, port, out):
    """The hook's exchange of one step: every rank's [K | V] row to the
    rotating owner dst = (chunk_id - 1) % world (bench_ghostserve_rdp.py:
    302-332), over gloo with host tensors; three chunks, so the owner moves."""
    import torch.distributed as dist
    dist.init_process_group("gloo", init_method=f"tcp://127.0.0.1:{port}", rank=rank,
                            world_size=world)
    try:
        serving = load_pkg().serving
        hook = serving.KVParityHook(star_base=0, metrics_file=None)
        got = []
        for _ in range(3):
            cid, dst = hook.counter.next(torch.device("cpu"))
            S = 6
            mine = torch.arange(S, dtype=torch.int16) + 100 * (rank + 1) + cid
            rows = torch.full((world + 2, S), -1, dtype=torch.int16) if rank == dst else None
            hook._gather_rows(dist, mine, rows, dst, torch.device("cpu"))
            got.append((cid, dst, rows[:world].tolist() if rows is not None else None))
        out[rank] = got
    finally:
        dist.destroy_process_group()


def test_row_exchange_two_ranks_reaches_the_rotating_owner():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    ctx = mp.get_context("spawn")
    with ctx.Manager() as m:
        out = m.dict()
        procs = [ctx.Process(target=_rows_rank, args=(r, 2, port, out)) for r in range(2)]
        for p in procs:
            p.start()
        for p in procs:
            p.join(120)
            assert p.exitcode == 0
        for cid in (1, 2, 3):
            dst = (cid - 1) % 2
            want = [[100 * (r + 1) + cid + i for i in range(6)] for r in range(2)]
            for rank in range(2):
                c, d, rows = out[rank][cid - 1]
                assert (c, d) == (cid, dst)
                assert rows == (want if rank == dst else None), (cid, rank)


class _Hook:
    def __init__(self, fail=False):
        self.calls, self.fail = [], fail

    def on_extend(self, pool, slots):
        if self.fail:
            raise RuntimeError("boom")
        self.calls.append((pool, slots))


class _Batch:
    def __init__(self, slots):
        self.slot_mapping = slots


class _Backend:
    def __init__(self, attr):
        setattr(self, attr, torch.zeros(4, 2, 1, 8))
        self.seen = []

    def forward_extend(self, q, k=None, batch=None, save_kv_cache=True):
        self.seen.append((q, k, batch, save_kv_cache))
        return "out"


class _Runner:
    def __init__(self, backend, name="attn_backend"):
        setattr(self, name, backend)


@pytest.mark.parametrize("attr", ["kv_buffer", "kv_pool", "kv_cache"])
def test_install_passes_arguments_through_and_feeds_the_hook(attr):
    serving = load_pkg().serving
    be = _Backend(attr)
    hook = _Hook()
    assert serving.install(_Runner(be), hook) is hook
    b = _Batch([3, -1, 0])
    assert be.forward_extend("q", k="k", batch=b, save_kv_cache=False) == "out"
    assert be.seen == [("q", "k", b, False)]
    assert len(hook.calls) == 1 and hook.calls[0][1] == [3, -1, 0]
    assert hook.calls[0][0] is getattr(be, attr)
    # the batch may also come as the first positional argument
    be.forward_extend(_Batch([1]))
    assert hook.calls[-1][1] == [1]
    # a second install keeps the first hook and does not wrap twice
    assert serving.install(_Runner(be), _Hook()) is hook
    be.forward_extend("q", batch=b)
    assert len(hook.calls) == 3


def test_install_reports_hook_errors_without_failing_the_step():
    serving = load_pkg().serving
    be = _Backend("kv_pool")
    errs = []
    serving.install(_Runner(be, "attention_backend"), _Hook(fail=True), on_error=errs.append)
    assert be.forward_extend("q", batch=_Batch([0])) == "out"
    assert len(errs) == 1 and "boom" in str(errs[0])


def test_install_needs_a_backend_with_forward_extend():
    serving = load_pkg().serving
    with pytest.raises(ValueError):
        serving.install(object())


def test_hook_reads_the_reference_environment(monkeypatch, tmp_path):
    serving = load_pkg().serving
    monkeypatch.setenv("RDP_STAR_BASE", "7")
    monkeypatch.setenv("FT_METRICS_FILE", str(tmp_path / "x.jsonl"))
    monkeypatch.setenv("FT_PROG_START_MONO", "12.5")
    h = serving.KVParityHook()
    assert h.star_base == 7 and h.metrics.path == str(tmp_path / "x.jsonl")
    assert h.prog_start_mono == 12.5
    assert os.environ["RDP_STAR_BASE"] == "7"
