"""Serving hook on the GPU: the split delta gather, and whole steps through
the forward_extend wrapper checked against the oracle's star-diagonal parity
of the reference's [K | V] row (bench_ghostserve_rdp.py:105-150, :340-389)."""
import json

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _pool(gpu, T=300, H=2, D=64, seed=0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(T, 2, H, D, generator=g).to(torch.bfloat16).to(gpu)


def test_gather_split_matches_indexing(pkg, gpu):
    pool = _pool(gpu)
    T, _, H, D = pool.shape
    slots = torch.tensor([5, 17, 3, 299, 0, 42], dtype=torch.int32, device=gpu)
    n = slots.numel()
    kv = pkg.paged.PagedKV(pool.view(1, T, 1, 2, H, D), slots.view(1, n), 0, n)
    k = torch.empty(n * H * D, dtype=torch.bfloat16, device=gpu)
    v = torch.empty_like(k)
    kv.gather_split(k, v)
    idx = slots.long()
    assert torch.equal(k.view(torch.int16), pool[idx, 0].reshape(-1).view(torch.int16))
    assert torch.equal(v.view(torch.int16), pool[idx, 1].reshape(-1).view(torch.int16))


class _Batch:
    def __init__(self, slots):
        self.slot_mapping = slots


class _Backend:
    def __init__(self, pool):
        self.kv_buffer = pool

    def forward_extend(self, q, batch=None):
        return q


class _Runner:
    def __init__(self, be):
        self.attn_backend = be


@pytest.mark.parametrize("star_base", [0, 5])
def test_hook_steps_match_oracle(pkg, ora, gpu, tmp_path, star_base):
    pool = _pool(gpu, seed=star_base)
    be = _Backend(pool)
    path = tmp_path / "metrics.jsonl"
    hook = pkg.serving.install(_Runner(be), pkg.serving.KVParityHook(
        star_base=star_base, metrics_file=str(path), prog_start_mono=0.0, probe_h2d=True),
        on_error=lambda e: (_ for _ in ()).throw(e))
    steps = [[7, 8, 9, -1, 10], [-1, -1], [100, 3, 250, 251, 252, 253, 11, 12]]
    got = []
    for st in steps:
        be.forward_extend("q", batch=_Batch(torch.tensor(st, device=gpu)))
        hook.flush()
        got.append(hook.last_parity)
    recs = [json.loads(x) for x in path.read_text().splitlines()]
    assert [r["chunk_id"] for r in recs] == [1, 2]   # the empty step codes nothing
    for r in recs:
        assert r["dst_rank"] == 0 and r["first_chunk_wall_ms"] is not None
        t = r["timings"]
        assert set(t) == {"rdp_encode_ms", "rdp_decode_ms", "gpu_to_cpu_ms", "cpu_to_gpu_ms",
                          "parity_bytes"}
        assert t["rdp_encode_ms"] >= 0 and t["gpu_to_cpu_ms"] >= 0 and t["cpu_to_gpu_ms"] >= 0
        assert t["rdp_decode_ms"] is None
    host = pool.cpu().view(torch.int16).numpy().view(np.uint16)
    for st, (P, Q), rec in zip([steps[0], steps[2]], [got[0], got[2]], recs):
        act = [s for s in st if s != -1]
        row = np.concatenate([host[act, 0].reshape(-1), host[act, 1].reshape(-1)])
        S = row.size
        rows = np.zeros((3, S), np.uint16)
        rows[0] = row
        ora.gs_parity(rows, 1, S, star_base)
        assert np.array_equal(P.numpy().view(np.uint16), rows[1])
        assert np.array_equal(Q.numpy().view(np.uint16), rows[2])
        assert rec["timings"]["parity_bytes"] == 2 * S * 2


def _row_of(host, slots):
    act = [s for s in slots if s != -1]
    return np.concatenate([host[act, 0].reshape(-1), host[act, 1].reshape(-1)])


def test_hook_repeated_shapes_and_host_slots(pkg, ora, gpu, monkeypatch):
    """Steps of two shapes in turn, each repeated with new slots (a plan is
    evicted and rebuilt when only one is kept), the slots given as a device
    tensor, a host tensor or a list: every chunk's P/Q is the oracle's."""
    monkeypatch.setattr(pkg.serving.KVParityHook, "MAX_PLANS", 1)
    pool = _pool(gpu, T=400, seed=3)
    host = pool.cpu().view(torch.int16).numpy().view(np.uint16)
    hook = pkg.serving.KVParityHook(star_base=2)
    rng = np.random.default_rng(4)
    for i in range(7):
        n = 5 if i % 3 else 9
        sl = [int(x) for x in rng.choice(400, n, replace=False)]
        if i == 2:
            sl[1] = -1
        arg = [torch.tensor(sl, device=gpu), torch.tensor(sl), sl][i % 3]
        assert hook.on_extend(pool, arg) == i + 1
        hook.flush()
        P, Q = hook.last_parity
        row = _row_of(host, sl)
        rows = np.zeros((3, row.size), np.uint16)
        rows[0] = row
        ora.gs_parity(rows, 1, row.size, 2)
        assert np.array_equal(P.numpy().view(np.uint16), rows[1]), i
        assert np.array_equal(Q.numpy().view(np.uint16), rows[2]), i


def test_owner_step_at_group_of_eight(pkg, ora, gpu):
    """The parity owner's step in a group of 8 ranks, in one process: row 0
    is this rank's delta, rows 1-7 whatever the buffer holds (set here), and
    P/Q are those of all 8 rows; three steps, so both row buffers are
    reused."""
    pool = _pool(gpu, T=500, H=1, D=128, seed=5)
    host = pool.cpu().view(torch.int16).numpy().view(np.uint16)
    hook = pkg.serving.KVParityHook(star_base=0)
    rng = np.random.default_rng(6)
    for i in range(3):
        sl = [int(x) for x in rng.choice(500, 64, replace=False)]
        if i == 0:
            hook.step_as_owner(pool, torch.tensor(sl, device=gpu), 8)
            hook.flush()
            plan = next(iter(hook._plans.values()))
            for b in range(2):
                plan.rows[b][1:8].view(torch.uint16).copy_(
                    torch.from_numpy(rng.integers(0, 65536, (7, plan.S), dtype=np.uint16)).to(gpu))
            torch.cuda.synchronize()
        b = plan.turn if i else None
        others = plan.rows[plan.turn][1:8].cpu().numpy().view(np.uint16).copy() if i else None
        hook.step_as_owner(pool, torch.tensor(sl, device=gpu), 8)
        hook.flush()
        if not i:
            continue
        P, Q = hook.last_parity
        rows = np.zeros((10, plan.S), np.uint16)
        rows[0] = _row_of(host, sl)
        rows[1:8] = others
        ora.gs_parity(rows, 8, plan.S, 0)
        assert np.array_equal(P.numpy().view(np.uint16), rows[8]), (i, b)
        assert np.array_equal(Q.numpy().view(np.uint16), rows[9]), (i, b)


def test_hook_step_split_calls_and_checks(pkg, ora, gpu):
    """kvec_hook_step through the C ABI in the two halves a multi-rank step
    uses: the gather of this rank's row alone (no host copy), then, after the
    rows have arrived, P/Q and their copy to pinned memory on a second stream
    with the four events; P, Q and the row against the oracle.  Then the
    argument checks: a row outside the group, a delta that is not a row's
    size, a separate copy stream without event 1."""
    import ctypes
    lib = pkg._lib
    pool = _pool(gpu, T=300, H=1, D=64, seed=9)
    T, _, H, D = pool.shape
    host = pool.cpu().view(torch.int16).numpy().view(np.uint16)
    world, rank, n = 4, 2, 24
    rng = np.random.default_rng(10)
    sl = rng.choice(T, n, replace=False).astype(np.int32)
    slots_dev = torch.empty(n, dtype=torch.int32, device=gpu)
    staging = torch.from_numpy(sl.copy()).pin_memory()
    kv = pkg.paged.PagedKV(pool.view(1, T, 1, 2, H, D), slots_dev.view(1, n), 0, n)
    S = 2 * n * H * D
    rows = torch.from_numpy(rng.integers(0, 65536, (world + 2, S), dtype=np.uint16).view(np.int16)).to(gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    lib.call("kvec_hook_step", kv.c, staging.data_ptr(), rows.data_ptr(), rank, world, S, 3, None, stream,
             None, None, None)
    side = torch.cuda.Stream(device=gpu)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in evs:
        e.record()
    ev_arr = (ctypes.c_void_p * 4)(*[e.cuda_event for e in evs])
    pq = torch.empty((2, S), dtype=torch.int16, pin_memory=True)
    lib.call("kvec_hook_step", None, None, rows.data_ptr(), 0, world, S, 3, pq.data_ptr(), stream,
             side.cuda_stream, None, ev_arr)
    evs[3].synchronize()
    torch.cuda.synchronize()
    got = rows.cpu().numpy().view(np.uint16)
    assert np.array_equal(got[rank], _row_of(host, sl.tolist()))
    want = got.copy()
    want[world:] = 0
    ora.gs_parity(want, world, S, 3)
    assert np.array_equal(got[world:], want[world:])
    assert np.array_equal(pq.numpy().view(np.uint16), want[world:])
    assert evs[0].elapsed_time(evs[1]) >= 0 and evs[2].elapsed_time(evs[3]) >= 0
    bad = [
        (kv.c, None, rows.data_ptr(), world, world, S, 0, None, stream, None, None, None),
        (kv.c, None, rows.data_ptr(), 0, world, S + 8, 0, None, stream, None, None, None),
        (None, None, rows.data_ptr(), 0, world, S, 0, pq.data_ptr(), stream, side.cuda_stream, None, None),
    ]
    for args in bad:
        with pytest.raises(lib.KvecError, match="kvec_hook_step"):
            lib.call("kvec_hook_step", *args)
    torch.cuda.synchronize()


@pytest.mark.parametrize("probe", [False, True])
def test_hook_ring_wraps_with_steps_in_flight(pkg, ora, gpu, tmp_path, probe):
    """Eleven steps issued without a flush between them (the pinned P/Q ring
    holds four): every step gets its record, in chunk order, and the last
    step's P/Q is the oracle's; the host slot maps alternate between the two
    staging buffers while earlier uploads may still be queued.  With the
    reference's host-to-device probe, a ring slot is reused only after its
    step's probe copy too."""
    import json
    pool = _pool(gpu, T=600, H=1, D=128, seed=12)
    host = pool.cpu().view(torch.int16).numpy().view(np.uint16)
    path = tmp_path / "m.jsonl"
    hook = pkg.serving.KVParityHook(star_base=1, metrics_file=str(path), probe_h2d=probe)
    rng = np.random.default_rng(13)
    sets = [rng.choice(600, 40, replace=False).tolist() for _ in range(11)]
    for sl in sets:
        hook.on_extend(pool, torch.tensor(sl))
    hook.flush()
    hook.metrics.close()
    recs = [json.loads(x) for x in path.read_text().splitlines()]
    assert [r["chunk_id"] for r in recs] == list(range(1, 12))
    assert all((r["timings"]["cpu_to_gpu_ms"] is not None) == probe for r in recs)
    P, Q = hook.last_parity
    row = _row_of(host, sets[-1])
    rows = np.zeros((3, row.size), np.uint16)
    rows[0] = row
    ora.gs_parity(rows, 1, row.size, 1)
    assert np.array_equal(P.numpy().view(np.uint16), rows[1])
    assert np.array_equal(Q.numpy().view(np.uint16), rows[2])
