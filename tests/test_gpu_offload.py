"""Parity offload to pinned host memory on a side stream, ordered after the
encode, and the restore of lost device parity from the host copy."""
import numpy as np
import pytest
import torch

from test_gpu_chunked import setup

pytestmark = pytest.mark.gpu


def test_offload_and_restore(pkg, gpu):
    L, B, pps, pt, H, D, k, p, m, ct = 2, 3, 8, 16, 1, 128, 5, 7, 3, 32
    _, _, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct, False, seed=8)
    par = [st.P, st.Q] + list(st.rs)
    off = pkg.offload.ParityOffload(par)
    n = st.region_bytes
    evs = []
    for c in range(nc):
        st.encode(pkg.chunked.chunk_kv(pool_d, table_d, c, ct), c)
        evs.append(off.to_host(st.region(c), n))    # copy of chunk c overlaps encode of c+1
    for e in evs:
        e.synchronize()
    torch.cuda.synchronize()
    for d, h in zip(par, off.host):
        assert np.array_equal(d.cpu().numpy(), h.numpy())
    want = [t.clone() for t in par]
    for t in par:
        t[st.region(1):st.region(2)] = 0xEE           # chunk 1's device parity lost
    off.to_device(st.region(1), n)
    torch.cuda.synchronize()
    for t, w in zip(par, want):
        assert torch.equal(t, w)


def test_offload_restore_waits_for_queued_work(pkg, gpu):
    """A restore queued right behind an encode of the same bytes starts after
    it: the restored bytes are the host copy, not the encode's output."""
    L, B, pps, pt, H, D, k, p, m, ct = 2, 3, 8, 16, 1, 128, 5, 7, 3, 32
    _, _, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct, False, seed=9)
    par = [st.P, st.Q] + list(st.rs)
    off = pkg.offload.ParityOffload(par)
    n = st.region_bytes
    for h in off.host:
        h.fill_(0x42)
    kv0 = pkg.chunked.chunk_kv(pool_d, table_d, 0, ct)
    for _ in range(4):
        st.encode(kv0, 0)                            # queued on the current stream
    off.to_device(0, n)                              # must run after the encodes
    torch.cuda.synchronize()
    for t in par:
        assert bool((t[:n] == 0x42).all())


def test_offload_rejects_bad_ranges(pkg, gpu):
    t = [torch.zeros(6 * 64, dtype=torch.uint8, device=gpu)]
    off = pkg.offload.ParityOffload(t)
    with pytest.raises(ValueError):
        off.to_host(6 * 64 - 16, 32)
    with pytest.raises(ValueError):
        pkg.offload.ParityOffload([torch.zeros(100, dtype=torch.uint8, device=gpu),
                                   torch.zeros(64, dtype=torch.uint8, device=gpu)])
