"""spec RDP in the striped geometry (stripes of (p-1)*unit bytes, rows of
min(unit, R - s*unit) bytes) on the GPU through the C ABI, bit-exact against
the oracle: encode, every erasure pattern of the decode, the fused paged
gather + encode, and a graph capture of the encode."""
import itertools

import numpy as np
import pytest
import torch

from test_gpu_paged import make_pool, pool_bytes

pytestmark = pytest.mark.gpu


def _to_dev(arrs, dev):
    return [torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).to(dev) for a in arrs]


# (p, k, R, unit): full stripes only, a partial last stripe whose rows are not
# a multiple of 1 KiB, a unit >= R (one stripe), the generic decode's p
@pytest.mark.parametrize("p,k,R,U", [(7, 6, 3 * 65536 + 5 * 1024 + 16, 65536),
                                     (7, 6, 4 * 4096, 4096), (7, 6, 16, 1024),
                                     (7, 4, 2 * 2048 + 48, 2048), (5, 4, 3072, 1024),
                                     (3, 2, 5 * 1024 + 512, 1024), (11, 10, 5000 * 16, 2048),
                                     (13, 12, 2048 + 16, 1024), (7, 6, 4096, 65536)])
def test_striped_encode_matches_oracle(pkg, ora, gpu, p, k, R, U):
    rng = np.random.default_rng(p * 100 + k + R % 97)
    data = [rng.integers(0, 256, (p - 1) * R, dtype=np.uint8) for _ in range(k)]
    Pw, Qw = ora.rdp_encode(data, p, unit=U)
    d = _to_dev(data, gpu)
    P = torch.full(((p - 1) * R,), 0xAA, dtype=torch.uint8, device=gpu)
    Q = torch.full(((p - 1) * R,), 0x55, dtype=torch.uint8, device=gpu)
    pkg.spec.rdp_encode(d, P, Q, p, unit_bytes=U)
    torch.cuda.synchronize()
    assert np.array_equal(P.cpu().numpy(), Pw)
    assert np.array_equal(Q.cpu().numpy(), Qw)


def test_striped_differs_from_planes(pkg, ora, gpu):
    """The unit changes which bytes form an RDP instance: with more than one
    stripe the parity differs from the single-stripe layout's."""
    p, k, R = 7, 6, 4096
    rng = np.random.default_rng(5)
    data = [rng.integers(0, 256, (p - 1) * R, dtype=np.uint8) for _ in range(k)]
    d = _to_dev(data, gpu)
    outs = []
    for U in (0, 1024):
        P = torch.empty((p - 1) * R, dtype=torch.uint8, device=gpu)
        Q = torch.empty_like(P)
        pkg.spec.rdp_encode(d, P, Q, p, unit_bytes=U)
        outs.append(Q.cpu().numpy())
    assert not np.array_equal(outs[0], outs[1])


# compiled networks for (7, 6), (5, 4), (3, 2); the generic kernel otherwise
@pytest.mark.parametrize("p,k,R,U", [(7, 6, 3 * 1024 + 5 * 16, 1024), (5, 4, 2 * 2048 + 1024, 2048),
                                     (3, 2, 1024 + 32, 1024), (7, 5, 2 * 1024 + 16, 1024),
                                     (11, 10, 1024 + 16, 1024)])
def test_striped_decode_all_patterns(pkg, ora, gpu, p, k, R, U):
    rng = np.random.default_rng(p + 17 * k + R)
    data = [rng.integers(0, 256, (p - 1) * R, dtype=np.uint8) for _ in range(k)]
    Pw, Qw = ora.rdp_encode(data, p, unit=U)
    full = data + [Pw, Qw]
    pats = [(e, -1) for e in range(k + 2)] + list(itertools.combinations(range(k + 2), 2))
    for e0, e1 in pats:
        cols = [x.copy() for x in full]
        for e in (e0, e1):
            if e >= 0:
                cols[e][:] = rng.integers(0, 256, cols[e].shape, dtype=np.uint8)
        dev = _to_dev(cols, gpu)
        pkg.spec.rdp_decode(dev, p, [e0, e1], unit_bytes=U)
        torch.cuda.synchronize()
        for s in range(k + 2):
            assert np.array_equal(dev[s].cpu().numpy(), full[s]), (p, k, e0, e1, s)


def test_striped_decode_inconsistent_input_matches_oracle(pkg, ora, gpu):
    """Non-codeword input: the GPU and the oracle apply the same map per stripe."""
    p, k, R, U = 7, 6, 2 * 1024 + 256, 1024
    rng = np.random.default_rng(41)
    for e0, e1 in [(2, -1), (k, k + 1), (0, 5), (1, k)]:
        cols = [rng.integers(0, 256, (p - 1) * R, dtype=np.uint8) for _ in range(k + 2)]
        want = [c.copy() for c in cols]
        ora.rdp_decode(want, p, e0, e1, unit=U)
        dev = _to_dev(cols, gpu)
        pkg.spec.rdp_decode(dev, p, [e0, e1], unit_bytes=U)
        torch.cuda.synchronize()
        for s in range(k + 2):
            assert np.array_equal(dev[s].cpu().numpy(), want[s]), (e0, e1, s)


@pytest.mark.parametrize("p,k,U", [(7, 6, 4096), (7, 6, 1024), (5, 4, 2048), (7, 3, 65536)])
def test_striped_fused_gather_encode(pkg, ora, gpu, p, k, U):
    L, B, pps, pt, H, D = 4, 3, 5, 16, 1, 128
    pool, table = make_pool(gpu, L, B, pps, pt, H, D, torch.bfloat16, seed=p * k + U)
    kv = pkg.paged.PagedKV(pool.to(gpu), table.to(gpu), 0, pps * pt)
    R = pkg.paged.rdp_row_bytes_for(kv, k, p)
    n = (p - 1) * R
    data = [torch.full((n,), 0x77, dtype=torch.uint8, device=gpu) for _ in range(k)]
    P = torch.empty(n, dtype=torch.uint8, device=gpu)
    Q = torch.empty(n, dtype=torch.uint8, device=gpu)
    pkg.paged.rdp_encode_paged(kv, data, P, Q, p, R, unit_bytes=U)
    stream = ora.kv_gather(pool_bytes(pool), table.numpy(), pt, 0, pps * pt).reshape(-1)
    padded = np.zeros(k * n, np.uint8)
    padded[: stream.size] = stream
    want_data = [padded[j * n:(j + 1) * n] for j in range(k)]
    Pw, Qw = ora.rdp_encode(want_data, p, unit=U)
    for j in range(k):
        assert np.array_equal(data[j].cpu().numpy(), want_data[j]), j
    assert np.array_equal(P.cpu().numpy(), Pw)
    assert np.array_equal(Q.cpu().numpy(), Qw)


def test_striped_paged_rejects_unit_off_record(pkg, gpu):
    L, B, pps, pt, H, D = 1, 1, 2, 16, 1, 96      # records of 384 B
    pool, table = make_pool(gpu, L, B, pps, pt, H, D, torch.bfloat16, seed=2)
    kv = pkg.paged.PagedKV(pool.to(gpu), table.to(gpu), 0, pps * pt)
    p, k = 7, 6
    R = pkg.paged.rdp_row_bytes_for(kv, k, p)
    n = (p - 1) * R
    data = [torch.zeros(n, dtype=torch.uint8, device=gpu) for _ in range(k)]
    P, Q = torch.zeros_like(data[0]), torch.zeros_like(data[0])
    with pytest.raises(RuntimeError, match="unit_bytes"):
        pkg.paged.rdp_encode_paged(kv, data, P, Q, p, R, unit_bytes=1024)


def test_striped_encode_in_hip_graph(pkg, ora, gpu):
    """A captured striped encode replays correctly, with eager work between
    replays and fresh data each time."""
    p, k, R, U = 7, 6, 3 * 4096 + 1024, 4096
    d = [torch.empty((p - 1) * R, dtype=torch.uint8, device=gpu) for _ in range(k)]
    P = torch.empty((p - 1) * R, dtype=torch.uint8, device=gpu)
    Q = torch.empty_like(P)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.spec.rdp_encode(d, P, Q, p, unit_bytes=U)     # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        pkg.spec.rdp_encode(d, P, Q, p, unit_bytes=U)
    rng = np.random.default_rng(3)
    for it in range(3):
        host = [rng.integers(0, 256, (p - 1) * R, dtype=np.uint8) for _ in range(k)]
        for t, h in zip(d, host):
            t.copy_(torch.from_numpy(h))
        P.fill_(it)
        g.replay()
        torch.cuda.synchronize()
        Pw, Qw = ora.rdp_encode(host, p, unit=U)
        assert np.array_equal(P.cpu().numpy(), Pw) and np.array_equal(Q.cpu().numpy(), Qw), it


def _garble_shard_in_pool(kv, e, n, seed):
    """Overwrite the pool bytes that data shard e holds (stream bytes
    [e*n, (e+1)*n)) with seeded noise."""
    s = kv.gather()
    lo, hi = e * n, min((e + 1) * n, s.numel())
    if lo < hi:
        g = torch.Generator(device="cpu").manual_seed(seed)
        s[lo:hi] = torch.randint(0, 256, (hi - lo,), generator=g, dtype=torch.uint8).to(s.device)
        kv.scatter(s)


# (p, k, unit, keep_data): the compiled p = 7, k = 6 networks reading the
# survivors from the pool, and the generic map (data buffers kept, other codes)
@pytest.mark.parametrize("p,k,U,keep", [(7, 6, 4096, False), (7, 6, 0, False), (7, 6, 1024, True),
                                        (5, 4, 2048, False), (7, 3, 4096, True)])
def test_paged_decode_restores_pool_every_pattern(pkg, ora, gpu, p, k, U, keep):
    L, B, pps, pt, H, D = 2, 3, 4, 16, 1, 128
    pool, table = make_pool(gpu, L, B, pps, pt, H, D, torch.bfloat16, seed=p + k + U)
    kv = pkg.paged.PagedKV(pool.to(gpu), table.to(gpu), 0, pps * pt)
    R = pkg.paged.rdp_row_bytes_for(kv, k, p)
    n = (p - 1) * R
    data = [torch.empty(n, dtype=torch.uint8, device=gpu) for _ in range(k)]
    P = torch.empty(n, dtype=torch.uint8, device=gpu)
    Q = torch.empty(n, dtype=torch.uint8, device=gpu)
    pkg.paged.rdp_encode_paged(kv, data, P, Q, p, R, unit_bytes=U)
    torch.cuda.synchronize()
    pool0 = kv.pool.clone()
    data0 = [d.clone() for d in data]
    P0, Q0 = P.clone(), Q.clone()
    pats = [(e, -1) for e in range(k + 2)] + list(itertools.combinations(range(k + 2), 2))
    for i, (e0, e1) in enumerate(pats):
        for e in (e0, e1):
            if e < 0:
                continue
            if e < k:
                _garble_shard_in_pool(kv, e, n, seed=i * 10 + e)
                if keep:
                    data[e].fill_(0xA5)
            else:
                (P if e == k else Q).fill_(0x3C)
        pkg.paged.rdp_decode_paged(kv, P, Q, [e0, e1], k, p, R, unit_bytes=U,
                                   data=data if keep else None)
        torch.cuda.synchronize()
        assert torch.equal(kv.pool, pool0), (e0, e1)
        assert torch.equal(P, P0) and torch.equal(Q, Q0), (e0, e1)
        if keep:
            assert all(torch.equal(a, b) for a, b in zip(data, data0)), (e0, e1)


def test_paged_decode_matches_oracle_on_noncodeword(pkg, ora, gpu):
    """On parity that does not match the pool, the rebuilt pool bytes are the
    oracle decode of the gathered stripe (the same fixed map)."""
    p, k, U = 7, 6, 4096
    L, B, pps, pt, H, D = 2, 2, 4, 16, 1, 128
    pool, table = make_pool(gpu, L, B, pps, pt, H, D, torch.bfloat16, seed=77)
    kv = pkg.paged.PagedKV(pool.to(gpu), table.to(gpu), 0, pps * pt)
    R = pkg.paged.rdp_row_bytes_for(kv, k, p)
    n = (p - 1) * R
    rng = np.random.default_rng(8)
    Ph = rng.integers(0, 256, n, dtype=np.uint8)
    Qh = rng.integers(0, 256, n, dtype=np.uint8)
    P, Q = torch.from_numpy(Ph).to(gpu), torch.from_numpy(Qh).to(gpu)
    for e0, e1 in [(1, 4), (0, 6), (2, 7), (5, -1)]:
        stream = kv.gather().cpu().numpy()
        padded = np.zeros(k * n, np.uint8)
        padded[: stream.size] = stream
        cols = [padded[j * n:(j + 1) * n].copy() for j in range(k)] + [P.cpu().numpy(), Q.cpu().numpy()]
        ora.rdp_decode(cols, p, e0, e1, unit=U)
        pkg.paged.rdp_decode_paged(kv, P, Q, [e0, e1], k, p, R, unit_bytes=U)
        torch.cuda.synchronize()
        got = kv.gather().cpu().numpy()
        want = np.concatenate(cols[:k])[: got.size]
        assert np.array_equal(got, want), (e0, e1)
        assert np.array_equal(P.cpu().numpy(), cols[k]) and np.array_equal(Q.cpu().numpy(), cols[k + 1])
