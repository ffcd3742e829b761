"""Seeded random sweeps of the gs kernels against the oracle: row counts,
row lengths (and so row misalignments), star bases and buffer offsets that
the hand-picked cases do not reach.  The draws are fixed by the seed, so the
cases are the same on every run."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

_R = np.random.default_rng(20260)


def _draw(n, f):
    return [f(i) for i in range(n)]


PQ = _draw(24, lambda i: (int(_R.integers(1, 41)), int(_R.integers(1, 9000)),
                          int(_R.choice([0, 1, 7, -1, -40, 10 ** 7, int(_R.integers(-100, 100))]))))
BACKUP = _draw(16, lambda i: (int(_R.integers(1, 300)), int(_R.integers(1, 200)), int(_R.integers(1, 20)),
                              int(_R.integers(-5, 40)), int(_R.integers(0, 8)), bool(_R.integers(0, 2)),
                              int(_R.integers(-3, 30))))
XOR = _draw(16, lambda i: (int(_R.integers(1, 12)), int(_R.integers(1, 20000)), int(_R.integers(0, 16)),
                           int(_R.integers(0, 16))))
RS16 = _draw(16, lambda i: (int(_R.integers(1, 9)), int(_R.integers(1, 6)), int(_R.integers(1, 9000)),
                            int(_R.integers(0, 8)), int(_R.integers(0, 8))))


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


@pytest.mark.parametrize("nd,S,sb", PQ)
def test_sweep_gs_parity(pkg, ora, gpu, nd, S, sb):
    rng = np.random.default_rng(nd * 10007 + S)
    rows = rng.integers(0, 65536, (nd + 2, S), dtype=np.uint16)
    want = rows.copy()
    ora.gs_parity(want, nd, S, sb)
    d = dev(rows, gpu)
    pkg.rdp_kv_ops.compute_rdp_parity(d, nd, S, sb)
    assert np.array_equal(d.cpu().numpy(), want)


@pytest.mark.parametrize("T,n,nd,S_extra,soff,fuse,sb", BACKUP)
def test_sweep_gs_backup(pkg, ora, gpu, T, n, nd, S_extra, soff, fuse, sb):
    tn = T * n
    S = max(1, -(-2 * tn // nd) + S_extra)
    koff = soff if fuse else (soff + 1) % 8
    voff = (soff + tn) % 8 if fuse else (soff + tn + 3) % 8
    rng = np.random.default_rng(T * 7 + n * 13 + nd)
    K = rng.integers(0, 65536, tn, dtype=np.uint16)
    V = rng.integers(0, 65536, tn, dtype=np.uint16)
    init = rng.integers(0, 65536, (nd + 2, S), dtype=np.uint16)
    want = init.copy()
    ora.gs_pack(K.reshape(T, n), V.reshape(T, n), want, nd, S, T, n)
    ora.gs_parity(want, nd, S, sb)
    kb = torch.zeros(tn + 16, dtype=torch.int16, device=gpu)
    vb = torch.zeros(tn + 16, dtype=torch.int16, device=gpu)
    kb[koff:koff + tn] = dev(K.view(np.int16), gpu)
    vb[voff:voff + tn] = dev(V.view(np.int16), gpu)
    sbuf = torch.full(((nd + 2) * S + 16,), 0x5A5A, dtype=torch.int16, device=gpu)
    sbuf[soff:soff + (nd + 2) * S] = dev(init.reshape(-1).view(np.int16), gpu)
    sh = sbuf[soff:soff + (nd + 2) * S].view(nd + 2, S)
    pkg.rdp.rdp_kernel.fused_backup_full_kv(kb[koff:koff + tn].view(T, n), vb[voff:voff + tn].view(T, n),
                                            sh, nd, S, T, n, sb)
    assert np.array_equal(sh.cpu().numpy().view(np.uint16), want)
    assert bool((torch.cat([sbuf[:soff], sbuf[soff + (nd + 2) * S:]]) == 0x5A5A).all())


@pytest.mark.parametrize("nd,S,doff,soff", XOR)
def test_sweep_xor_encode(pkg, ora, gpu, nd, S, doff, soff):
    rng = np.random.default_rng(nd * 31 + S)
    data = rng.integers(0, 256, nd * S, dtype=np.uint8)
    want = ora.xor_encode(data, nd, S)
    dbuf = torch.zeros(nd * S + 16, dtype=torch.uint8, device=gpu)
    dbuf[doff:doff + nd * S] = dev(data, gpu)
    sbuf = torch.full(((nd + 1) * S + 16,), 0x77, dtype=torch.uint8, device=gpu)
    sh = sbuf[soff:soff + (nd + 1) * S].view(nd + 1, S)
    pkg.xor.xor_kernel.encode_xor(dbuf[doff:doff + nd * S], sh, nd, S)
    assert np.array_equal(sh.cpu().numpy(), want)
    assert bool((torch.cat([sbuf[:soff], sbuf[soff + (nd + 1) * S:]]) == 0x77).all())


@pytest.mark.parametrize("k,m,S,doff,soff", RS16)
def test_sweep_rs16_encode(pkg, ora, gpu, k, m, S, doff, soff):
    ex, lg = ora.gf16_tables()
    rng = np.random.default_rng(k * 101 + m * 7 + S)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    want = ora.rs16_encode(data, k, m, S, ex, lg)
    dbuf = torch.zeros(k * S + 8, dtype=torch.int16, device=gpu)
    dbuf[doff:doff + k * S] = dev(data.view(np.int16), gpu)
    sbuf = torch.full(((k + m) * S + 8,), 0x2468, dtype=torch.int16, device=gpu)
    sh = sbuf[soff:soff + (k + m) * S].view(k + m, S)
    gex, glg = pkg.rs.device_gf_tables(gpu)
    pkg.rs.rs_kernel.encode_rs_u16(dbuf[doff:doff + k * S].view(torch.uint16), sh.view(torch.uint16),
                                   k, m, S, gex, glg)
    assert np.array_equal(sh.cpu().numpy().view(np.uint16), want)
    assert bool((torch.cat([sbuf[:soff], sbuf[soff + (k + m) * S:]]) == 0x2468).all())


# ------------------------------------------------------------------ spec codes
RDP = _draw(20, lambda i: (lambda p: (p, int(_R.integers(1, p)), 16 * int(_R.integers(1, 3000)),
                                      sorted(_R.choice(int(_R.integers(1, p)) + 2, 2, replace=False).tolist())))(
    int(_R.choice([3, 5, 7, 11, 13]))))
RS8 = _draw(16, lambda i: (lambda k: (k, int(_R.integers(1, min(8, 64 // k) + 1)), 16 * int(_R.integers(1, 4000))))(
    int(_R.integers(1, 33))))


@pytest.mark.parametrize("p,k,R,er", RDP)
def test_sweep_rdp_encode_decode(pkg, ora, gpu, p, k, R, er):
    er = [e for e in er if e < k + 2]
    rng = np.random.default_rng(p * 1000 + k * 10 + R)
    data = [rng.integers(0, 256, (p - 1, R), dtype=np.uint8) for _ in range(k)]
    P, Q = ora.rdp_encode(data, p)
    d = [dev(x.reshape(-1), gpu) for x in data]
    Pg = torch.empty_like(d[0])
    Qg = torch.empty_like(d[0])
    pkg.spec.rdp_encode(d, Pg, Qg, p)
    assert np.array_equal(Pg.cpu().numpy().reshape(p - 1, R), P)
    assert np.array_equal(Qg.cpu().numpy().reshape(p - 1, R), Q)
    sh = d + [Pg, Qg]
    want = [t.clone() for t in sh]
    for e in er:
        sh[e].fill_(0xEE)
    pkg.spec.rdp_decode(sh, p, er)
    for a, b in zip(sh, want):
        assert torch.equal(a, b)


@pytest.mark.parametrize("k,m,S", RS8)
def test_sweep_rs8_encode_decode(pkg, ora, gpu, k, m, S):
    rng = np.random.default_rng(k * 100 + m + S)
    data = [rng.integers(0, 256, S, dtype=np.uint8) for _ in range(k)]
    par = ora.rs8_encode(data, m)
    d = [dev(x, gpu) for x in data]
    pg = [torch.empty_like(d[0]) for _ in range(m)]
    pkg.spec.rs8_encode(d, pg)
    for a, b in zip(pg, par):
        assert np.array_equal(a.cpu().numpy(), b)
    sh = d + pg
    want = [t.clone() for t in sh]
    ne = int(rng.integers(1, m + 1))
    er = sorted(rng.choice(k + m, ne, replace=False).tolist())
    for e in er:
        sh[e].fill_(0x11)
    pkg.spec.rs8_decode(sh, k, er)
    for a, b in zip(sh, want):
        assert torch.equal(a, b)


# ------------------------------------------------------------------ gs RS16 reconstruct
# Its own generator, so the draws above stay as they were.  k up to 10 and up
# to 2 lost rows reach both the piece kernel (k <= 8, m <= 2) and the tile
# kernel; any row length and tensor offset; erased rows and parity choices
# drawn per case.
_R2 = np.random.default_rng(20261)


def _rs16_rec_case(i):
    k = int(_R2.integers(1, 11))
    mp = int(_R2.integers(1, 6))
    nm = int(_R2.integers(1, min(k, mp, 3) + 1))
    miss = sorted(_R2.choice(k, nm, replace=False).tolist())
    pused = sorted(_R2.choice(mp, nm, replace=False).tolist())
    return (k, mp, int(_R2.integers(1, 20000)), int(_R2.integers(0, 8)), miss, pused)


RS16REC = [_rs16_rec_case(i) for i in range(20)]


@pytest.mark.parametrize("k,mp,S,soff,miss,pused", RS16REC)
def test_sweep_rs16_reconstruct(pkg, ora, gpu, k, mp, S, soff, miss, pused):
    ex, lg = ora.gf16_tables()
    rng = np.random.default_rng(k * 131 + mp * 17 + S)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    ref = ora.rs16_encode(data, k, mp, S, ex, lg)
    sh = ref.copy()
    sh[miss] = rng.integers(0, 65536, (len(miss), S), dtype=np.uint16)
    # the oracle's rebuild (the original rows unless the reference's system is
    # singular for these parity rows, where its Gauss-Jordan gives other bytes)
    want = sh.copy()
    ora.rs16_reconstruct(want, S, k, mp, list(miss), list(pused), ex, lg)
    buf = torch.full(((k + mp) * S + 8,), 0x1B1B, dtype=torch.int16, device=gpu)
    buf[soff:soff + (k + mp) * S] = dev(sh.reshape(-1).view(np.int16), gpu)
    d = buf[soff:soff + (k + mp) * S].view(k + mp, S).view(torch.uint16)
    gex, glg = pkg.rs.device_gf_tables(gpu)
    pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(
        d, S, k, mp, torch.tensor(miss, dtype=torch.int32, device=gpu),
        torch.tensor(pused, dtype=torch.int32, device=gpu), gex, glg)
    assert np.array_equal(d.cpu().numpy(), want)
    assert bool((torch.cat([buf[:soff], buf[soff + (k + mp) * S:]]) == 0x1B1B).all())
