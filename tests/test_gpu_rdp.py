"""spec RDP on the GPU through the C ABI, bit-exact against the oracle."""
import itertools

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _to_dev(arrs, dev):
    return [torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).to(dev) for a in arrs]


def _host(t, shape):
    return t.cpu().numpy().reshape(shape)


@pytest.mark.parametrize("p,k,R", [(7, 6, 4096), (7, 6, 16), (7, 6, 144 * 1024 + 16),
                                   (3, 2, 512), (5, 4, 1024), (5, 2, 2048), (7, 3, 4096),
                                   (11, 10, 1024), (13, 12, 2048), (13, 5, 96)])
def test_rdp_encode_matches_oracle(pkg, ora, gpu, p, k, R):
    rng = np.random.default_rng(p * 1000 + k)
    data = [rng.integers(0, 256, (p - 1, R), dtype=np.uint8) for _ in range(k)]
    Pw, Qw = ora.rdp_encode(data, p)
    d = _to_dev(data, gpu)
    P = torch.full(((p - 1) * R,), 0xAA, dtype=torch.uint8, device=gpu)
    Q = torch.full(((p - 1) * R,), 0x55, dtype=torch.uint8, device=gpu)
    pkg.spec.rdp_encode(d, P, Q, p)
    torch.cuda.synchronize()
    assert np.array_equal(_host(P, (p - 1, R)), Pw)
    assert np.array_equal(_host(Q, (p - 1, R)), Qw)


# (7, 6), (5, 4), (3, 2): compiled networks; the others: the generic kernel of each p
@pytest.mark.parametrize("p,k", [(7, 6), (5, 4), (3, 2), (7, 4), (11, 10), (13, 12), (3, 1), (5, 2)])
def test_rdp_decode_all_patterns(pkg, ora, gpu, p, k):
    R = 1024 + 16
    rng = np.random.default_rng(p + 17 * k)
    data = [rng.integers(0, 256, (p - 1, R), dtype=np.uint8) for _ in range(k)]
    Pw, Qw = ora.rdp_encode(data, p)
    full = data + [Pw, Qw]
    pats = [(e, -1) for e in range(k + 2)] + list(itertools.combinations(range(k + 2), 2))
    for e0, e1 in pats:
        cols = [x.copy() for x in full]
        for e in (e0, e1):
            if e >= 0:
                cols[e][:] = rng.integers(0, 256, cols[e].shape, dtype=np.uint8)
        dev = _to_dev(cols, gpu)
        pkg.spec.rdp_decode(dev, p, [e0, e1])
        torch.cuda.synchronize()
        for s in range(k + 2):
            assert np.array_equal(_host(dev[s], (p - 1, R)), full[s]), (p, k, e0, e1, s)


@pytest.mark.parametrize("p,k", [(7, 6), (11, 7), (5, 3)])   # compiled networks, then the generic kernel
def test_rdp_decode_inconsistent_input_matches_oracle(pkg, ora, gpu, p, k):
    """On input that is not a codeword the decoder is still a fixed function of
    the surviving bytes; the GPU and the oracle pick the same equations."""
    R = 256
    rng = np.random.default_rng(99 + p * k)
    pats = [(2, -1), (k, -1), (k + 1, -1), (0, k + 1), (k, k + 1), (1, k - 1), (0, k)]
    for e0, e1 in pats:
        cols = [rng.integers(0, 256, (p - 1, R), dtype=np.uint8) for _ in range(k + 2)]
        want = [c.copy() for c in cols]
        ora.rdp_decode(want, p, e0, e1)
        dev = _to_dev(cols, gpu)
        pkg.spec.rdp_decode(dev, p, [e0, e1])
        torch.cuda.synchronize()
        for s in range(k + 2):
            assert np.array_equal(_host(dev[s], (p - 1, R)), want[s]), (e0, e1, s)


# ------------------------------------------------------------------ RS GF(2^8)
@pytest.mark.parametrize("k,m,S", [(6, 2, 4096), (5, 3, 1024 + 16), (4, 2, 16), (8, 2, 2048),
                                   (10, 4, 512), (3, 1, 4096), (7, 3, 160), (12, 5, 64)])
def test_rs8_encode_matches_oracle(pkg, ora, gpu, k, m, S):
    assert np.array_equal(pkg.spec.rs8_cauchy(k, m), ora.rs8_cauchy(k, m))
    rng = np.random.default_rng(k * 10 + m)
    data = [rng.integers(0, 256, S, dtype=np.uint8) for _ in range(k)]
    want = ora.rs8_encode(data, m)
    d = _to_dev(data, gpu)
    par = [torch.full((S,), 0x33, dtype=torch.uint8, device=gpu) for _ in range(m)]
    pkg.spec.rs8_encode(d, par)
    torch.cuda.synchronize()
    for i in range(m):
        assert np.array_equal(par[i].cpu().numpy(), want[i]), i


@pytest.mark.parametrize("k,m", [(6, 2), (5, 3), (4, 2), (7, 3), (10, 4)])
def test_rs8_decode_all_patterns(pkg, ora, gpu, k, m):
    S = 2048 + 16
    rng = np.random.default_rng(k * 31 + m)
    data = [rng.integers(0, 256, S, dtype=np.uint8) for _ in range(k)]
    full = data + ora.rs8_encode(data, m)
    pats = [e for n in range(1, m + 1) for e in itertools.combinations(range(k + m), n)]
    if len(pats) > 60:
        pats = [pats[i] for i in rng.choice(len(pats), 60, replace=False)]
    for er in pats:
        sh = [x.copy() for x in full]
        for e in er:
            sh[e][:] = rng.integers(0, 256, S, dtype=np.uint8)
        want = [x.copy() for x in sh]
        ora.rs8_decode(want, k, m, er)
        dev_sh = _to_dev(sh, gpu)
        pkg.spec.rs8_decode(dev_sh, k, er)
        torch.cuda.synchronize()
        for s in range(k + m):
            got = dev_sh[s].cpu().numpy()
            assert np.array_equal(got, want[s]) and np.array_equal(got, full[s]), (er, s)


def test_rdp_flat_addressing_large_shards(pkg, ora, gpu):
    """Shards of 4 GiB or more are addressed with flat 64-bit pointers (the
    buffer-resource kernels reach below 4 GiB): the encode and the compiled
    decode networks at p = 7, k = 6 with row planes of 715,827,904 B, so each
    shard holds 4,294,967,424 B.  P and Q are checked against the oracle on
    sampled stripe columns; decodes are byte-compared at full size."""
    p, k, R = 7, 6, 715_827_904
    nb = (p - 1) * R
    free, _ = torch.cuda.mem_get_info(gpu)
    if free < (k + 4) * nb + (8 << 30):
        pytest.skip(f"needs {((k + 4) * nb) >> 30} GiB of free device memory")
    shards = [torch.empty(nb, dtype=torch.uint8, device=gpu) for _ in range(k + 2)]
    try:
        for t in shards[:k]:
            t.random_(0, 256)
        pkg.spec.rdp_encode(shards[:k], shards[k], shards[k + 1], p=p)
        rng = np.random.default_rng(7)
        offs = np.sort(rng.choice(R // 16, 512, replace=False)) * 16
        lane = (offs[:, None] + np.arange(16)[None, :]).reshape(-1)
        idx = torch.from_numpy((np.arange(p - 1)[:, None] * R + lane[None, :]).reshape(-1)).to(gpu)
        cols = [t[idx].cpu().numpy().reshape(p - 1, -1) for t in shards]
        Pw, Qw = ora.rdp_encode(cols[:k], p)
        assert np.array_equal(cols[k], Pw) and np.array_equal(cols[k + 1], Qw)
        for a, b in [(0, 1), (2, 6), (6, 7), (3, -1)]:
            keep = [shards[e].clone() for e in (a, b) if e >= 0]
            for e in (a, b):
                if e >= 0:
                    shards[e].zero_()
            pkg.spec.rdp_decode(shards, p, [a, b])
            torch.cuda.synchronize()
            for e, want in zip([e for e in (a, b) if e >= 0], keep):
                assert torch.equal(shards[e], want), (a, b, e)
            del keep
    finally:
        del shards
        torch.cuda.empty_cache()
