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


@pytest.mark.parametrize("p,k", [(7, 6), (5, 4), (3, 2), (7, 4), (11, 10), (13, 12)])
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


def test_rdp_decode_inconsistent_input_matches_oracle(pkg, ora, gpu):
    """On input that is not a codeword the decoder is still a fixed function of
    the surviving bytes; the GPU and the oracle pick the same equations."""
    p, k, R = 7, 6, 256
    rng = np.random.default_rng(99)
    for e0, e1 in [(2, -1), (6, -1), (7, -1), (0, 7), (6, 7), (1, 4), (3, 6)]:
        cols = [rng.integers(0, 256, (p - 1, R), dtype=np.uint8) for _ in range(k + 2)]
        want = [c.copy() for c in cols]
        ora.rdp_decode(want, p, e0, e1)
        dev = _to_dev(cols, gpu)
        pkg.spec.rdp_decode(dev, p, [e0, e1])
        torch.cuda.synchronize()
        for s in range(k + 2):
            assert np.array_equal(_host(dev[s], (p - 1, R)), want[s]), (e0, e1, s)
