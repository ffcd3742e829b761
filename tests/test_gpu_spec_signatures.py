"""The spec codes behind the reference's own signatures: rdp.fused_backup_full_kv
/ fused_recovery_full_kv (benchmark/rdp/main.py:44-126) and rs.forward_encode_kv
/ backwards_decode_kv (benchmark/rs/main.py:63-206) with scheme="spec".  Lost
rows are really zeroed, every erasure pattern the code covers is recovered
byte-exact, and the parity rows equal the oracle's textbook RDP / GF(2^8) RS
of the packed data rows."""
import itertools

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _kv(B, H, T, D, dtype, seed, gpu):
    g = torch.Generator(device="cpu").manual_seed(seed)
    k = torch.randn(B, H, T, D, generator=g).to(dtype)
    v = torch.randn(B, H, T, D, generator=g).to(dtype)
    return k.to(gpu), v.to(gpu)


def _rows(shards):
    return [r.cpu().numpy() for r in shards.view(torch.uint8).view(shards.shape[0], -1)]


# (B, H, T, D, nd): the reference demo's shape (1 x 8 heads x 512 x 128, 8 data
# shards -> p = 11), six shards (p = 7), an odd small shape (p = 5)
@pytest.mark.parametrize("B,H,T,D,nd", [(1, 8, 512, 128, 8), (1, 2, 300, 128, 6), (2, 1, 7, 5, 4)])
def test_rdp_spec_scheme_recovers_every_pair(pkg, ora, gpu, B, H, T, D, nd):
    rdp = pkg.rdp
    k, v = _kv(B, H, T, D, torch.bfloat16, B * T + nd, gpu)
    pkg_ = rdp.fused_backup_full_kv(k, v, nd, scheme="spec")
    p = pkg_["p"]
    assert p == rdp.spec_prime(nd) and p - 1 >= nd
    sh = pkg_["shards_KV"]
    S = pkg_["shard_size"]
    assert sh.shape == (nd + 2, S) and (2 * S) % (16 * (p - 1)) == 0
    assert pkg_["pad_words"] == nd * S - 2 * T * B * H * D
    rows = _rows(sh)
    Pw, Qw = ora.rdp_encode(rows[:nd], p, unit=pkg.spec.RDP_UNIT)
    assert np.array_equal(rows[nd], Pw) and np.array_equal(rows[nd + 1], Qw)
    full = sh.clone()
    pats = [(a, -1) for a in range(nd + 2)] + list(itertools.combinations(range(nd + 2), 2))
    for a, b in pats:
        for e in (a, b):
            if e >= 0:
                sh[e].zero_()
        k2, v2, stats = rdp.fused_recovery_full_kv(pkg_, a, b)
        assert torch.equal(sh, full), (a, b)
        assert torch.equal(k2, k) and torch.equal(v2, v), (a, b)
        assert stats["recover_ms"] >= 0


def test_rdp_ghostserve_scheme_unchanged(pkg, gpu):
    """The default scheme still returns the reference's star-diagonal code."""
    k, v = _kv(1, 2, 64, 16, torch.float16, 3, gpu)
    a = pkg.rdp.fused_backup_full_kv(k, v, 6)
    assert a["scheme"] == "ghostserve" and a["shard_size"] == -(-2 * 64 * 32 // 6)
    with pytest.raises(ValueError, match="scheme"):
        pkg.rdp.fused_backup_full_kv(k, v, 6, scheme="textbook")


@pytest.mark.parametrize("nd,npar", [(6, 2), (5, 3), (4, 1)])
def test_rs_spec_scheme_recovers_every_pattern(pkg, ora, gpu, nd, npar):
    rs = pkg.rs
    k, v = _kv(1, 1, 333, 128, torch.float16, nd * 10 + npar, gpu)
    shards, meta = rs.forward_encode_kv(k, v, nd, npar, scheme="spec")
    assert meta["scheme"] == "spec" and meta["shard_sz"] % 8 == 0
    rows = _rows(shards)
    par = ora.rs8_encode(rows[:nd], npar)
    for i in range(npar):
        assert np.array_equal(rows[nd + i], par[i]), i
    full = shards.clone()
    pats = [e for n_ in range(1, npar + 1) for e in itertools.combinations(range(nd + npar), n_)]
    for er in pats:
        for e in er:
            shards[e].zero_()
        K, V = rs.backwards_decode_kv(shards, meta, list(er))
        assert torch.equal(shards, full), er
        assert torch.equal(K, k) and torch.equal(V, v), er
    with pytest.raises(RuntimeError, match="Not enough parity"):
        rs.backwards_decode_kv(shards, meta, list(range(npar + 1)))
