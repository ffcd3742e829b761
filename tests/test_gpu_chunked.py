"""Chunked coding of a paged fp8 KV cache (RDP p + RS(k, m) on shared data
shards, one chunk at a time) against the oracle's gather + RDP + RS8, and
decode of every erasure class straight back into the pool pages."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def fp8_pool(L, npages, pt, H, D, seed):
    """fp8 e4m3 bytes drawn uniformly, NaN encodings (0x7F, 0xFF) excluded."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 254, (L, npages, pt, 2, H, D), dtype=np.uint8)
    b = b + (b >= 0x7F).astype(np.uint8)  # skip 0x7F; 0xFF is never reached
    return torch.from_numpy(b).view(torch.float8_e4m3fn)


def setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, chunk_tokens, keep_data, seed, unit_bytes=None):
    npages = B * pps + 3
    pool = fp8_pool(L, npages, pt, H, D, seed)
    rng = np.random.default_rng(seed + 1)
    table = torch.from_numpy(rng.permutation(npages)[: B * pps].astype(np.int32).reshape(B, pps))
    n_chunks = pps * pt // chunk_tokens
    pool_d, table_d = pool.to(gpu), table.to(gpu)
    kv0 = pkg.chunked.chunk_kv(pool_d, table_d, 0, chunk_tokens)
    scales = torch.rand(L, dtype=torch.float32, device=gpu)
    st = pkg.chunked.ChunkedStripes(kv0.stream_bytes(), 2 * kv0.token_bytes, n_chunks, gpu,
                                    k=k, p=p, m=m, keep_data=keep_data, scales=scales,
                                    unit_bytes=unit_bytes)
    return pool, table, pool_d, table_d, n_chunks, st


def pool_u8(pool):
    L = pool.shape[0]
    npages, pt = pool.shape[1], pool.shape[2]
    return pool.contiguous().view(torch.uint8).cpu().numpy().reshape(L, npages, pt, 2, -1)


CONFIGS = [
    # L, B, pps, pt, H, D, k, p, m, chunk_tokens
    (2, 3, 4, 16, 1, 128, 5, 7, 3, 16),
    (3, 2, 6, 16, 1, 64, 6, 7, 2, 32),
    (2, 2, 8, 8, 2, 32, 4, 5, 2, 16),
    (1, 1, 4, 4, 1, 16, 2, 3, 1, 4),
]


@pytest.mark.parametrize("cfg", CONFIGS)
@pytest.mark.parametrize("keep_data", [True, False])
def test_chunked_encode_matches_oracle(pkg, ora, gpu, cfg, keep_data):
    L, B, pps, pt, H, D, k, p, m, ct = cfg
    pool, table, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct,
                                                 keep_data, seed=sum(cfg))
    W, data, P, Q, rs = ora.chunked_encode(pool_u8(pool), table.numpy(), pt, ct, nc, k, p, m,
                                           st.unit_bytes)
    assert st.width == W and st.row_bytes == nc * W
    sentinel = 0xA5
    for t in st.shards():
        t.fill_(sentinel)
    for c in range(nc):
        st.encode(pkg.chunked.chunk_kv(pool_d, table_d, c, ct), c)
        torch.cuda.synchronize()
        # chunk c wrote exactly its own region
        later = st.region(c + 1)
        for t in st.shards():
            assert bool((t[later:] == sentinel).all()), f"chunk {c} wrote past its region"
    got = [t.cpu().numpy() for t in st.shards()]
    want = (data if keep_data else []) + [P, Q] + rs
    names = ([f"data{j}" for j in range(k)] if keep_data else []) + ["P", "Q"] + \
        [f"rs{i}" for i in range(m)]
    for n, g_, w_ in zip(names, got, want):
        assert np.array_equal(g_, w_), n
    assert st.scales is not None and st.scales.shape == (L,)


@pytest.mark.parametrize("unit", [1024, 2048, 4096])
def test_chunked_encode_short_last_stripe(pkg, ora, gpu, unit):
    """Rows of 4608 bytes in stripes of `unit` bytes: the last stripe's rows
    (512 bytes at 4096) end before the 1 KiB pieces its unit spans, and the
    pieces past the end must write nothing; two chunks, data kept."""
    cfg = (2, 4, 8, 16, 1, 128, 5, 7, 3, 64)
    L, B, pps, pt, H, D, k, p, m, ct = cfg
    pool, table, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct, True,
                                                 seed=7 + unit, unit_bytes=unit)
    assert st.width == 4608 and st.width % unit != 0 and nc == 2
    W, data, P, Q, rs = ora.chunked_encode(pool_u8(pool), table.numpy(), pt, ct, nc, k, p, m, unit)
    for t in st.shards():
        t.fill_(0xA5)
    for c in range(nc):
        st.encode(pkg.chunked.chunk_kv(pool_d, table_d, c, ct), c)
    torch.cuda.synchronize()
    for n, g_, w_ in zip(range(k + 2 + m), [t.cpu().numpy() for t in st.shards()], data + [P, Q] + rs):
        assert np.array_equal(g_, w_), n


def erase(pkg, st, kv, c, erased, gen):
    """Overwrite chunk c's region of the erased shards: data in the pool pages
    (through the stream and the scatter), parity in its region.  Returns
    whether a pool byte was overwritten (bytes past the stream are padding)."""
    k, nr = st.k, st.region_bytes
    reg = slice(st.region(c), st.region(c) + nr)
    s = kv.gather()
    n = s.numel()
    touched = False
    for e in erased:
        if e < k:
            lo, hi = e * nr, min((e + 1) * nr, n)
            if lo < n:
                touched = True
                s[lo:hi] = torch.randint(0, 256, (hi - lo,), generator=gen,
                                         dtype=torch.uint8).to(s.device)
            if st.data is not None:
                st.data[e][reg] = 0x3C
        else:
            st.shards()[(k if st.data is not None else 0) + e - k][reg] = 0x5A
    kv.scatter(s)
    return touched


PATTERNS = [
    [2], [0, 4], [1, 2, 3], [0, 5], [3, 6], [5, 6], [7], [0, 7, 8],
    [0, 1, 7, 8], [2, 5, 7, 8, 9], [4, 6, 9], [5, 6, 7, 8, 9],
    # the RDP path with every RS parity re-encoded in the same pass
    [1, 3, 7, 8, 9], [0, 7, 8, 9], [3, 6, 7, 8, 9], [0, 4, 7, 9],
]


@pytest.mark.parametrize("keep_data", [True, False])
def test_chunked_decode_restores_pool(pkg, gpu, keep_data):
    L, B, pps, pt, H, D, k, p, m, ct = CONFIGS[0]
    pool, table, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct,
                                                 keep_data, seed=3)
    for c in range(nc):
        st.encode(pkg.chunked.chunk_kv(pool_d, table_d, c, ct), c)
    torch.cuda.synchronize()
    ref_pool = pool_d.clone()
    ref_sh = [t.clone() for t in st.shards()]
    gen = torch.Generator().manual_seed(9)
    for i, er in enumerate(PATTERNS):
        c = i % nc
        kv = pkg.chunked.chunk_kv(pool_d, table_d, c, ct)
        touched = erase(pkg, st, kv, c, er, gen)
        assert touched == (not torch.equal(pool_d.view(torch.uint8), ref_pool.view(torch.uint8)))
        st.decode(kv, c, er)
        torch.cuda.synchronize()
        assert torch.equal(pool_d.view(torch.uint8), ref_pool.view(torch.uint8)), er
        for j, (t, r) in enumerate(zip(st.shards(), ref_sh)):
            assert torch.equal(t, r), (er, j)


@pytest.mark.parametrize("unit", [2048, 4096])
def test_chunked_decode_short_last_stripe(pkg, gpu, unit):
    """Rows of 4608 bytes in stripes of `unit` bytes (the encode test's shape):
    the decode's blocks own one 1 KiB piece of a stripe, and those whose piece
    starts past the short last stripe's end must write nothing, on the RS path
    (one to three lost data shards) and the RDP path (data with RS parity
    lost); the pool and every shard restored."""
    L, B, pps, pt, H, D, k, p, m, ct = (2, 4, 8, 16, 1, 128, 5, 7, 3, 64)
    _, _, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct, True,
                                          seed=11 + unit, unit_bytes=unit)
    assert st.width == 4608 and st.width % unit != 0 and nc == 2
    for c in range(nc):
        st.encode(pkg.chunked.chunk_kv(pool_d, table_d, c, ct), c)
    torch.cuda.synchronize()
    ref_pool = pool_d.clone()
    ref_sh = [t.clone() for t in st.shards()]
    gen = torch.Generator().manual_seed(12)
    for i, er in enumerate([[0], [1, 4], [0, 2, 3], [2, 7], [0, 7, 8], [1, 3, 7, 8, 9]]):
        c = i % nc
        kv = pkg.chunked.chunk_kv(pool_d, table_d, c, ct)
        erase(pkg, st, kv, c, er, gen)
        st.decode(kv, c, er)
        torch.cuda.synchronize()
        assert torch.equal(pool_d.view(torch.uint8), ref_pool.view(torch.uint8)), (unit, er)
        for j, (t, r) in enumerate(zip(st.shards(), ref_sh)):
            assert torch.equal(t, r), (unit, er, j)


def test_chunked_decode_rejects_undecodable(pkg, gpu):
    L, B, pps, pt, H, D, k, p, m, ct = CONFIGS[0]
    _, _, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct, False, seed=4)
    kv = pkg.chunked.chunk_kv(pool_d, table_d, 0, ct)
    st.encode(kv, 0)
    with pytest.raises(pkg._lib.KvecError, match="cannot be decoded"):
        st.decode(kv, 0, [0, 1, 2, 7])  # 3 data, 2 RS parities left, RDP covers 2
    with pytest.raises(pkg._lib.KvecError):
        st.decode(kv, 0, [0, 1, 5, 7, 8, 9])


@pytest.mark.parametrize("cfg", CONFIGS[1:])
def test_chunked_decode_other_shapes(pkg, gpu, cfg):
    L, B, pps, pt, H, D, k, p, m, ct = cfg
    _, _, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct, True,
                                          seed=sum(cfg) + 1)
    for c in range(nc):
        st.encode(pkg.chunked.chunk_kv(pool_d, table_d, c, ct), c)
    torch.cuda.synchronize()
    ref_pool = pool_d.clone()
    ref_sh = [t.clone() for t in st.shards()]
    gen = torch.Generator().manual_seed(10)
    pats = [[0], [k - 1, k], [0, k + 1], [k, k + 1], list(range(min(m, k)))]
    pats += [[0, k + 2], [k + 2]]
    for i, er in enumerate(pats):
        c = i % nc
        kv = pkg.chunked.chunk_kv(pool_d, table_d, c, ct)
        erase(pkg, st, kv, c, er, gen)
        st.decode(kv, c, er)
        torch.cuda.synchronize()
        assert torch.equal(pool_d.view(torch.uint8), ref_pool.view(torch.uint8)), (cfg, er)
        for j, (t, r) in enumerate(zip(st.shards(), ref_sh)):
            assert torch.equal(t, r), (cfg, er, j)


def test_chunked_encode_repeatable_at_scale(pkg, ora, gpu):
    """A 64 MiB fp8 chunk (about 1,100 blocks): encoding it twice gives the same
    bytes, which match the oracle at full size."""
    L, B, pps, pt, H, D, k, p, m, ct = 8, 16, 128, 16, 1, 128, 5, 7, 3, 2048
    pool, table, pool_d, table_d, nc, st = setup(pkg, gpu, L, B, pps, pt, H, D, k, p, m, ct,
                                                 False, seed=21)
    kv = pkg.chunked.chunk_kv(pool_d, table_d, 0, ct)
    st.encode(kv, 0)
    first = [t.clone() for t in st.shards()]
    for _ in range(3):
        st.encode(kv, 0)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(st.shards(), first)):
            assert torch.equal(a, b), f"shard {i} differs between two encodes"
    W, nr = st.width, st.region_bytes
    cells = ora.chunk_cells(kv.gather().cpu().numpy(), k, p, W)
    data = [np.ascontiguousarray(cells[j]) for j in range(k)]
    Pw, Qw = ora.rdp_encode(data, p, st.unit_bytes)
    rsw = ora.rs8_encode(data, m)
    got = [t[:nr].cpu().numpy() for t in st.shards()]
    assert np.array_equal(got[0], Pw) and np.array_equal(got[1], Qw)
    for i in range(m):
        assert np.array_equal(got[2 + i], rsw[i]), i
