"""Pins the CPU oracle (oracle/kvec_oracle.c) to mathematics.

The reference ships no tests, golden vectors or CPU implementation, so each
oracle function is fixed here by a check that does not retype its formula:

  GF(2^16) tables      carry-less multiply mod 0x1100B on random pairs; the
                       exp walk is a permutation of the 65535 units; alpha^16
  GF(2^8) tables       all 65536 products vs carry-less multiply mod 0x11D;
                       published alpha^8..alpha^15 values of this field
  Cauchy block         C[i][j] * ((k+i) ^ j) == 1; every k x k submatrix of
                       [I; C] has full rank (MDS)
  RS8 encode           matrix-vector product through the brute-force table
  RS8 decode           round trip for every erasure pattern of <= m shards
  RDP encode (spec)    hand-derived single-cell answers; the row and diagonal
                       equations of the code hold; linearity
  RDP decode (spec)    round trip for every pair of the k+2 shards; GF(2) rank
                       of every 2-column erasure system is full (p=3,5,7)
  XOR encode/recon     XOR of all shards is 0; k=1 gives P == D; round trip;
                       no-op for 0 or 2 missing indices
  gs RDP parity        P ^ all rows == 0; single-word answers for the diagonal
                       shift and the star skip (hand-derived); nd=1 closed form
  gs RDP recover       unerased input comes back unchanged (the reference
                       benchmark's own scenario); zeroed rows give the closed
                       form a = a ^ b, b = 0; single erasure round trip
  gs pack / load_full  identity on the token-major stream
  RS16 encode          single nonzero symbol x at shard i gives
                       Par_p = x * alpha^((p+1) i) (carry-less arithmetic)
  RS16 reconstruct     round trip for every erasure set of <= m data shards
  paged gather         numpy fancy indexing of the pool, pool[slots, kv]
"""
import itertools

import numpy as np
import pytest

import gfref


@pytest.fixture(scope="module")
def M8():
    return gfref.gf8_mul_table()


# ------------------------------------------------------------------ fields
def test_gf16_tables(ora):
    ex, lg = ora.gf16_tables()
    assert ex.shape == (131070,) and lg.shape == (65536,)
    units = ex[:65535].astype(np.int64)
    assert np.array_equal(np.sort(units), np.arange(1, 65536)), "alpha not primitive"
    assert np.array_equal(ex[65535:], ex[:65535])
    assert np.array_equal(lg[ex[:65535]], np.arange(65535, dtype=np.uint16))
    assert int(ex[16]) == 0x100B  # x^16 = x^12 + x^3 + x + 1
    rng = np.random.default_rng(1)
    a = rng.integers(1, 65536, 20000, dtype=np.int64)
    b = rng.integers(1, 65536, 20000, dtype=np.int64)
    via_tables = ex[(lg[a].astype(np.int64) + lg[b].astype(np.int64)) % 65535]
    assert np.array_equal(via_tables, gfref.gf16_mul(a, b))


def test_gf8_tables(ora, M8):
    ex, lg = ora.gf8_tables()
    assert list(ex[8:16]) == [0x1D, 0x3A, 0x74, 0xE8, 0xCD, 0x87, 0x13, 0x26]
    assert np.array_equal(np.sort(ex[:255].astype(int)), np.arange(1, 256))
    for a in range(256):
        for b in (0, 1, 2, 0x53, 0x8E, 0xFF, a):
            assert ora.gf8_mul(a, b) == M8[a, b]
    assert ora.gf8_inv(2) == 0x8E
    for a in range(1, 256):
        assert M8[a, ora.gf8_inv(a)] == 1


def test_gf8_all_products(ora, M8):
    ex, lg = ora.gf8_tables()
    a = np.arange(1, 256)[:, None]
    b = np.arange(1, 256)[None, :]
    via = ex[lg[a].astype(int) + lg[b].astype(int)]
    assert np.array_equal(via, M8[1:, 1:])


@pytest.mark.parametrize("k,m", [(6, 2), (5, 3), (4, 4), (10, 4)])
def test_cauchy_mds(ora, M8, k, m):
    C = ora.rs8_cauchy(k, m)
    for i in range(m):
        for j in range(k):
            assert M8[C[i, j], (k + i) ^ j] == 1
    G = np.vstack([np.eye(k, dtype=np.uint8), C])
    for rows in itertools.combinations(range(k + m), k):
        assert gfref.gf8_rank(M8, G[list(rows)]) == k


# ------------------------------------------------------------------ RS8
@pytest.mark.parametrize("k,m", [(6, 2), (5, 3)])
def test_rs8_encode_matches_matvec(ora, M8, k, m):
    rng = np.random.default_rng(k * 10 + m)
    S = 1000
    data = [rng.integers(0, 256, S, dtype=np.uint8) for _ in range(k)]
    par = ora.rs8_encode(data, m)
    C = ora.rs8_cauchy(k, m)
    for i in range(m):
        want = np.zeros(S, np.uint8)
        for j in range(k):
            want ^= M8[C[i, j]][data[j]]
        assert np.array_equal(par[i], want)


@pytest.mark.parametrize("k,m", [(6, 2), (5, 3), (3, 1)])
def test_rs8_decode_all_patterns(ora, k, m):
    rng = np.random.default_rng(7)
    S = 513
    data = [rng.integers(0, 256, S, dtype=np.uint8) for _ in range(k)]
    par = ora.rs8_encode(data, m)
    full = data + par
    for ne in range(1, m + 1):
        for er in itertools.combinations(range(k + m), ne):
            sh = [x.copy() for x in full]
            for e in er:
                sh[e][:] = rng.integers(0, 256, S, dtype=np.uint8)
            ora.rs8_decode(sh, k, m, er)
            for s in range(k + m):
                assert np.array_equal(sh[s], full[s]), (er, s)
    with pytest.raises(ValueError):
        ora.rs8_decode([x.copy() for x in full], k, m, list(range(m + 1)))


# ------------------------------------------------------------------ spec RDP
def _rdp_rand(p, k, R, seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, 256, (p - 1, R), dtype=np.uint8) for _ in range(k)]


def test_rdp_single_cell_answers(ora):
    # p = 5, cell (row 2, column 1) set: P[2] = 1; diagonal (2+1)%5 = 3 gets it
    # from the data cell and diagonal (2+4)%5 = 1 gets it from P[2].
    p, k, R = 5, 4, 1
    data = [np.zeros((p - 1, R), np.uint8) for _ in range(k)]
    data[1][2, 0] = 1
    P, Q = ora.rdp_encode(data, p)
    assert P[:, 0].tolist() == [0, 0, 1, 0]
    assert Q[:, 0].tolist() == [0, 1, 0, 1]
    # cell (row 0, column 3): diagonal 3 from data; P[0] lies on diagonal 4,
    # which is the unstored one.
    data[1][2, 0] = 0
    data[3][0, 0] = 0x80
    P, Q = ora.rdp_encode(data, p)
    assert P[:, 0].tolist() == [0x80, 0, 0, 0]
    assert Q[:, 0].tolist() == [0, 0, 0, 0x80]
    # cell (row 3, column 1): diagonal 4 is unstored; P[3] lies on diagonal 2.
    data[3][0, 0] = 0
    data[1][3, 0] = 0x11
    P, Q = ora.rdp_encode(data, p)
    assert P[:, 0].tolist() == [0, 0, 0, 0x11]
    assert Q[:, 0].tolist() == [0, 0, 0x11, 0]


@pytest.mark.parametrize("p,k", [(3, 2), (5, 4), (7, 6), (7, 4), (11, 10), (13, 7)])
def test_rdp_equations_hold(ora, p, k):
    R = 97
    data = _rdp_rand(p, k, R, p * 100 + k)
    P, Q = ora.rdp_encode(data, p)
    cols = [data[j] if j < k else np.zeros((p - 1, R), np.uint8) for j in range(p - 1)] + [P]
    for r in range(p - 1):
        acc = np.zeros(R, np.uint8)
        for c in range(p):
            acc ^= cols[c][r]
        assert not acc.any()
    for d in range(p - 1):
        acc = Q[d].copy()
        for c in range(p):
            r = (d - c) % p
            if r < p - 1:
                acc ^= cols[c][r]
        assert not acc.any(), d


def _stripe_rows(buf, p, R, U, s):
    """Rows of stripe s of a striped shard, located by the geometry's
    definition (row r at s*(p-1)*U + r*g_s, g_s = min(U, R - s*U))."""
    g = min(U, R - s * U)
    base = s * (p - 1) * U
    return [buf[base + r * g: base + (r + 1) * g] for r in range(p - 1)]


@pytest.mark.parametrize("p,k,R,U", [(7, 6, 3 * 64 + 48, 64), (5, 4, 96, 32), (7, 3, 80, 16),
                                     (3, 2, 50, 16), (11, 10, 40, 16)])
def test_rdp_striped_equations_hold(ora, p, k, R, U):
    """Every stripe of the striped layout satisfies the row and diagonal
    equations on its own rows (the last stripe's rows are shorter), and every
    byte of the shards belongs to exactly one stripe row."""
    rng = np.random.default_rng(R + U)
    data = [rng.integers(0, 256, (p - 1) * R, dtype=np.uint8) for _ in range(k)]
    P, Q = ora.rdp_encode(data, p, unit=U)
    ns = -(-R // U)
    seen = np.zeros((p - 1) * R, np.int32)
    for s in range(ns):
        g = min(U, R - s * U)
        base = s * (p - 1) * U
        seen[base: base + (p - 1) * g] += 1
        cols = [_stripe_rows(data[j], p, R, U, s) if j < k else [np.zeros(g, np.uint8)] * (p - 1)
                for j in range(p - 1)] + [_stripe_rows(P, p, R, U, s)]
        Qs = _stripe_rows(Q, p, R, U, s)
        for r in range(p - 1):
            acc = np.zeros(g, np.uint8)
            for c in range(p):
                acc ^= cols[c][r]
            assert not acc.any(), (s, r)
        for d in range(p - 1):
            acc = Qs[d].copy()
            for c in range(p):
                r = (d - c) % p
                if r < p - 1:
                    acc ^= cols[c][r]
            assert not acc.any(), (s, d)
    assert (seen == 1).all()


def test_rdp_striped_planted_byte(ora):
    """A single data byte at row 1, offset 5 of stripe 2 (p = 5, U = 16,
    R = 40: stripes of rows 16, 16, 8) lands in P at the same place and in Q on
    diagonal (1 + column) mod 5, nowhere else."""
    p, k, R, U = 5, 4, 40, 16
    data = [np.zeros((p - 1) * R, np.uint8) for _ in range(k)]
    s, r, o, j = 2, 1, 5, 2
    g = min(U, R - s * U)                     # 8
    pos = s * (p - 1) * U + r * g + o         # 128 + 8 + 5
    data[j][pos] = 0x5A
    P, Q = ora.rdp_encode(data, p, unit=U)
    assert P.nonzero()[0].tolist() == [pos] and P[pos] == 0x5A
    d_data = (r + j) % p                      # 3
    d_p = (r + p - 1) % p                     # the P cell's diagonal: 0
    want = sorted(s * (p - 1) * U + d * g + o for d in (d_data, d_p) if d < p - 1)
    assert Q.nonzero()[0].tolist() == want
    assert all(Q[x] == 0x5A for x in want)
    # unit 0 and unit >= R are the single-stripe layout
    Pa, Qa = ora.rdp_encode(data, p, unit=0)
    Pb, Qb = ora.rdp_encode(data, p, unit=4 * R)
    assert np.array_equal(Pa, Pb) and np.array_equal(Qa, Qb)
    assert not np.array_equal(Qa, Q)


@pytest.mark.parametrize("p,k,U", [(7, 6, 16), (5, 2, 32), (11, 10, 16)])
def test_rdp_striped_decode_all_pairs(ora, p, k, U):
    R = 3 * U + 16
    rng = np.random.default_rng(p * k)
    data = [rng.integers(0, 256, (p - 1) * R, dtype=np.uint8) for _ in range(k)]
    P, Q = ora.rdp_encode(data, p, unit=U)
    full = data + [P, Q]
    pats = [(e, -1) for e in range(k + 2)] + list(itertools.combinations(range(k + 2), 2))
    for e0, e1 in pats:
        cols = [x.copy() for x in full]
        for e in (e0, e1):
            if e >= 0:
                cols[e][:] = rng.integers(0, 256, cols[e].shape, dtype=np.uint8)
        ora.rdp_decode(cols, p, e0, e1, unit=U)
        for s in range(k + 2):
            assert np.array_equal(cols[s], full[s]), (e0, e1, s)


def test_rdp_linearity(ora):
    p, k, R = 7, 6, 64
    a = _rdp_rand(p, k, R, 1)
    b = _rdp_rand(p, k, R, 2)
    Pa, Qa = ora.rdp_encode(a, p)
    Pb, Qb = ora.rdp_encode(b, p)
    Pab, Qab = ora.rdp_encode([x ^ y for x, y in zip(a, b)], p)
    assert np.array_equal(Pab, Pa ^ Pb) and np.array_equal(Qab, Qa ^ Qb)


@pytest.mark.parametrize("p,k", [(3, 2), (5, 4), (5, 2), (7, 6), (7, 3), (11, 10)])
def test_rdp_decode_all_pairs(ora, p, k):
    R = 33
    data = _rdp_rand(p, k, R, 5 + p + k)
    P, Q = ora.rdp_encode(data, p)
    full = data + [P, Q]
    rng = np.random.default_rng(p)
    pats = [(e, -1) for e in range(k + 2)] + list(itertools.combinations(range(k + 2), 2))
    for e0, e1 in pats:
        cols = [x.copy() for x in full]
        for e in (e0, e1):
            if e >= 0:
                cols[e][:] = rng.integers(0, 256, cols[e].shape, dtype=np.uint8)
        ora.rdp_decode(cols, p, e0, e1)
        for s in range(k + 2):
            assert np.array_equal(cols[s], full[s]), (p, k, e0, e1, s)


@pytest.mark.parametrize("p", [3, 5, 7])
def test_rdp_two_column_systems_full_rank(p):
    """Every 2-column erasure leaves a GF(2) system of full rank.  Written from
    the code's definition as bit rows, independent of the oracle."""
    rows = p - 1
    ncell = (p + 1) * rows  # columns 0..p-1 (data + P) and Q

    def idx(c, r):
        return c * rows + r

    eqs = []
    for r in range(rows):
        eqs.append(sum(1 << idx(c, r) for c in range(p)))
    for d in range(rows):
        v = 1 << idx(p, d)
        for c in range(p):
            r = (d - c) % p
            if r < rows:
                v |= 1 << idx(c, r)
        eqs.append(v)
    for x, y in itertools.combinations(range(p + 1), 2):
        mask = sum(1 << idx(c, r) for c in (x, y) for r in range(rows))
        assert gfref.gf2_rank([e & mask for e in eqs]) == 2 * rows, (x, y)


# ------------------------------------------------------------------ gs XOR
def test_xor_encode_invariants(ora):
    rng = np.random.default_rng(3)
    for nd, S in [(4, 1000), (1, 17), (3, 5)]:
        data = rng.integers(0, 256, nd * S, dtype=np.uint8)
        sh = ora.xor_encode(data, nd, S)
        assert np.array_equal(sh[:nd].reshape(-1), data)
        assert not np.bitwise_xor.reduce(sh, axis=0).any()
        if nd == 1:
            assert np.array_equal(sh[1], sh[0])


def test_xor_reconstruct_round_trip(ora):
    rng = np.random.default_rng(4)
    nd, S = 4, 999
    data = rng.integers(0, 256, nd * S, dtype=np.uint8)
    ref = ora.xor_encode(data, nd, S)
    for miss in range(nd + 1):
        sh = ref.copy()
        sh[miss] = 0
        rec = ora.xor_reconstruct(sh, S, nd, [miss])
        assert np.array_equal(sh, ref) and np.array_equal(rec[0], ref[miss])
    for missing in ([], [0, 1], [nd + 1], [-1]):
        sh = ref.copy()
        sh[0] = 0
        ora.xor_reconstruct(sh, S, nd, missing)
        assert not sh[0].any() and np.array_equal(sh[1:], ref[1:])


def test_pack_unpack_kv_identity(ora):
    rng = np.random.default_rng(5)
    n, T = 24, 7
    k = rng.integers(0, 65536, n * T, dtype=np.uint16)
    v = rng.integers(0, 65536, n * T, dtype=np.uint16)
    b = ora.pack_kv(k, v, n, T)
    assert np.array_equal(b, np.concatenate([k, v]).astype("<u2").view(np.uint8))
    assert np.array_equal(ora.unpack_kv(b, n, T), np.concatenate([k, v]))


# ------------------------------------------------------------------ gs RDP
def _gs_rows(nd, S, seed):
    rng = np.random.default_rng(seed)
    sh = np.zeros((nd + 2, S), np.uint16)
    sh[:nd] = rng.integers(0, 65536, (nd, S), dtype=np.uint16)
    return sh


def test_gs_parity_row_invariant(ora):
    for nd, S in [(6, 101), (8, 64), (1, 9), (3, 2)]:
        sh = _gs_rows(nd, S, nd + S)
        ora.gs_parity(sh, nd, S, 0)
        assert not np.bitwise_xor.reduce(sh[: nd + 1], axis=0).any()


def test_gs_parity_single_word_answers(ora):
    # nd=3, S=7, star_base=0: row r skips column r.  A word at (row 2, col 5)
    # lands on diagonal (5 + 2) % 7 = 0.
    nd, S = 3, 7
    sh = np.zeros((nd + 2, S), np.uint16)
    sh[2, 5] = 0xBEEF
    ora.gs_parity(sh, nd, S, 0)
    assert sh[3].tolist() == [0, 0, 0, 0, 0, 0xBEEF, 0]
    assert sh[4].tolist() == [0xBEEF, 0, 0, 0, 0, 0, 0]
    # the star column of row 2 is column 2: its word reaches P but not Q
    sh[:] = 0
    sh[2, 2] = 0x1234
    ora.gs_parity(sh, nd, S, 0)
    assert sh[3, 2] == 0x1234 and not sh[4].any()
    # star_base=4: row 1 skips column 5; row 1 col 6 goes to diagonal 0
    sh[:] = 0
    sh[1, 5] = 7
    sh[1, 6] = 9
    ora.gs_parity(sh, nd, S, 4)
    assert sh[4].tolist() == [9, 0, 0, 0, 0, 0, 0]
    # a negative remainder never matches a column: nothing is skipped
    sh[:] = 0
    sh[0, 3] = 5
    ora.gs_parity(sh, nd, S, -10)
    assert sh[4].tolist() == [0, 0, 0, 5, 0, 0, 0]
    sh[:] = 0
    sh[0, 4] = 5  # (-3 + 0) % 7 == -3 in C: column 4 is not skipped either
    ora.gs_parity(sh, nd, S, -3)
    assert sh[4, 4] == 5


def test_gs_parity_nd1_closed_form(ora):
    S = 50
    sh = _gs_rows(1, S, 11)
    for sb in (0, 3, 49, 77):
        s = sh.copy()
        ora.gs_parity(s, 1, S, sb)
        want = s[0].copy()
        want[sb % S] = 0
        assert np.array_equal(s[1], s[0]) and np.array_equal(s[2], want)


def test_gs_recover_semantics(ora):
    nd, S = 6, 128
    ref = _gs_rows(nd, S, 21)
    ora.gs_parity(ref, nd, S, 0)
    # the reference benchmark never erases: decode returns the input
    for a, b in [(0, 1), (4, 2), (3, -1), (-1, 5), (7, 2), (2, 2)]:
        sh = ref.copy()
        ora.gs_recover(sh, nd, S, 0, a, b)
        assert np.array_equal(sh, ref), (a, b)
    # zeroed pair: a <- a ^ b, b stays zero (the recovery is not a decode)
    sh = ref.copy()
    sh[1] = 0
    sh[4] = 0
    ora.gs_recover(sh, nd, S, 0, 4, 1)
    assert np.array_equal(sh[1], ref[1] ^ ref[4]) and not sh[4].any()
    # a single zeroed row is recovered through P
    for a in range(nd):
        sh = ref.copy()
        sh[a] = 0
        ora.gs_recover(sh, nd, S, 0, a, -1)
        assert np.array_equal(sh, ref)
    # parity indices are dropped: data + P loss rebuilds only the data row
    sh = ref.copy()
    sh[2] = 0
    sh[nd] = 0
    ora.gs_recover(sh, nd, S, 0, 2, nd)
    assert np.array_equal(sh[2], np.bitwise_xor.reduce(ref[[0, 1, 3, 4, 5]], axis=0))


def test_gs_pack_load_full_identity(ora):
    rng = np.random.default_rng(8)
    T, n, nd = 9, 10, 4
    K = rng.integers(0, 65536, (T, n), dtype=np.uint16)
    V = rng.integers(0, 65536, (T, n), dtype=np.uint16)
    sh = ora.gs_backup(K, V, nd, 0)
    S = sh.shape[1]
    assert S == (2 * T * n + (nd - 2 * T * n % nd) % nd) // nd
    flat = sh[:nd].reshape(-1)
    assert np.array_equal(flat[: T * n], K.reshape(-1))
    assert np.array_equal(flat[T * n: 2 * T * n], V.reshape(-1))
    assert not flat[2 * T * n:].any()
    out = ora.gs_load_full(sh, nd, S, T, n)
    assert np.array_equal(out, np.concatenate([K.reshape(-1), V.reshape(-1)]))


def test_gs_pack_row(ora):
    rng = np.random.default_rng(9)
    w = 40
    k = rng.integers(0, 65536, w, dtype=np.uint16)
    v = rng.integers(0, 65536, w, dtype=np.uint16)
    rows = np.zeros((5, 2 * w + 3), np.uint16)
    ora.gs_pack_row(k, v, rows, 2)
    assert np.array_equal(rows[2, :w], k) and np.array_equal(rows[2, w:2 * w], v)
    assert not rows[[0, 1, 3, 4]].any() and not rows[2, 2 * w:].any()


# ------------------------------------------------------------------ gs RS16
def test_rs16_single_symbol_answers(ora):
    ex, lg = ora.gf16_tables()
    k, m, S = 5, 3, 4
    for i in range(k):
        for x in (1, 2, 0x8001, 0xFFFF):
            data = np.zeros(k * S, np.uint16)
            data[i * S + 1] = x
            sh = ora.rs16_encode(data, k, m, S, ex, lg)
            for p in range(m):
                want = int(gfref.gf16_mul(x, gfref.gf16_pow2((p + 1) * i)))
                assert sh[k + p].tolist() == [0, want, 0, 0], (i, x, p)


def test_rs16_reconstruct_round_trip(ora):
    ex, lg = ora.gf16_tables()
    rng = np.random.default_rng(10)
    k, m, S = 6, 3, 77
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    ref = ora.rs16_encode(data, k, m, S, ex, lg)
    assert np.array_equal(ref[:k].reshape(-1), data)
    for nm in (1, 2, 3):
        for miss in itertools.combinations(range(k), nm):
            for pused in itertools.combinations(range(m), nm):
                sh = ref.copy()
                sh[list(miss)] = 0
                ora.rs16_reconstruct(sh, S, k, m, list(miss), list(pused), ex, lg)
                assert np.array_equal(sh, ref), (miss, pused)


# ------------------------------------------------------------------ gather
@pytest.mark.parametrize("tb,page_tokens,tok_off,T", [(256, 16, 0, 48), (128, 4, 8, 13)])
def test_kv_gather_matches_indexing(ora, tb, page_tokens, tok_off, T):
    rng = np.random.default_rng(12)
    L, B, pps = 3, 2, 8
    pool_pages = B * pps + 5
    pool = rng.integers(0, 256, (L, pool_pages, page_tokens, 2, tb), dtype=np.uint8)
    pt = rng.permutation(pool_pages)[: B * pps].reshape(B, pps).astype(np.int32)
    got = ora.kv_gather(pool, pt, page_tokens, tok_off, T)
    t = np.arange(tok_off, tok_off + T)
    slots = pt[:, t // page_tokens] * page_tokens + t % page_tokens  # [B, T]
    tokpool = pool.reshape(L, pool_pages * page_tokens, 2, tb)
    for kv in range(2):
        want = tokpool[:, slots.reshape(-1), kv].reshape(L, B, T, tb)
        assert np.array_equal(got[:, :, :, kv], want)


# ------------------------------------------------------------------ chunked
def test_chunk_cells_cut_and_pad(ora):
    """The k pieces read in order give back the stream, then zeros."""
    rng = np.random.default_rng(11)
    k, p, rec = 5, 7, 32
    for n in (1, 31, 32 * 30, 32 * 30 + 5, 999):
        s = rng.integers(0, 256, n, dtype=np.uint8)
        W = ora.chunk_width(n, k, p, rec)
        assert W % rec == 0 and k * (p - 1) * W >= n and k * (p - 1) * (W - rec) < n
        cells = ora.chunk_cells(s, k, p, W)
        assert cells.shape == (k, (p - 1) * W)
        flat = cells.reshape(-1)
        assert np.array_equal(flat[:n], s) and not flat[n:].any()


@pytest.mark.parametrize("unit", [0, 64, 128])
def test_chunked_encode_is_per_chunk(ora, unit):
    """Chunk c owns region c of every shard ((p-1)*W bytes at c*(p-1)*W): the
    data regions hold the gathered chunk's pieces side by side, and each
    region's P, Q and RS parity are the codes of that region alone (striped
    geometry with rows of W bytes and the given unit)."""
    rng = np.random.default_rng(12 + unit)
    L, B, pps, pt, tb = 2, 3, 4, 16, 32
    npages = B * pps + 2
    pool = rng.integers(0, 256, (L, npages, pt, 2, tb), dtype=np.uint8)
    table = rng.permutation(npages)[: B * pps].astype(np.int32).reshape(B, pps)
    k, p, m, ct, nc = 5, 7, 3, 16, 4
    W, data, P, Q, rs = ora.chunked_encode(pool, table, pt, ct, nc, k, p, m, unit)
    n = (p - 1) * W
    assert all(x.size == nc * n for x in data + [P, Q] + rs)
    for c in range(nc):
        reg = slice(c * n, (c + 1) * n)
        s = ora.kv_gather(pool, table, pt, c * ct, ct)
        cells = ora.chunk_cells(s, k, p, W)
        for j in range(k):
            assert np.array_equal(data[j][reg], cells[j])
        Pc, Qc = ora.rdp_encode([np.ascontiguousarray(cells[j]) for j in range(k)], p, unit)
        assert np.array_equal(P[reg], Pc) and np.array_equal(Q[reg], Qc)
        rc = ora.rs8_encode([np.ascontiguousarray(cells[j]) for j in range(k)], m)
        for i in range(m):
            assert np.array_equal(rs[i][reg], rc[i])
    # every row of every stripe of a region satisfies RDP's equations (pinned
    # independently of the oracle's encode in test_rdp_striped_equations_hold)
    if unit:
        c, s_ = 1, 0
        g = min(unit, W - s_ * unit)
        base = c * n + s_ * (p - 1) * unit
        rows = lambda x: [x[base + r * g: base + (r + 1) * g] for r in range(p - 1)]  # noqa: E731
        Pr = rows(P)
        for r in range(p - 1):
            acc = Pr[r].copy()
            for j in range(k):
                acc ^= rows(data[j])[r]
            assert not acc.any()
