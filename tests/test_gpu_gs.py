"""gs family (the reference's own codes) on the GPU, bit-exact against the
oracle's restatement of benchmark/{xor,rdp,rs}/kernel.cu and
bench_ghostserve_rdp.py, through the reference-compatible Python signatures."""
import itertools

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def host(t):
    return t.cpu().numpy()


# ------------------------------------------------------------------ XOR
@pytest.mark.parametrize("nd,S", [(4, 262144), (8, 1000), (3, 17), (5, 1), (1, 33), (6, 4111),
                                  (7, 16), (2, 4096 * 3 + 5), (3, 8192), (6, 8192 + 15),
                                  (5, 8192 * 3 + 1)])
def test_xor_encode_matches_oracle(pkg, ora, gpu, nd, S):
    rng = np.random.default_rng(nd * 7 + S)
    data = rng.integers(0, 256, nd * S, dtype=np.uint8)
    want = ora.xor_encode(data, nd, S)
    shards = torch.full((nd + 1, S), 0x5A, dtype=torch.uint8, device=gpu)
    pkg.xor.xor_kernel.encode_xor(dev(data, gpu), shards, nd, S)
    assert np.array_equal(host(shards), want)


# The data rows ride on the parity kernel's loads when data and shards are
# disjoint and equally aligned modulo 16 bytes (else a separate copy): offsets
# into guard-filled buffers cover both paths, misaligned row starts, whole
# tiles and partial tails, and nothing outside the shard tensor may change.
@pytest.mark.parametrize("nd,S", [(6, 8192), (3, 4096 * 2 + 10), (4, 1000), (2, 17), (1, 4096),
                                  (2, 8192 * 2 + 3)])
@pytest.mark.parametrize("doff,soff", [(0, 0), (5, 5), (3, 7), (0, 16), (11, 27)])
def test_xor_encode_fused_copy_offsets(pkg, ora, gpu, nd, S, doff, soff):
    rng = np.random.default_rng(nd * 1000 + S + doff)
    data = rng.integers(0, 256, nd * S, dtype=np.uint8)
    want = ora.xor_encode(data, nd, S)
    dbuf = torch.zeros(nd * S + 64, dtype=torch.uint8, device=gpu)
    dbuf[doff:doff + nd * S] = dev(data, gpu)
    sbuf = torch.full(((nd + 1) * S + 64,), 0xA5, dtype=torch.uint8, device=gpu)
    shards = sbuf[soff:soff + (nd + 1) * S].view(nd + 1, S)
    pkg.xor.xor_kernel.encode_xor(dbuf[doff:doff + nd * S], shards, nd, S)
    assert np.array_equal(host(shards), want)
    rest = torch.cat([sbuf[:soff], sbuf[soff + (nd + 1) * S:]])
    assert bool((rest == 0xA5).all())


# forward_encode_kv's pack and the encode in one call (kvec_xor_encode_kv): the
# one-pass kernel for 16-byte-aligned K, V and shards with K a multiple of 16
# bytes (rows aligned or not, padding, partial last tiles, nd 1..8), and the
# copies-then-encode path otherwise (nd > 8, K not a multiple of 16, rows under
# one tile, K or V misaligned); the shard tensor's surroundings stay untouched.
@pytest.mark.parametrize("nd,kb,extra,koff,voff", [
    (6, 196608, 0, 0, 0), (3, 100000, 6, 0, 0), (8, 40000, 13, 0, 16), (1, 8192, 3000, 16, 0),
    (2, 4096, 0, 0, 0), (7, 65536, 4099, 0, 0),
    (9, 40000, 7, 0, 0), (4, 1000, 1, 0, 0), (2, 1024, 77, 0, 0), (5, 65536, 0, 3, 0), (5, 65536, 0, 0, 7)])
def test_xor_encode_kv_matches_oracle(pkg, ora, gpu, nd, kb, extra, koff, voff):
    S = -(-2 * kb // nd) + extra
    rng = np.random.default_rng(nd * 101 + kb + extra)
    K = rng.integers(0, 256, kb, dtype=np.uint8)
    V = rng.integers(0, 256, kb, dtype=np.uint8)
    padded = np.zeros(nd * S, np.uint8)
    padded[:kb], padded[kb:2 * kb] = K, V
    want = ora.xor_encode(padded, nd, S)
    kbuf = torch.zeros(kb + 32, dtype=torch.uint8, device=gpu)
    vbuf = torch.zeros(kb + 32, dtype=torch.uint8, device=gpu)
    kbuf[koff:koff + kb] = dev(K, gpu)
    vbuf[voff:voff + kb] = dev(V, gpu)
    sbuf = torch.full(((nd + 1) * S + 64,), 0xA5, dtype=torch.uint8, device=gpu)
    shards = sbuf[16:16 + (nd + 1) * S]
    pkg._lib.call("kvec_xor_encode_kv", kbuf[koff:].data_ptr(), vbuf[voff:].data_ptr(), kb,
                  shards.data_ptr(), nd, S, pkg._lib.stream_handle(gpu))
    assert np.array_equal(host(shards).reshape(nd + 1, S), want)
    assert bool((torch.cat([sbuf[:16], sbuf[16 + (nd + 1) * S:]]) == 0xA5).all())


# kvec_xor_recover_kv: a lost data row (one pass), a lost P, nothing lost, no
# output bytes, and an output overlapping the shard tensor (the two-step path).
@pytest.mark.parametrize("nd,S,out_bytes", [(6, 4096 * 3 + 37, 6 * (4096 * 3 + 37) - 5), (3, 1001, 2000),
                                            (9, 5000, 9 * 5000), (5, 8192 * 3 + 37, 5 * (8192 * 3 + 37) - 9)])
def test_xor_recover_kv_matches_oracle(pkg, ora, gpu, nd, S, out_bytes):
    rng = np.random.default_rng(nd + S)
    enc = ora.xor_encode(rng.integers(0, 256, nd * S, dtype=np.uint8), nd, S)
    st = pkg._lib.stream_handle(gpu)
    for missing in [0, nd - 1, nd, -1]:
        sh = enc.copy()
        if missing >= 0:
            sh[missing] = 0x77
        d = dev(sh, gpu)
        out = torch.full((out_bytes + 32,), 0xEE, dtype=torch.uint8, device=gpu)
        pkg._lib.call("kvec_xor_recover_kv", d.data_ptr(), out[16:].data_ptr(), nd, S, out_bytes,
                      missing, st)
        want = enc if missing >= 0 else sh
        assert np.array_equal(host(d), want), missing
        assert np.array_equal(host(out[16:16 + out_bytes]), want[:nd].reshape(-1)[:out_bytes]), missing
        assert bool((torch.cat([out[:16], out[16 + out_bytes:]]) == 0xEE).all())
    # no output bytes: the row is still rebuilt
    d = dev(np.where(np.arange(nd + 1)[:, None] == 1, 0, enc).astype(np.uint8), gpu)
    pkg._lib.call("kvec_xor_recover_kv", d.data_ptr(), 0, nd, S, 0, 1, st)
    assert np.array_equal(host(d), enc)
    # an output inside the shard tensor's own P row (its first out bytes): rebuild, then copy
    n = min(out_bytes, S)
    sh = enc.copy()
    sh[0] = 0
    d = dev(sh, gpu)
    pkg._lib.call("kvec_xor_recover_kv", d.data_ptr(), d[nd].data_ptr(), nd, S, n, 0, st)
    assert np.array_equal(host(d)[:nd], enc[:nd])
    assert np.array_equal(host(d)[nd, :n], enc[:nd].reshape(-1)[:n])


def test_xor_encode_kv_rejects_short_shards(pkg, gpu):
    t = torch.zeros(64, dtype=torch.uint8, device=gpu)
    with pytest.raises(pkg._lib.KvecError, match="exceed"):
        pkg._lib.call("kvec_xor_encode_kv", t.data_ptr(), t.data_ptr(), 32, t.data_ptr(), 2, 16,
                      pkg._lib.stream_handle(gpu))


@pytest.mark.parametrize("nd,S", [(4, 262144), (8, 999), (3, 17), (5, 3), (6, 4096 * 3 + 37), (2, 5000),
                                  (6, 8192 * 3 + 37), (3, 8192)])
def test_xor_reconstruct_matches_oracle(pkg, ora, gpu, nd, S):
    rng = np.random.default_rng(S)
    data = rng.integers(0, 256, nd * S, dtype=np.uint8)
    ref = ora.xor_encode(data, nd, S)
    for missing in [[m] for m in range(nd + 1)] + [[], [0, 1], [nd + 1], [-2]]:
        sh = ref.copy()
        if missing and 0 <= missing[0] <= nd:
            sh[missing[0]] = rng.integers(0, 256, S, dtype=np.uint8)
        want = sh.copy()
        want_miss = np.full((1, S), 0xEE, np.uint8)
        if len(missing) == 1 and 0 <= missing[0] <= nd:
            want_miss = ora.xor_reconstruct(want, S, nd, missing)
        else:
            ora.xor_reconstruct(want, S, nd, missing)
        d = dev(sh, gpu)
        rec_miss = torch.full((1, S), 0xEE, dtype=torch.uint8, device=gpu)
        mi = torch.tensor(missing, dtype=torch.int32, device=gpu)
        pkg.xor.xor_kernel.reconstruct_xor(d, d, rec_miss, S, nd, mi)
        assert np.array_equal(host(d), want), missing
        assert np.array_equal(host(rec_miss), want_miss), missing


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("nd", [4, 8, 3])
def test_xor_forward_backward_round_trip(pkg, ora, gpu, dtype, nd):
    B, H, T, D = 1, 2, 37, 128
    g = torch.Generator(device="cpu").manual_seed(nd)
    k = torch.randn(B, H, T, D, generator=g).to(dtype)
    v = torch.randn(B, H, T, D, generator=g).to(dtype)
    pk = pkg.xor.forward_encode_kv(k.to(gpu), v.to(gpu), nd, 1)
    es = k.element_size()
    kb = k.contiguous().view(torch.uint8).numpy().reshape(-1)
    vb = v.contiguous().view(torch.uint8).numpy().reshape(-1)
    stream = np.concatenate([kb, vb])
    S = pk["shard_size"]
    assert pk["total_bytes"] == 2 * es * T * B * H * D
    padded = np.zeros(nd * S, np.uint8)
    padded[: stream.size] = stream
    assert np.array_equal(host(pk["shards_KV"]), ora.xor_encode(padded, nd, S))
    for miss in range(nd + 1):
        pk2 = dict(pk)
        pk2["shards_KV"] = pk["shards_KV"].clone()
        pk2["shards_KV"][miss].fill_(0x5A)          # the lost shard's bytes are garbage
        kr, vr, st = pkg.xor.backwards_decode_kv(pk2, [miss])
        assert torch.equal(pk2["shards_KV"], pk["shards_KV"]), miss   # rebuilt in place
        assert kr.dtype == dtype and kr.shape == k.shape
        assert torch.equal(kr.cpu().view(torch.uint8), k.view(torch.uint8))
        assert torch.equal(vr.cpu().view(torch.uint8), v.view(torch.uint8))
        assert set(st) == {"reconstruct_ms", "reconstruct_io", "unpack_io"}
    with pytest.raises(ValueError):
        pkg.xor.backwards_decode_kv(pk, [0, 1])
    with pytest.raises(ValueError):
        pkg.xor.forward_encode_kv(k.to(gpu), v.to(gpu), nd, 2)


# ------------------------------------------------------------------ gs RDP
@pytest.mark.parametrize("nd,S", [(8, 5000), (6, 101), (1, 9), (3, 2), (2, 1), (13, 4103),
                                  (8, 2048), (8, 2049), (4, 16), (5, 24577), (8, 7),
                                  (8, 4096), (8, 4097), (6, 4096 * 6 + 1),
                                  # rows whose Q window starts more than one chunk
                                  # back (misalignment - 2 r < -16)
                                  (13, 4096), (11, 4100), (20, 4105), (16, 2000)])
@pytest.mark.parametrize("star_base", [0, 3, -1, -5, 10 ** 6])
def test_gs_rdp_parity_matches_oracle(pkg, ora, gpu, nd, S, star_base):
    rng = np.random.default_rng(nd * 1000 + S)
    rows = np.zeros((nd + 2, S), np.uint16)
    rows[:nd] = rng.integers(0, 65536, (nd, S), dtype=np.uint16)
    rows[nd:] = 0xABCD
    want = rows.copy()
    ora.gs_parity(want, nd, S, star_base)
    d = dev(rows, gpu)
    pkg.rdp_kv_ops.compute_rdp_parity(d, nd, S, star_base)
    assert np.array_equal(host(d), want)


def test_gs_rdp_parity_row_stride_is_S(pkg, ora, gpu):
    """compute_rdp_parity indexes with stride S even when rows is wider
    (bench_ghostserve_rdp.py:185-198)."""
    nd, S, W = 3, 40, 64
    rng = np.random.default_rng(1)
    rows = rng.integers(0, 65536, (nd + 3, W), dtype=np.uint16)
    want = rows.reshape(-1)[: (nd + 2) * S].reshape(nd + 2, S).copy()
    ora.gs_parity(want, nd, S, 1)
    d = dev(rows, gpu)
    pkg.rdp_kv_ops.compute_rdp_parity(d, nd, S, 1)
    got = host(d).reshape(-1)
    assert np.array_equal(got[: (nd + 2) * S], want.reshape(-1))
    assert np.array_equal(got[(nd + 2) * S:], rows.reshape(-1)[(nd + 2) * S:])


# The pack (K_TN || V_TN into the data rows) rides on the parity kernel when
# K and V are equally aligned modulo 16 with their place in the rows; offsets
# (in u16 words) pick that path or the copy-then-parity one.  The rows'
# padding keeps the caller's bytes (here a guard pattern) and enters P/Q as
# is; nothing outside the row tensor changes.
@pytest.mark.parametrize("T,n,nd,S_extra,koff,voff,soff,sb", [
    (64, 128, 6, 0, 0, 0, 0, 0),          # 2Tn multiple of 16: fused
    (3, 5, 4, 2, 1, 0, 1, 3),             # K/V boundary inside a chunk: fused
    (3, 5, 4, 2, 2, 0, 1, 0),             # K misaligned with its rows: copies
    (256, 1024, 6, 0, 5, 5, 5, -1),       # many tiles, misaligned rows: fused
    (256, 1024, 6, -900, 0, 0, 0, 2),     # K/V larger than the rows: truncated
    (100, 77, 13, 37, 3, 7, 3, 1000000),  # padding words, odd sizes: fused
    (2048, 9, 1, 0, 0, 0, 0, 0),          # one data row: fused
    (40, 50, 3, 5, 7, 7, 7, -5),          # fused
    (40, 50, 3, 5, 7, 3, 7, -5),          # V misaligned with its rows: copies
    (1, 5, 2, 3, 0, 5, 0, 0),             # K of 10 bytes: both boundaries in one chunk
    (2, 3, 3, 1, 0, 6, 0, 1),             # K of 12 bytes
])
def test_gs_fused_backup_layouts(pkg, ora, gpu, T, n, nd, S_extra, koff, voff, soff, sb):
    tn = T * n
    S = -(-2 * tn // nd) + S_extra
    rng = np.random.default_rng(T * 31 + n + nd)
    K = rng.integers(0, 65536, tn, dtype=np.uint16)
    V = rng.integers(0, 65536, tn, dtype=np.uint16)
    init = rng.integers(0, 65536, (nd + 2) * S, dtype=np.uint16).reshape(nd + 2, S)
    want = init.copy()
    ora.gs_pack(K.reshape(T, n), V.reshape(T, n), want, nd, S, T, n)
    ora.gs_parity(want, nd, S, sb)
    kb = torch.zeros(tn + 16, dtype=torch.int16, device=gpu)
    vb = torch.zeros(tn + 16, dtype=torch.int16, device=gpu)
    kb[koff:koff + tn] = dev(K.view(np.int16), gpu)
    vb[voff:voff + tn] = dev(V.view(np.int16), gpu)
    sbuf = torch.full(((nd + 2) * S + 32,), 0x3C3C, dtype=torch.int16, device=gpu)
    sbuf[soff:soff + (nd + 2) * S] = dev(init.reshape(-1).view(np.int16), gpu)
    shards = sbuf[soff:soff + (nd + 2) * S].view(nd + 2, S)
    pkg.rdp.rdp_kernel.fused_backup_full_kv(kb[koff:koff + tn].view(T, n),
                                            vb[voff:voff + tn].view(T, n), shards, nd, S, T, n, sb)
    assert np.array_equal(host(shards).view(np.uint16), want)
    rest = torch.cat([sbuf[:soff], sbuf[soff + (nd + 2) * S:]])
    assert bool((rest == 0x3C3C).all())


# The fused backup's batched tiles with K, V and the shard tensor 16-byte
# aligned and rows of at least one 4 KiB tile, for every row count nd <= 8:
# the K/V boundary inside a row, padding words holding the caller's bytes
# (they enter P/Q as is and are never written), star bases inside, outside and
# before the rows, guard words after the shard tensor.
@pytest.mark.parametrize("nd", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("S_extra,sb", [(0, 0), (3, -1), (7, 5), (1, 123457)])
def test_gs_backup_aligned_every_nd(pkg, ora, gpu, nd, S_extra, sb):
    T, n = 97, 136                      # K of 26,384 bytes
    tn = T * n
    S = -(-2 * tn // nd) + S_extra
    rng = np.random.default_rng(nd * 100 + S_extra)
    K = rng.integers(0, 65536, tn, dtype=np.uint16)
    V = rng.integers(0, 65536, tn, dtype=np.uint16)
    init = rng.integers(0, 65536, (nd + 2) * S, dtype=np.uint16).reshape(nd + 2, S)
    want = init.copy()
    ora.gs_pack(K.reshape(T, n), V.reshape(T, n), want, nd, S, T, n)
    ora.gs_parity(want, nd, S, sb)
    sbuf = torch.full(((nd + 2) * S + 64,), 0x3C3C, dtype=torch.int16, device=gpu)
    sbuf[:(nd + 2) * S] = dev(init.reshape(-1).view(np.int16), gpu)
    shards = sbuf[:(nd + 2) * S].view(nd + 2, S)
    pkg.rdp.rdp_kernel.fused_backup_full_kv(dev(K.view(np.int16), gpu).view(T, n),
                                            dev(V.view(np.int16), gpu).view(T, n), shards, nd, S, T, n, sb)
    assert np.array_equal(host(shards).view(np.uint16), want)
    assert bool((sbuf[(nd + 2) * S:] == 0x3C3C).all())


@pytest.mark.parametrize("B,H,T,D,nd", [(1, 8, 512, 128, 8), (2, 1, 33, 128, 6), (1, 2, 5, 64, 3),
                                        (1, 1, 7, 3, 4)])
def test_gs_backup_and_recovery(pkg, ora, gpu, B, H, T, D, nd):
    g = torch.Generator(device="cpu").manual_seed(T)
    K = torch.randn(B, H, T, D, generator=g).half()
    V = torch.randn(B, H, T, D, generator=g).half()
    n = B * H * D
    pk = pkg.rdp.fused_backup_full_kv(K.to(gpu), V.to(gpu), nd, star_base=0)
    K_TN = K.permute(2, 0, 1, 3).contiguous().view(T, n).view(torch.uint16).numpy()
    V_TN = V.permute(2, 0, 1, 3).contiguous().view(T, n).view(torch.uint16).numpy()
    want = ora.gs_backup(K_TN, V_TN, nd, 0)
    assert set(pk) >= {"shards_KV", "shard_size", "seq_len", "n", "num_data_shards", "star_base",
                       "shape_BHTD", "backup_ms", "pad_words"}
    assert np.array_equal(host(pk["shards_KV"]), want)
    S = pk["shard_size"]
    for a, b in [(-1, -1), (0, 1), (nd - 1, 0), (2 % nd, -1), (-1, nd - 1), (nd, 1), (1, 1)]:
        sh = want.copy()
        # erase the named data rows, as a real loss would
        for x in (a, b):
            if 0 <= x < nd:
                sh[x] = 0
        exp = sh.copy()
        ora.gs_recover(exp, nd, S, 0, a, b)
        exp_out = ora.gs_load_full(exp, nd, S, T, n)
        pk2 = dict(pk)
        pk2["shards_KV"] = dev(sh, gpu)
        kr, vr, st = pkg.rdp.fused_recovery_full_kv(pk2, a, b)
        assert np.array_equal(host(pk2["shards_KV"]), exp), (a, b)
        got = np.concatenate([kr.permute(2, 0, 1, 3).contiguous().cpu().view(torch.uint16).numpy().reshape(-1),
                              vr.permute(2, 0, 1, 3).contiguous().cpu().view(torch.uint16).numpy().reshape(-1)])
        assert np.array_equal(got, exp_out), (a, b)
        assert "recover_ms" in st


@pytest.mark.parametrize("sb", [-2, 3, -7])
def test_gs_recovery_star_base(pkg, ora, gpu, sb):
    """A backup with star_base sb and recoveries under it: one lost row for
    any sb; two lost rows when (sb + a) % S >= 0 for the lower row a, where
    star_base changes no output byte (the reference's star-cell write lands
    in row a, which is rebuilt); (sb + a) % S < 0 addresses outside row a in
    the reference and is refused, the shards left as they were."""
    B, H, T, D, nd = 1, 2, 40, 64, 6
    g = torch.Generator(device="cpu").manual_seed(11)
    K = torch.randn(B, H, T, D, generator=g).half()
    V = torch.randn(B, H, T, D, generator=g).half()
    n = B * H * D
    pk = pkg.rdp.fused_backup_full_kv(K.to(gpu), V.to(gpu), nd, star_base=sb)
    K_TN = K.permute(2, 0, 1, 3).contiguous().view(T, n).view(torch.uint16).numpy()
    V_TN = V.permute(2, 0, 1, 3).contiguous().view(T, n).view(torch.uint16).numpy()
    want = ora.gs_backup(K_TN, V_TN, nd, sb)
    assert np.array_equal(host(pk["shards_KV"]), want)
    S = pk["shard_size"]
    for a, b in [(0, 3), (2, 4), (5, 1), (3, -1), (-1, 0), (4, 4)]:
        sh = want.copy()
        for x in (a, b):
            if 0 <= x < nd:
                sh[x] = 0x5A5A
        pk2 = dict(pk)
        pk2["shards_KV"] = dev(sh, gpu)
        lo = min(x for x in (a, b) if x >= 0) if (a >= 0 or b >= 0) else -1
        two = a >= 0 and b >= 0 and a != b
        if two and sb + lo < 0 and (sb + lo) % S != 0:
            with pytest.raises(RuntimeError, match="star_base"):
                pkg.rdp.fused_recovery_full_kv(pk2, a, b)
            assert np.array_equal(host(pk2["shards_KV"]), sh), (a, b)
            continue
        exp = sh.copy()
        ora.gs_recover(exp, nd, S, sb, a, b)
        kr, vr, _ = pkg.rdp.fused_recovery_full_kv(pk2, a, b)
        assert np.array_equal(host(pk2["shards_KV"]), exp), (a, b)


# The recovery's rebuild and copy-out run as one pass: shard tensors 0 or 10
# bytes past alignment, outputs misaligned differently, rows of odd length
# (partial last tiles), padding words in the last data row, nd up to 10 (the
# row-at-a-time path past 8), every kind of missing pair, and guard words on
# both sides of both buffers.
@pytest.mark.parametrize("nd", [1, 2, 3, 6, 8, 9, 10])
@pytest.mark.parametrize("soff,ooff", [(0, 0), (5, 3)])
@pytest.mark.parametrize("T,n", [(41, 200), (96, 211)])
def test_gs_recover_layouts(pkg, ora, gpu, nd, soff, ooff, T, n):
    total = 2 * T * n
    S = -(-total // nd) + 3
    rng = np.random.default_rng(nd * 13 + soff + T)
    base = rng.integers(0, 65536, (nd + 2, S), dtype=np.uint16)
    for a, b in [(-1, -1), (0, 1), (nd - 1, -1), (-1, 0), (1, 0), (nd, -1)]:
        sh = base.copy()
        for x in (a, b):
            if 0 <= x < nd:
                sh[x] = 0
        exp = sh.copy()
        ora.gs_recover(exp, nd, S, 0, a, b)
        exp_out = ora.gs_load_full(exp, nd, S, T, n)
        sbuf = torch.full(((nd + 2) * S + 16,), 0x3C3C, dtype=torch.int16, device=gpu)
        sbuf[soff:soff + (nd + 2) * S] = dev(sh.reshape(-1).view(np.int16), gpu)
        obuf = torch.full((total + 16,), 0x5A5A, dtype=torch.int16, device=gpu)
        shards = sbuf[soff:soff + (nd + 2) * S].view(nd + 2, S)
        pkg.rdp.rdp_kernel.fused_recovery_full_kv(shards, obuf[ooff:ooff + total], nd, S, T, n, 0, a, b)
        assert np.array_equal(host(shards).view(np.uint16), exp), (a, b)
        assert np.array_equal(host(obuf[ooff:ooff + total]).view(np.uint16), exp_out), (a, b)
        assert bool((torch.cat([sbuf[:soff], sbuf[soff + (nd + 2) * S:]]) == 0x3C3C).all())
        assert bool((torch.cat([obuf[:ooff], obuf[ooff + total:]]) == 0x5A5A).all())


def test_gs_single_row_recovery_restores_kv(pkg, gpu):
    B, H, T, D, nd = 1, 4, 64, 128, 8
    K = torch.randn(B, H, T, D, device=gpu).half()
    V = torch.randn(B, H, T, D, device=gpu).half()
    pk = pkg.rdp.fused_backup_full_kv(K, V, nd)
    pk["shards_KV"][5].view(torch.int16).zero_()
    kr, vr, _ = pkg.rdp.fused_recovery_full_kv(pk, 5)
    assert torch.equal(kr.view(torch.int16), K.view(torch.int16))
    assert torch.equal(vr.view(torch.int16), V.view(torch.int16))


def test_gs_pack_row(pkg, ora, gpu):
    rng = np.random.default_rng(3)
    world, w = 4, 1000
    S = 2 * w + 1
    rows = np.zeros((world + 2, S), np.uint16)
    d = dev(rows, gpu)
    for r in range(world):
        k = rng.integers(0, 65536, w, dtype=np.uint16)
        v = rng.integers(0, 65536, w, dtype=np.uint16)
        ora.gs_pack_row(k, v, rows, r)
        pkg.rdp_kv_ops.pack_row_from_block(dev(k, gpu).view(torch.float16).view(1, 1, w, 1),
                                           dev(v, gpu).view(torch.float16).view(1, 1, w, 1), d, r)
    assert np.array_equal(host(d), rows)
    ora.gs_parity(rows, world, S, 2)
    pkg.rdp_kv_ops.compute_rdp_parity(d, nd=world, S=S, star_base=2)
    assert np.array_equal(host(d), rows)
    with pytest.raises(RuntimeError):
        pkg.rdp_kv_ops.pack_row_from_block(dev(np.zeros(S, np.uint16), gpu).view(torch.float16),
                                           dev(np.zeros(S, np.uint16), gpu).view(torch.float16), d, 0)
    # a row outside the tensor is rejected before anything is written
    kz = dev(np.ones(w, np.uint16), gpu).view(torch.float16)
    for bad in (world + 2, -1):
        with pytest.raises(RuntimeError, match="row must be in"):
            pkg.rdp_kv_ops.pack_row_from_block(kz, kz, d, bad)
    assert np.array_equal(host(d), rows)


# ------------------------------------------------------------------ gs RS16
@pytest.mark.parametrize("k,m,S", [(8, 2, 4096), (6, 2, 44741), (5, 3, 1000), (4, 1, 3), (6, 2, 8192),
                                   (3, 2, 8192 * 3 + 5),
                                   (8, 0, 100), (10, 4, 2049), (1, 1, 77), (16, 3, 8),
                                   (6, 7, 1001), (3, 16, 513), (48, 1, 300)])
def test_rs16_encode_matches_oracle(pkg, ora, gpu, k, m, S):
    ex, lg = ora.gf16_tables()
    rng = np.random.default_rng(k * 100 + m)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    data[rng.integers(0, k * S, k * S // 7)] = 0  # zeros take the reference's skip
    want = ora.rs16_encode(data, k, m, S, ex, lg)
    shards = torch.zeros((k + m, S), dtype=torch.uint16, device=gpu)
    gex, glg = pkg.rs.device_gf_tables(gpu)
    pkg.rs.rs_kernel.encode_rs_u16(dev(data, gpu), shards, k, m, S, gex, glg)
    assert np.array_equal(host(shards), want)


@pytest.mark.parametrize("k,m,S", [(6, 2, 16384 + 5), (4, 1, 3000), (7, 2, 9)])
def test_rs16_encode_other_generator(pkg, ora, gpu, k, m, S):
    """Tables of the same field with generator alpha^2 = 4 (log base 4): the
    coefficients alpha'^((p+1) i) are no longer chains of doublings, so the
    encode must leave its Horner path and still give the reference's bytes for
    these tables."""
    ex0, lg0 = ora.gf16_tables()
    ex, lg = _gen4_tables(ora)
    assert ex[1] == 4 and all(ex[lg[x]] == x for x in (1, 2, 3, 0x8000, 0xFFFF))
    rng = np.random.default_rng(k * 7 + S)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    want = ora.rs16_encode(data, k, m, S, ex, lg)
    assert not np.array_equal(want, ora.rs16_encode(data, k, m, S, ex0, lg0))
    shards = torch.zeros((k + m, S), dtype=torch.uint16, device=gpu)
    pkg.rs.rs_kernel.encode_rs_u16(dev(data, gpu), shards, k, m, S, dev(ex, gpu), dev(lg, gpu))
    assert np.array_equal(host(shards), want)


@pytest.mark.parametrize("k,m,S", [(6, 2, 4096), (3, 3, 4096 * 2 + 5), (4, 1, 1000), (2, 2, 9)])
@pytest.mark.parametrize("doff,soff", [(0, 0), (3, 3), (1, 5), (0, 8), (7, 15)])
def test_rs16_encode_fused_copy_offsets(pkg, ora, gpu, k, m, S, doff, soff):
    """Offsets in u16 words: equal offsets modulo 8 words take the fused copy."""
    ex, lg = ora.gf16_tables()
    rng = np.random.default_rng(k * 100 + S + doff)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    want = ora.rs16_encode(data, k, m, S, ex, lg)
    dbuf = torch.zeros(k * S + 32, dtype=torch.int16, device=gpu)
    dbuf[doff:doff + k * S] = dev(data.view(np.int16), gpu)
    sbuf = torch.full(((k + m) * S + 32,), 0x1234, dtype=torch.int16, device=gpu)
    shards = sbuf[soff:soff + (k + m) * S].view(k + m, S)
    gex, glg = pkg.rs.device_gf_tables(gpu)
    pkg.rs.rs_kernel.encode_rs_u16(dbuf[doff:doff + k * S].view(torch.uint16),
                                   shards.view(torch.uint16), k, m, S, gex, glg)
    assert np.array_equal(host(shards).view(np.uint16), want)
    rest = torch.cat([sbuf[:soff], sbuf[soff + (k + m) * S:]])
    assert bool((rest == 0x1234).all())


@pytest.mark.parametrize("k,m,S", [(8, 2, 4099), (6, 3, 1000), (5, 3, 9), (9, 5, 2051)])
def test_rs16_reconstruct_matches_oracle(pkg, ora, gpu, k, m, S):
    ex, lg = ora.gf16_tables()
    rng = np.random.default_rng(S)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    ref = ora.rs16_encode(data, k, m, S, ex, lg)
    gex, glg = pkg.rs.device_gf_tables(gpu)
    for nm in range(1, m + 1):
        for miss in list(itertools.combinations(range(k), nm))[:12]:
            for pused in list(itertools.combinations(range(m), nm))[:3]:
                sh = ref.copy()
                sh[list(miss)] = rng.integers(0, 65536, (nm, S), dtype=np.uint16)
                want = sh.copy()
                ora.rs16_reconstruct(want, S, k, m, list(miss), list(pused), ex, lg)
                assert np.array_equal(want, ref)
                d = dev(sh, gpu)
                pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(
                    d, S, k, m, torch.tensor(miss, dtype=torch.int32, device=gpu),
                    torch.tensor(pused, dtype=torch.int32, device=gpu), gex, glg)
                assert np.array_equal(host(d), want), (miss, pused)


def _gen4_tables(ora):
    """Tables of the same field with generator alpha^2 = 4 (log base 4)."""
    ex0, lg0 = ora.gf16_tables()
    n = np.arange(2 * 65535, dtype=np.int64)
    ex = ex0[(2 * n) % 65535].astype(np.uint16)
    lg = ((lg0.astype(np.int64) * 32768) % 65535).astype(np.uint16)   # 2 * 32768 = 1 mod 65535
    lg[0] = 0
    return ex, lg


def _poly_tables(poly):
    """exp/log tables of GF(2^16) with the primitive polynomial `poly`, generator 2."""
    ex = np.zeros(2 * 65535, np.uint16)
    lg = np.zeros(65536, np.uint16)
    x = 1
    for i in range(65535):
        ex[i] = x
        lg[x] = i
        x <<= 1
        if x & 0x10000:
            x ^= poly
    ex[65535:] = ex[:65535]
    return ex, lg


@pytest.mark.parametrize("k,S", [(6, 44741), (3, 4096 * 2 + 5)])
def test_rs16_horner_field_with_top_reduction_bit(pkg, ora, gpu, k, S):
    """Tables of GF(2^16) over x^16 + x^15 + x^4 + x + 1 (0x18013, generator
    2): the reduction word 2^16 = 0x8013 has its top bit set, so 2^17 needs a
    second reduction, which the times-4 steps of the encode's second parity
    and of the reconstruct's syndromes (a table of the two shifted-out bits)
    must apply."""
    m = 2
    ex, lg = _poly_tables(0x18013)
    assert ex[1] == 2 and ex[16] == 0x8013 and len(set(ex[:65535].tolist())) == 65535
    rng = np.random.default_rng(k + S)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    want = ora.rs16_encode(data, k, m, S, ex, lg)
    gex, glg = dev(ex, gpu), dev(lg, gpu)
    shards = torch.zeros((k + m, S), dtype=torch.uint16, device=gpu)
    pkg.rs.rs_kernel.encode_rs_u16(dev(data, gpu), shards, k, m, S, gex, glg)
    assert np.array_equal(host(shards), want)
    for miss, pused in [((0, k - 1), (0, 1)), ((1,), (1,)), ((k - 1,), (0,)), ((0, 1), (1, 0))]:
        sh = want.copy()
        sh[list(miss)] = 0x1234
        expect = sh.copy()
        ora.rs16_reconstruct(expect, S, k, m, list(miss), list(pused), ex, lg)
        assert np.array_equal(expect, want)
        d = dev(sh, gpu)
        pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(
            d, S, k, m, torch.tensor(miss, dtype=torch.int32, device=gpu),
            torch.tensor(pused, dtype=torch.int32, device=gpu), gex, glg)
        assert np.array_equal(host(d), expect), (miss, pused)


@pytest.mark.parametrize("k,mp,S,soff,gen4", [(6, 2, 44741, 0, False), (6, 2, 44741, 3, False),
                                              (6, 2, 44741, 5, True), (8, 3, 5003, 7, False),
                                              (4, 2, 517, 1, True), (2, 2, 1000, 2, False),
                                              (1, 1, 9, 0, False), (7, 4, 2048, 6, True)])
def test_rs16_reconstruct_offsets_and_generators(pkg, ora, gpu, k, mp, S, soff, gen4):
    """The reconstruct with the shard tensor at word offset soff of a larger
    buffer (the bytes around it stay untouched), every data row of a small
    code lost (k = m), the last parity row used, and tables with generator 4
    (no chains of doublings: the byte maps of every coefficient)."""
    ex, lg = _gen4_tables(ora) if gen4 else ora.gf16_tables()
    rng = np.random.default_rng(k * 1000 + S + soff)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    ref = ora.rs16_encode(data, k, mp, S, ex, lg)
    gex, glg = dev(ex, gpu), dev(lg, gpu)
    cases = [((0,), (mp - 1,)), ((k - 1,), (0,))]
    if k >= 2 and mp >= 2:
        cases += [((0, k - 1), (mp - 2, mp - 1)), ((k - 1, 0), (mp - 1, 0))]
    for miss, pused in cases:
        sh = ref.copy()
        sh[list(miss)] = rng.integers(0, 65536, (len(miss), S), dtype=np.uint16)
        want = sh.copy()
        ora.rs16_reconstruct(want, S, k, mp, list(miss), list(pused), ex, lg)
        assert np.array_equal(want, ref)
        buf = torch.full(((k + mp) * S + 16,), 0x2A2A, dtype=torch.int16, device=gpu)
        buf[soff:soff + (k + mp) * S] = dev(sh.reshape(-1).view(np.int16), gpu)
        d = buf[soff:soff + (k + mp) * S].view(k + mp, S).view(torch.uint16)
        pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(
            d, S, k, mp, torch.tensor(miss, dtype=torch.int32, device=gpu),
            torch.tensor(pused, dtype=torch.int32, device=gpu), gex, glg)
        assert np.array_equal(host(d), want), (miss, pused)
        rest = torch.cat([buf[:soff], buf[soff + (k + mp) * S:]])
        assert bool((rest == 0x2A2A).all()), (miss, pused)


@pytest.mark.parametrize("k", range(1, 9))
@pytest.mark.parametrize("S,soff,gen4", [(4096, 0, False), (8192 * 2 + 7, 3, False), (4096 * 3 + 1, 5, True)])
def test_rs16_reconstruct_tiles(pkg, ora, gpu, k, S, soff, gen4):
    """Rows of at least one 8 KiB tile with k <= 8 take the one-shot tile
    reconstruct (each wave building the inverse's byte maps).  Every single
    and every pair of lost rows, parity rows in either order and up to parity 2, a
    repeated parity row (the reference's singular system, whose second
    Gauss-Jordan step is skipped: the output is not the data but must still be
    the reference's), the tensor at an odd word offset, and tables with
    generator 4."""
    mp = 3
    ex, lg = _gen4_tables(ora) if gen4 else ora.gf16_tables()
    rng = np.random.default_rng(k * 31 + S + soff)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    ref = ora.rs16_encode(data, k, mp, S, ex, lg)
    gex, glg = dev(ex, gpu), dev(lg, gpu)
    pairs = [(0, 1), (1, 0), (2, 0), (1, 2), (1, 1), (2, 2)]
    cases = [((i,), (i % mp,)) for i in range(k)]
    cases += [(mi, pairs[n % len(pairs)]) for n, mi in enumerate(itertools.combinations(range(k), 2))]
    cases += [((k - 1, 0), (0, 1))] if k >= 2 else []
    buf = torch.full(((k + mp) * S + 16,), 0x2A2A, dtype=torch.int16, device=gpu)
    d = buf[soff:soff + (k + mp) * S].view(k + mp, S).view(torch.uint16)
    for miss, pused in cases:
        sh = ref.copy()
        sh[list(miss)] = rng.integers(0, 65536, (len(miss), S), dtype=np.uint16)
        want = sh.copy()
        ora.rs16_reconstruct(want, S, k, mp, list(miss), list(pused), ex, lg)
        assert np.array_equal(want, ref) == (len(set(pused)) == len(pused)), (miss, pused)
        buf[soff:soff + (k + mp) * S] = dev(sh.reshape(-1).view(np.int16), gpu)
        pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(
            d, S, k, mp, torch.tensor(miss, dtype=torch.int32, device=gpu),
            torch.tensor(pused, dtype=torch.int32, device=gpu), gex, glg)
        assert np.array_equal(host(d), want), (miss, pused)
        rest = torch.cat([buf[:soff], buf[soff + (k + mp) * S:]])
        assert bool((rest == 0x2A2A).all()), (miss, pused)


# ------------------------------------------- RS16 at k * m beyond 48 maps
# The reference's encode takes any k and m and its reconstruct any k with
# m <= 16 (benchmark/rs/kernel.cu:67-102, :105-222): these shapes run the
# Horner kernels (one multiplier per output, the inverse by a thread per entry).
@pytest.mark.parametrize("k,m,S", [(10, 5, 8192 * 2 + 3), (16, 4, 4096), (25, 2, 30001), (7, 7, 9),
                                   (49, 1, 1000), (5, 20, 517), (3, 17, 2048 * 5),
                                   (16, 4, 4096 * 3 + 8), (17, 3, 6168), (13, 4, 4096 * 4)])
@pytest.mark.parametrize("doff,soff", [(0, 0), (3, 5), (8, 0)])
def test_rs16_encode_any_k_m(pkg, ora, gpu, k, m, S, doff, soff):
    """Offsets in u16 words: the data and shard tensors at any alignment;
    the words around the shard tensor stay untouched.  With three or four
    parities over 16-byte-aligned data rows (doff 0 or 8, S a multiple of 8)
    the full tiles run on the ring kernel and a partial last tile on the
    general one (S = 4096 * 3 + 8: three full tiles and 16 bytes; 6168: one
    and 4,144 bytes); otherwise every tile runs on the general kernel."""
    ex, lg = ora.gf16_tables()
    rng = np.random.default_rng(k * 1000 + m * 10 + S)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    data[rng.integers(0, k * S, k * S // 7)] = 0
    want = ora.rs16_encode(data, k, m, S, ex, lg)
    dbuf = torch.zeros(k * S + 16, dtype=torch.int16, device=gpu)
    dbuf[doff:doff + k * S] = dev(data.view(np.int16), gpu)
    sbuf = torch.full(((k + m) * S + 16,), 0x1234, dtype=torch.int16, device=gpu)
    shards = sbuf[soff:soff + (k + m) * S].view(k + m, S)
    gex, glg = pkg.rs.device_gf_tables(gpu)
    pkg.rs.rs_kernel.encode_rs_u16(dbuf[doff:doff + k * S].view(torch.uint16), shards.view(torch.uint16),
                                   k, m, S, gex, glg)
    assert np.array_equal(host(shards).view(np.uint16), want)
    rest = torch.cat([sbuf[:soff], sbuf[soff + (k + m) * S:]])
    assert bool((rest == 0x1234).all())


@pytest.mark.parametrize("k,m,S,poly", [(12, 5, 5003, None), (20, 3, 4099, None), (25, 3, 2 * 8192 + 9, 0x18013),
                                         (49, 1, 777, 0x18013), (20, 4, 8192 + 8, None), (18, 4, 4096 * 2, 0x18013)])
def test_rs16_encode_any_k_m_other_generator(pkg, ora, gpu, k, m, S, poly):
    """Tables with generator 4 (poly None): the per-output multiplier is
    gf_exp[p + 1] of those tables, through its byte maps even where
    generator-2 tables take doubling chains (m <= 4); and generator-2 tables
    of x^16 + x^15 + x^4 + x + 1, whose reduction word has its top bit set,
    through the chains.  The bytes are the reference's for those tables."""
    ex, lg = _gen4_tables(ora) if poly is None else _poly_tables(poly)
    rng = np.random.default_rng(5)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    want = ora.rs16_encode(data, k, m, S, ex, lg)
    shards = torch.zeros((k + m, S), dtype=torch.uint16, device=gpu)
    pkg.rs.rs_kernel.encode_rs_u16(dev(data, gpu), shards, k, m, S, dev(ex, gpu), dev(lg, gpu))
    assert np.array_equal(host(shards), want)


@pytest.mark.parametrize("k,mp,S,soff,gen4", [(16, 4, 4096 * 2 + 5, 0, False), (20, 3, 1000, 3, False),
                                              (25, 2, 8192 + 1, 1, False), (13, 4, 517, 0, True),
                                              (20, 16, 300, 2, False), (17, 16, 2048 * 3, 0, True)])
def test_rs16_reconstruct_any_k(pkg, ora, gpu, k, mp, S, soff, gen4):
    """Lost sets of m rows with k * m > 48 (up to all 16 parities): first,
    last and scattered rows, parity rows in any order, a repeated parity row
    (the reference's singular system: Gauss-Jordan skips a step, the output is
    not the data but must still be the reference's), the tensor at a word
    offset with the words around it untouched."""
    ex, lg = _gen4_tables(ora) if gen4 else ora.gf16_tables()
    rng = np.random.default_rng(k * 100 + mp + S)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    ref = ora.rs16_encode(data, k, mp, S, ex, lg)
    gex, glg = dev(ex, gpu), dev(lg, gpu)
    cases = []
    for nm in sorted({mp, max(1, mp - 1), mp // 2 + 1}):
        if k * nm <= 48:
            continue
        rows = list(range(k))
        cases.append((tuple(rows[:nm]), tuple(range(nm))))
        cases.append((tuple(rows[-nm:]), tuple(reversed(range(mp - nm, mp)))))
        pick = rng.choice(k, nm, replace=False)
        cases.append((tuple(int(x) for x in pick), tuple(int(x) for x in rng.permutation(mp)[:nm])))
        if nm >= 2:
            cases.append((tuple(int(x) for x in rng.choice(k, nm, replace=False)), (0,) * 2 + tuple(range(2, nm))))
    assert cases
    buf = torch.full(((k + mp) * S + 16,), 0x2A2A, dtype=torch.int16, device=gpu)
    d = buf[soff:soff + (k + mp) * S].view(k + mp, S).view(torch.uint16)
    for miss, pused in cases:
        sh = ref.copy()
        sh[list(miss)] = rng.integers(0, 65536, (len(miss), S), dtype=np.uint16)
        want = sh.copy()
        ora.rs16_reconstruct(want, S, k, mp, list(miss), list(pused), ex, lg)
        assert np.array_equal(want, ref) == (len(set(pused)) == len(pused)), (miss, pused)
        buf[soff:soff + (k + mp) * S] = dev(sh.reshape(-1).view(np.int16), gpu)
        pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(
            d, S, k, mp, torch.tensor(miss, dtype=torch.int32, device=gpu),
            torch.tensor(pused, dtype=torch.int32, device=gpu), gex, glg)
        assert np.array_equal(host(d), want), (miss, pused)
        rest = torch.cat([buf[:soff], buf[soff + (k + mp) * S:]])
        assert bool((rest == 0x2A2A).all()), (miss, pused)


@pytest.mark.parametrize("k,mp,S,soff,gen", [(16, 4, 2048 * 3 + 8, 0, 2), (25, 4, 2048 * 2, 8, 2),
                                             (13, 6, 2048 * 4 + 16, 0, 2), (20, 4, 2048 * 3, 0, 0x18013),
                                             (14, 4, 2048 * 2 + 8, 0, 4), (30, 4, 2048 + 8, 8, 2),
                                             (50, 4, 2048 * 2 + 8, 0, 2)])
def test_rs16_reconstruct_ring(pkg, ora, gpu, k, mp, S, soff, gen):
    """Up to four lost rows with k * m > 48 over 16-byte-aligned rows (soff
    and S multiples of 8 words): every tile on the ring kernel (syndromes by
    doubling chains over the surviving rows, each loaded two survivors
    ahead), partial last tiles included (S = 2048 * 3 + 8: a last tile of 16
    bytes in one-window tiles, 4,112 in two-window ones; 2048 * 4 + 16: 32
    bytes; 2048 * 3 with three lost rows: a two-window tile's first window
    only; k = 50: one lost row).  Lost rows at both ends and in runs (one
    chain then spans several rows), a repeated parity row (the reference's
    singular system), parity rows up to 3 and, with six parities, beyond 3
    (no chains: every tile on the byte-map kernel); generator-2 tables of
    x^16 + x^15 + x^4 + x + 1 (the reduction word's top bit set) and
    generator-4 tables (no chains)."""
    ex, lg = (ora.gf16_tables() if gen == 2 else _gen4_tables(ora) if gen == 4 else _poly_tables(gen))
    rng = np.random.default_rng(k * 7 + mp + S + gen)
    data = rng.integers(0, 65536, k * S, dtype=np.uint16)
    ref = ora.rs16_encode(data, k, mp, S, ex, lg)
    gex, glg = dev(ex, gpu), dev(lg, gpu)
    cases = []
    for nm in range(1, 5):
        if k * nm <= 48:
            continue
        cases.append((tuple(range(nm)), tuple(range(nm))))
        cases.append((tuple(range(k - nm, k)), tuple(reversed(range(nm)))))
        cases.append(((0, k - 1, 5, 6)[:nm], tuple(rng.permutation(4)[:nm].tolist())))
        cases.append(((8, 9, 10, 11)[:nm], (3, 1, 0, 2)[:nm]))
        cases.append((tuple(rng.choice(k, nm, replace=False).tolist()), tuple(rng.permutation(4)[:nm].tolist())))
        if nm >= 2:
            cases.append((tuple(rng.choice(k, nm, replace=False).tolist()), (0, 0, 2, 3)[:nm]))
        if mp > 4:
            cases.append((tuple(rng.choice(k, nm, replace=False).tolist()), (5, 2, 4, 0)[:nm]))
            cases.append(((0, 3, 4, k - 1)[:nm], (4, 3, 1, 0)[:nm]))
    assert cases
    buf = torch.full(((k + mp) * S + 16,), 0x2A2A, dtype=torch.int16, device=gpu)
    d = buf[soff:soff + (k + mp) * S].view(k + mp, S).view(torch.uint16)
    assert d.data_ptr() % 16 == 0
    for miss, pused in cases:
        sh = ref.copy()
        sh[list(miss)] = rng.integers(0, 65536, (len(miss), S), dtype=np.uint16)
        want = sh.copy()
        ora.rs16_reconstruct(want, S, k, mp, list(miss), list(pused), ex, lg)
        assert np.array_equal(want, ref) == (len(set(pused)) == len(pused)), (miss, pused)
        buf[soff:soff + (k + mp) * S] = dev(sh.reshape(-1).view(np.int16), gpu)
        pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(
            d, S, k, mp, torch.tensor(miss, dtype=torch.int32, device=gpu),
            torch.tensor(pused, dtype=torch.int32, device=gpu), gex, glg)
        assert np.array_equal(host(d), want), (miss, pused)
        rest = torch.cat([buf[:soff], buf[soff + (k + mp) * S:]])
        assert bool((rest == 0x2A2A).all()), (miss, pused)


def test_rs16_any_k_m_round_trip_and_refusals(pkg, gpu):
    """forward_encode_kv / backwards_decode_kv at (k, m) = (16, 4) with four
    lost data shards, and the reference's m <= 16 limit on the reconstruct."""
    K = torch.randn(1, 4, 100, 128, device=gpu).to(torch.float16)
    V = torch.randn(1, 4, 100, 128, device=gpu).to(torch.float16)
    shards, meta = pkg.rs.forward_encode_kv(K, V, 16, 4)
    er = shards.clone()
    for x in (0, 5, 9, 15):
        er[x].view(torch.int16).fill_(-1)
    kr, vr = pkg.rs.backwards_decode_kv(er, meta, [0, 5, 9, 15])
    assert torch.equal(kr.view(torch.int16), K.view(torch.int16))
    assert torch.equal(vr.view(torch.int16), V.view(torch.int16))
    gex, glg = pkg.rs.device_gf_tables(gpu)
    idx = torch.arange(17, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="<= 16"):
        pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(torch.zeros((40, 8), dtype=torch.uint16, device=gpu), 8, 20,
                                                    20, idx, idx, gex, glg)


@pytest.mark.parametrize("k,S", [(6, 100), (6, 4096 * 2 + 3), (25, 300)])
def test_rs16_bad_device_indices_write_nothing(pkg, gpu, k, S):
    """A lost row outside the data rows, a repeated lost row, a parity row
    outside the tensor or a negative index: nothing is written (k = 6: rows
    under one tile on the piece kernel, longer rows on the tile kernel; k = 25
    with two lost rows: the Horner kernel)."""
    m = 2
    d = torch.zeros((k + m, S), dtype=torch.uint16, device=gpu)
    d.view(torch.int16).fill_(7)
    gex, glg = pkg.rs.device_gf_tables(gpu)
    cases = [([0, k + 3], [0, 1]), ([3, 3], [0, 1]), ([1, 2], [0, 2]), ([-1, 0], [0, 1]), ([2, 0], [-1, 1]),
             ([k, 1], [0, 1])]
    if k <= 8:
        cases += [([-1], [0]), ([2], [-1]), ([k], [0])]
    for miss, pu in cases:
        pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(
            d, S, k, m, torch.tensor(miss, dtype=torch.int32, device=gpu),
            torch.tensor(pu, dtype=torch.int32, device=gpu), gex, glg)
        assert bool((d.view(torch.int16) == 7).all()), (miss, pu)


@pytest.mark.parametrize("k,m", [(8, 2), (6, 2), (5, 3)])
def test_rs16_forward_backward_round_trip(pkg, ora, gpu, k, m):
    B, H, T, D = 1, 8, 63, 128
    K = torch.randn(B, H, T, D, device=gpu).to(torch.bfloat16)
    V = torch.randn(B, H, T, D, device=gpu).to(torch.bfloat16)
    shards, meta = pkg.rs.forward_encode_kv(K, V, k, m)
    assert set(meta) >= {"B", "H", "T", "D", "N_k", "N_v", "total", "pad", "shard_sz",
                         "num_data", "num_parity"}
    ex, lg = ora.gf16_tables()
    S = meta["shard_sz"]
    stream = np.zeros(k * S, np.uint16)
    stream[: meta["total"]] = np.concatenate([K.cpu().view(torch.uint16).numpy().reshape(-1),
                                              V.cpu().view(torch.uint16).numpy().reshape(-1)])
    assert np.array_equal(host(shards), ora.rs16_encode(stream, k, m, S, ex, lg))
    for missing in [[0, 1], [k - 1], [k, 2], [1, k + m - 1], [k, k + 1]][: m + 2]:
        if len([x for x in missing if x < k]) > m - len([x for x in missing if x >= k]):
            continue
        er = shards.clone()
        for x in missing:
            er[x].view(torch.int16).zero_()
        kr, vr = pkg.rs.backwards_decode_kv(er, meta, missing)
        assert torch.equal(kr.view(torch.int16), K.view(torch.int16)), missing
        assert torch.equal(vr.view(torch.int16), V.view(torch.int16)), missing
    with pytest.raises(RuntimeError):
        pkg.rs.backwards_decode_kv(shards.clone(), meta, list(range(m + 1)))


# ---------------------------------------------------- P/Q interior tiles
# Interior tiles of stripes with nd <= 8 data rows take a path that requests
# every row's chunk at once: cover every nd there, row tensors whose start is
# 0 or 6 bytes past a 16-byte boundary, rows of odd length (every row
# misaligned differently), star words inside interior tiles, no star skip,
# and fused backups whose K/V and V/padding boundaries cross interior tiles.
@pytest.mark.parametrize("nd", range(1, 9))
@pytest.mark.parametrize("soff", [0, 3])
@pytest.mark.parametrize("S,sb", [(12295, 4100), (10000, -1), (4096 * 4, 9000)])
def test_gs_parity_interior_tiles(pkg, ora, gpu, nd, soff, S, sb):
    rng = np.random.default_rng(nd * 131 + soff * 7 + S)
    rows = rng.integers(0, 65536, (nd + 2, S), dtype=np.uint16)
    want = rows.copy()
    ora.gs_parity(want, nd, S, sb)
    buf = torch.full(((nd + 2) * S + 16,), 0x3C3C, dtype=torch.int16, device=gpu)
    buf[soff:soff + (nd + 2) * S] = dev(rows.reshape(-1).view(np.int16), gpu)
    d = buf[soff:soff + (nd + 2) * S].view(nd + 2, S)
    pkg.rdp_kv_ops.compute_rdp_parity(d.view(torch.uint16), nd, S, sb)
    assert np.array_equal(d.cpu().numpy().view(np.uint16), want)
    assert bool((torch.cat([buf[:soff], buf[soff + (nd + 2) * S:]]) == 0x3C3C).all())


# The first tile of a stripe without K/V takes the same path; there thread 0's
# Q words i < r of row r wrap to row r's last words.  star_base S - 6 puts the
# skipped word of rows 3, 4 and 5 on a wrapped word (diagonals 0, 2 and 4),
# star_base 0 puts it on unwrapped words of thread 0, -1 skips nothing in row
# 0.  S = 4096 is a one-tile stripe (8 KiB rows) and S = 2048 half of one;
# 524288 words is a Llama-3.1-8B TP8 prefill step's [K | V] rows (2048 tokens
# x 128 words).
@pytest.mark.parametrize("nd", range(1, 9))
@pytest.mark.parametrize("soff", [0, 3])
@pytest.mark.parametrize("S,sb", [(2048, 2042), (2048 * 3 + 5, 0), (6000, -1), (4096, 4095),
                                  (4096 * 2 + 3, 4096 * 2 - 3)])
def test_gs_parity_first_tile(pkg, ora, gpu, nd, soff, S, sb):
    rng = np.random.default_rng(nd * 29 + soff * 3 + S + sb)
    rows = rng.integers(0, 65536, (nd + 2, S), dtype=np.uint16)
    want = rows.copy()
    ora.gs_parity(want, nd, S, sb)
    buf = torch.full(((nd + 2) * S + 16,), 0x3C3C, dtype=torch.int16, device=gpu)
    buf[soff:soff + (nd + 2) * S] = dev(rows.reshape(-1).view(np.int16), gpu)
    d = buf[soff:soff + (nd + 2) * S].view(nd + 2, S)
    pkg.rdp_kv_ops.compute_rdp_parity(d.view(torch.uint16), nd, S, sb)
    assert np.array_equal(d.cpu().numpy().view(np.uint16), want)
    assert bool((torch.cat([buf[:soff], buf[soff + (nd + 2) * S:]]) == 0x3C3C).all())


@pytest.mark.parametrize("sb", [0, 524288 - 6])
def test_gs_parity_plugin_step_shape(pkg, ora, gpu, sb):
    nd, S = 8, 2 * 2048 * 128
    rng = np.random.default_rng(sb + 1)
    rows = np.zeros((nd + 2, S), dtype=np.uint16)
    rows[:nd] = rng.integers(0, 65536, (nd, S), dtype=np.uint16)
    want = rows.copy()
    ora.gs_parity(want, nd, S, sb)
    d = dev(rows, gpu)
    pkg.rdp_kv_ops.compute_rdp_parity(d, nd, S, sb)
    assert np.array_equal(d.cpu().numpy(), want)


@pytest.mark.parametrize("nd", range(1, 9))
@pytest.mark.parametrize("soff,S_extra", [(0, 0), (5, 2500), (3, 7000)])
def test_gs_backup_interior_tiles(pkg, ora, gpu, nd, soff, S_extra):
    T, n, sb = 192, 211, 2050     # rows of at least two 8 KiB tiles for every nd
    tn = T * n
    S = -(-2 * tn // nd) + S_extra
    koff, voff = soff, (soff + tn) % 8      # the alignment the fused pack needs
    rng = np.random.default_rng(nd * 17 + soff)
    K = rng.integers(0, 65536, tn, dtype=np.uint16)
    V = rng.integers(0, 65536, tn, dtype=np.uint16)
    init = np.zeros((nd + 2, S), dtype=np.uint16)
    want = init.copy()
    ora.gs_pack(K.reshape(T, n), V.reshape(T, n), want, nd, S, T, n)
    ora.gs_parity(want, nd, S, sb)
    kb = torch.zeros(tn + 16, dtype=torch.int16, device=gpu)
    vb = torch.zeros(tn + 16, dtype=torch.int16, device=gpu)
    kb[koff:koff + tn] = dev(K.view(np.int16), gpu)
    vb[voff:voff + tn] = dev(V.view(np.int16), gpu)
    sbuf = torch.full(((nd + 2) * S + 16,), 0x5A5A, dtype=torch.int16, device=gpu)
    sbuf[soff:soff + (nd + 2) * S] = 0
    sh = sbuf[soff:soff + (nd + 2) * S].view(nd + 2, S)
    pkg.rdp.rdp_kernel.fused_backup_full_kv(kb[koff:koff + tn].view(T, n), vb[voff:voff + tn].view(T, n),
                                            sh.view(torch.uint16), nd, S, T, n, sb)
    assert np.array_equal(sh.cpu().numpy().view(np.uint16), want)
    assert bool((torch.cat([sbuf[:soff], sbuf[soff + (nd + 2) * S:]]) == 0x5A5A).all())


# The fused first tile of an aligned row tensor takes the batched path too:
# star words on thread 0's wrapped words (star_base S - 6), and rows whose last
# 16 bytes lie in K, in V, in the padding or across the K/V or V/padding
# boundary (nd = 2 with no padding ends row 0 exactly at the K/V boundary).
@pytest.mark.parametrize("nd", range(1, 9))
@pytest.mark.parametrize("T,n,S_extra,sb_back", [(96, 211, 0, 6), (64, 128, 0, None), (50, 77, 1000, 6)])
def test_gs_backup_first_tile(pkg, ora, gpu, nd, T, n, S_extra, sb_back):
    tn = T * n
    S = -(-2 * tn // nd) + S_extra
    sb = 0 if sb_back is None else S - sb_back
    rng = np.random.default_rng(nd * 41 + T + n)
    K = rng.integers(0, 65536, tn, dtype=np.uint16)
    V = rng.integers(0, 65536, tn, dtype=np.uint16)
    want = np.zeros((nd + 2, S), dtype=np.uint16)
    ora.gs_pack(K.reshape(T, n), V.reshape(T, n), want, nd, S, T, n)
    ora.gs_parity(want, nd, S, sb)
    voff = tn % 8                           # V aligned like its place in the rows
    kb = dev(K.view(np.int16), gpu)
    vb = torch.zeros(tn + 16, dtype=torch.int16, device=gpu)
    vb[voff:voff + tn] = dev(V.view(np.int16), gpu)
    sh = torch.zeros((nd + 2, S), dtype=torch.uint16, device=gpu)
    pkg.rdp.rdp_kernel.fused_backup_full_kv(kb.view(T, n), vb[voff:voff + tn].view(T, n), sh, nd, S, T,
                                            n, sb)
    assert np.array_equal(sh.cpu().numpy(), want)


def test_gs_backup_reference_demo_shape(pkg, ora, gpu):
    """benchmark/rdp/main.py defaults: B=1, 8 heads, T=512, head_dim 128, 8 shards."""
    torch.manual_seed(0)
    keys = torch.randn(1, 8, 512, 128, device=gpu, dtype=torch.float16)
    values = torch.randn(1, 8, 512, 128, device=gpu, dtype=torch.float16)
    out = pkg.rdp.fused_backup_full_kv(keys, values, 8, star_base=0)
    K_TN = keys.permute(2, 0, 1, 3).reshape(512, -1).cpu().numpy().view(np.uint16)
    V_TN = values.permute(2, 0, 1, 3).reshape(512, -1).cpu().numpy().view(np.uint16)
    assert np.array_equal(out["shards_KV"].cpu().numpy(), ora.gs_backup(K_TN, V_TN, 8, 0))
