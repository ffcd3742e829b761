"""The C-ABI library loads on a CPU-only host, exports every symbol that
include/kvec.h declares, and rejects bad arguments before touching a device."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "kvec.h")


@pytest.fixture
def fake_ptrs():
    """Tests that pass made-up device addresses expect every call to fail on
    the host before any launch.  Should one pass its checks by mistake, its
    launch must not reach a real GPU: they run only where none is visible."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("made-up device addresses: CPU-only test")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvec_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported(pkg):
    L = pkg._lib.lib()
    names = declared_symbols()
    assert len(names) >= 5
    for n in names:
        assert hasattr(L, n), f"{n} declared in kvec.h but not exported"
    # the ctypes signature table covers exactly the header
    assert sorted(pkg._lib.SIGNATURES) == names


def test_status_strings(pkg):
    L = pkg._lib.lib()
    hdr = open(os.path.join(ROOT, "include", "kvec.h")).read()
    want = int(re.search(r"#define KVEC_VERSION (\d+)", hdr).group(1))
    assert L.kvec_version() == want
    assert pkg._lib.ABI_MAJOR == want // 10000
    assert L.kvec_strerror(0) == b"success"
    assert L.kvec_strerror(-1) == b"invalid argument"


def test_fastdiv_exact(pkg):
    L = C.CDLL(pkg._lib.LIB_PATH)
    f = L.kvec_internal_fastdiv
    f.restype = C.c_uint32
    f.argtypes = [C.c_uint32, C.c_uint32]
    rng = np.random.default_rng(0)
    divisors = [1, 2, 3, 5, 7, 16, 255, 256, 257, 2048, 32768, 65535, 65536, 1 << 31,
                (1 << 31) + 1, (1 << 32) - 1] + [int(x) for x in rng.integers(1, 1 << 32, 40)]
    for d in divisors:
        ns = [0, 1, d - 1, d, d + 1, (1 << 32) - 1, (1 << 32) - 2] + \
             [int(x) for x in rng.integers(0, 1 << 32, 200)]
        for n in ns:
            n &= 0xFFFFFFFF
            assert f(n, d) == n // d, (n, d)


def test_rdp_row_bytes(pkg):
    spec = pkg.spec
    # 512 MiB over k=6, p=7 -> 36 row planes, rounded up to 256 B
    R = spec.rdp_row_bytes(1 << 29, 6, 7, 256)
    assert R % 256 == 0 and 36 * R >= 1 << 29 and 36 * (R - 256) < 1 << 29
    assert spec.rdp_row_bytes(0, 6, 7) == 0
    assert spec.rdp_row_bytes(1, 2, 3, 16) == 16


def test_rdp_rejects_bad_arguments(pkg, fake_ptrs):
    L = pkg._lib.lib()
    arr = (C.c_void_p * 6)(*([16] * 6))
    assert L.kvec_rdp_encode(arr, 6, 16, 16, 4, 16, 0, None) == -1   # p not prime
    assert L.kvec_rdp_encode(arr, 7, 16, 16, 7, 16, 0, None) == -1   # k > p-1
    assert L.kvec_rdp_encode(arr, 6, 16, 16, 7, 24, 0, None) == -1   # row_bytes % 16
    assert L.kvec_rdp_encode(arr, 6, 16, 16, 17, 16, 0, None) == -2  # p too large
    assert b"p=17" in L.kvec_last_error()
    bad = (C.c_void_p * 6)(*([16] * 5 + [8]))
    assert L.kvec_rdp_encode(bad, 6, 16, 16, 7, 16, 0, None) == -1   # misaligned shard
    assert b"aligned" in L.kvec_last_error()
    assert L.kvec_rdp_decode(arr, 4, 5, 16, 0, 7, -1, None) == -1    # erased index > k+1
    # the stripe unit is 0 or a positive multiple of 1024
    assert L.kvec_rdp_encode(arr, 6, 16, 16, 7, 4096, 512, None) == -1
    assert b"unit_bytes" in L.kvec_last_error()
    assert L.kvec_rdp_encode(arr, 6, 16, 16, 7, 4096, -1024, None) == -1
    assert L.kvec_rdp_decode(arr, 4, 5, 4096, 1000, 0, -1, None) == -1


def test_xor_one_call_entries_reject_bad_arguments(pkg, fake_ptrs):
    """kvec_xor_encode_kv / kvec_xor_recover_kv validate sizes and pointers
    before any device call (the pointers below are never dereferenced)."""
    L = pkg._lib.lib()
    p = 4096
    # K and V larger than the data rows
    assert L.kvec_xor_encode_kv(p, p, 100, p, 2, 99, None) == -1
    assert b"exceed" in L.kvec_last_error()
    assert L.kvec_xor_encode_kv(p, p, 16, p, 0, 64, None) == -1        # no data shards
    assert L.kvec_xor_encode_kv(None, p, 16, p, 2, 64, None) == -1     # null K
    assert b"null" in L.kvec_last_error()
    assert L.kvec_xor_encode_kv(p, p, 0, p, 2, 0, None) == 0           # empty: nothing to do
    # recovery: missing index past P, output longer than the data rows, null output
    assert L.kvec_xor_recover_kv(p, p, 3, 64, 16, 4, None) == -1
    assert L.kvec_xor_recover_kv(p, p, 3, 64, 3 * 64 + 1, 0, None) == -1
    assert b"exceed" in L.kvec_last_error()
    assert L.kvec_xor_recover_kv(p, None, 3, 64, 16, 0, None) == -1
    assert L.kvec_xor_recover_kv(p, p, 3, 0, 0, 1, None) == 0          # empty rows


def test_pack_unpack_reject_bad_arguments(pkg, fake_ptrs):
    """xor_kernel.pack_kv / unpack_kv (benchmark/xor/kernel.cu:193-223): negative
    sizes and null pointers are refused on the host; zero words is a no-op."""
    L = pkg._lib.lib()
    p = 4096
    assert L.kvec_pack_kv(p, p, p, -1, 4, None) == -1
    assert L.kvec_pack_kv(p, p, p, 4, -2, None) == -1
    assert b"seq_len=-2" in L.kvec_last_error()
    assert L.kvec_pack_kv(None, p, p, 4, 4, None) == -1
    assert L.kvec_pack_kv(p, p, None, 4, 4, None) == -1
    assert b"null" in L.kvec_last_error()
    assert L.kvec_pack_kv(None, None, None, 0, 4, None) == 0
    assert L.kvec_unpack_kv(p, p, -1, 4, None) == -1
    assert L.kvec_unpack_kv(None, p, 4, 4, None) == -1
    assert L.kvec_unpack_kv(p, None, 4, 4, None) == -1
    assert L.kvec_unpack_kv(None, None, 4, 0, None) == 0


def test_copy_entries_reject_partial_overlap(pkg, fake_ptrs):
    """Entry points that copy the caller's data rows into the shard tensor
    accept the same buffer (no copy) or disjoint ones; a partial overlap has no
    stream-ordered meaning and is refused before any launch."""
    L = pkg._lib.lib()
    base, S = 1 << 20, 4096
    ex = lg = 4096
    # RS16: data_padded is k*S words; shards + one row overlaps it
    assert L.kvec_rs16_encode(base + 2 * S, base, 4, 2, S, ex, lg, None) == -1
    assert b"overlap" in L.kvec_last_error()
    # XOR: data rows [base + S, +4S) against the shard tensor at base
    assert L.kvec_xor_encode(base + S, base, 4, S, None) == -1
    assert b"overlap" in L.kvec_last_error()


def test_rs16_encode_limits(pkg, fake_ptrs):
    """The GF(2^16) encode takes every k >= 1 and m >= 0 whose exponents
    (p + 1) i fit the reference's int (benchmark/rs/kernel.cu:93); beyond that,
    KVEC_EUNSUPPORTED before any launch.  (k * m beyond 48 is no limit.)"""
    L = pkg._lib.lib()
    base, S = 1 << 20, 8
    ex = lg = 4096
    assert L.kvec_rs16_encode(base, base + (1 << 30), (1 << 16) + 1, 1 << 15, S, ex, lg, None) == -2
    assert b"out of range" in L.kvec_last_error()
    assert L.kvec_rs16_encode(base, base + (1 << 30), 2, 524281, S, ex, lg, None) == -2
    assert L.kvec_rs16_encode(base, base + (1 << 30), 0, 2, S, ex, lg, None) == -1
    # a valid shape with nothing to code (S = 0) returns before any launch
    assert L.kvec_rs16_encode(base, base + (1 << 30), 25, 2, 0, ex, lg, None) == 0
    assert L.kvec_rs16_encode(base, base + (1 << 30), 16, 16, 0, ex, lg, None) == 0


def test_gs_recover_refuses_negative_star_column(pkg, fake_ptrs):
    """Two lost rows with (star_base + a) % S < 0 (C's %, a the lower row):
    the reference's fill_a_star_from_P (benchmark/rdp/kernel.cu:268-282)
    would read and write outside row a, so the call is refused before any
    launch, whatever order the two rows are given in."""
    L = pkg._lib.lib()
    base, nd, S = 1 << 20, 6, 1000
    for sb, a, b in [(-1, 0, 3), (-3, 2, 1), (-1001, 4, 5), (-5, 5, 4)]:
        assert L.kvec_gs_rdp_recover(base, None, nd, S, 0, 0, sb, a, b, None) == -1, (sb, a, b)
        assert b"star_base" in L.kvec_last_error()


def test_loader_refuses_other_abi_major(pkg, monkeypatch):
    """A library whose major version differs from the one the bindings mirror
    is refused at load, before any call with mismatched arguments."""
    monkeypatch.setattr(pkg._lib, "_lib", None)
    monkeypatch.setattr(pkg._lib, "ABI_MAJOR", pkg._lib.ABI_MAJOR + 1)
    with pytest.raises(RuntimeError, match="ABI version"):
        pkg._lib.lib()


def test_product_fails_loudly_without_library(pkg, monkeypatch, tmp_path):
    monkeypatch.setattr(pkg._lib, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(pkg._lib, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        pkg._lib.lib()


def test_chunk_width(pkg):
    L = pkg._lib.lib()
    # 16 x 2048 tokens x 32 layers x 256 B records (fp8, 1 head x 128) over k=5, p=7
    n = 16 * 2048 * 32 * 256
    W = L.kvec_chunk_width(n, 5, 7, 256)
    assert W % 256 == 0 and 30 * W >= n and 30 * (W - 256) < n
    assert L.kvec_chunk_width(n, 5, 7, 24) == -1
    assert L.kvec_chunk_width(-1, 5, 7, 256) == -1


def test_chunk_rejects_bad_arguments(pkg, fake_ptrs):
    """Argument checks run on the host before any launch (fake aligned pointers)."""
    lib = pkg._lib
    L = lib.lib()
    G = 1 << 30  # disjoint fake buffers: pool, table, P, Q, RS parity
    kv = lib.PagedKV(G, 64, 2, 128, 16, 2 * G, 3, 4, 0, 16)
    rs = (C.c_void_p * 3)(5 * G, 6 * G, 7 * G)

    def stripe(**kw):
        a = dict(data=None, k=5, P=3 * G, Q=4 * G, p=7, rs=C.cast(rs, C.POINTER(C.c_void_p)),
                 m=3, row_bytes=1 << 20, region_off=0, width=256 * 64, unit_bytes=65536)
        a.update(kw)
        return lib.ChunkStripe(a["data"], a["k"], a["P"], a["Q"], a["p"], a["rs"], a["m"],
                               a["row_bytes"], a["region_off"], a["width"], a["unit_bytes"])

    def rc(**kw):
        return L.kvec_chunk_encode_paged(C.byref(kv), C.byref(stripe(**kw)), None)

    assert rc(p=9) == -1                       # not prime
    assert rc(k=7) == -1                       # k > p-1
    assert rc(width=250) == -1                 # not a record multiple
    assert rc(region_off=8) == -1              # misaligned region
    assert rc(region_off=6 * (1 << 20) - 256) == -1   # region past the shard
    assert b"region_off" in L.kvec_last_error()
    assert rc(unit_bytes=1536) == -1           # a record multiple, not a 1 KiB one
    assert rc(unit_bytes=-1024) == -1
    assert rc(width=256) == -1                 # cells too small for the chunk
    assert b"k*(p-1)*width" in L.kvec_last_error()
    assert rc(P=3 * G + 4) == -1               # misaligned parity
    assert rc(m=5) == -1
    assert rc(row_bytes=1 << 30) == -2         # (p-1)*R >= 4 GiB
    assert b"4 GiB" in L.kvec_last_error()
    er = (C.c_int32 * 1)(10)
    assert L.kvec_chunk_decode_paged(C.byref(kv), G, C.byref(stripe()), er, 1, None) == -1
    assert b"erased index 10" in L.kvec_last_error()
    assert L.kvec_chunk_decode_paged(C.byref(kv), 8 * G, C.byref(stripe()), er, 0, None) == -1
    assert b"kv->pool" in L.kvec_last_error()


def test_written_buffers_must_not_alias(pkg, fake_ptrs):
    """Every spec entry point refuses, before any launch, a buffer it writes
    that shares a byte with another buffer of the call: its kernels read
    their inputs while other blocks of the same launch write the outputs.
    Fake addresses; nothing is dereferenced and every call below fails."""
    lib = pkg._lib
    L = lib.lib()
    G = 1 << 30
    R = 4096
    nb = 6 * R

    def err():
        return L.kvec_last_error().decode()

    data = (C.c_void_p * 6)(*[G * (j + 1) for j in range(6)])
    assert L.kvec_rdp_encode(data, 6, 3 * G + 1024, 9 * G, 7, R, 0, None) == -1
    assert "P overlaps data[2]" in err()
    assert L.kvec_rdp_encode(data, 6, 8 * G, 8 * G + nb - 16, 7, R, 65536, None) == -1
    assert "P overlaps Q" in err()
    sh = (C.c_void_p * 8)(*[G * (j + 1) for j in range(6)] + [8 * G, 9 * G])
    sh[4] = 2 * G + nb - 16                     # lost shard 4 ends inside shard 1
    assert L.kvec_rdp_decode(sh, 6, 7, R, 0, 4, -1, None) == -1
    assert "shard[4] overlaps shard[1]" in err()
    assert L.kvec_rdp_decode(sh, 6, 7, R, 0, 7, 4, None) == -1

    par = (C.c_void_p * 2)(8 * G, G + 16)
    assert L.kvec_rs8_encode(data, 6, par, 2, R, None) == -1
    assert "parity[1] overlaps data[0]" in err()
    rs_sh = (C.c_void_p * 8)(*[G * (j + 1) for j in range(8)])
    rs_sh[5] = rs_sh[2]
    er = (C.c_int32 * 1)(2)
    assert L.kvec_rs8_decode(rs_sh, 6, 2, R, er, 1, None) == -1
    assert "shard[2] overlaps shard[5]" in err()

    # paged: 2 layers x 3 sequences x 16 tokens of 256-byte records
    pool, table = 20 * G, 21 * G
    kv = lib.PagedKV(pool, 64, 2, 128, 16, table, 3, 4, 0, 16)
    assert L.kvec_kv_gather(C.byref(kv), pool + 256, None) == -1
    assert "out overlaps pool" in err()
    assert L.kvec_kv_gather_split(C.byref(kv), 22 * G, table, None) == -1
    assert "out_v overlaps page_table" in err()
    assert L.kvec_kv_scatter(C.byref(kv), pool, pool + 512, None) == -1
    assert "pool overlaps in" in err()
    Rp = 768
    assert L.kvec_rdp_encode_paged(C.byref(kv), data, 6, pool + 4096, 9 * G, 7, Rp, 0, None) == -1
    assert "P overlaps pool" in err()
    dd = (C.c_void_p * 6)(*[G * (j + 1) for j in range(6)])
    dd[3] = 8 * G
    assert L.kvec_rdp_decode_paged(C.byref(kv), pool, dd, 6, 8 * G, 9 * G, 7, Rp, 0, 1, 3,
                                   None) == -1
    assert "P overlaps data[3]" in err()
    assert L.kvec_rdp_decode_paged(C.byref(kv), pool, None, 6, table, 9 * G, 7, Rp, 0, 1, -1,
                                   None) == -1
    assert "P overlaps page_table" in err()

    # chunked: an RS parity shard inside Q; a decode's pool inside P
    rs = (C.c_void_p * 3)(5 * G, 4 * G + 4096, 7 * G)
    ck = lib.PagedKV(G, 64, 2, 128, 16, 2 * G, 3, 4, 0, 16)
    st = lib.ChunkStripe(None, 5, 3 * G, 4 * G, 7, C.cast(rs, C.POINTER(C.c_void_p)), 3, 1 << 20,
                         0, 256 * 64, 65536)
    assert L.kvec_chunk_encode_paged(C.byref(ck), C.byref(st), None) == -1
    assert "Q overlaps rs[1]" in err()
    rs[1] = 6 * G
    ck2 = lib.PagedKV(3 * G + 4096, 64, 2, 128, 16, 2 * G, 3, 4, 0, 16)
    er2 = (C.c_int32 * 1)(0)
    assert L.kvec_chunk_decode_paged(C.byref(ck2), 3 * G + 4096, C.byref(st), er2, 1, None) == -1
    assert "pool overlaps P" in err()


def test_build_rejects_register_spills():
    """The build refuses kernels whose resource-usage remarks report spilled
    SGPRs or VGPRs; scratch without spills (a run-time indexed array) passes."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "_kvec_build_t", os.path.join(ROOT, "26mlsys-ae-ghostserve_amd", "_build.py"))
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    rem = "\n".join([
        "x.hip:1:1: remark: Function Name: k_ok [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     SGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:1:1: remark:     ScratchSize [bytes/lane]: 528 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:2:1: remark: Function Name: k_s [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:2:1: remark:     SGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:2:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:3:1: remark: Function Name: k_v [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:3:1: remark:     SGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:3:1: remark:     VGPRs Spill: 68 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert b.register_spills(rem) == [("k_s", "SGPRs", 3), ("k_v", "VGPRs", 68)]
