"""numpy front end of the CPU oracle (oracle/kvec_oracle.c).

TEST INFRASTRUCTURE ONLY.  The HIP kernels are compared against this
module; only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py import it.  The product package never does.

Every function takes and returns numpy arrays and mirrors one C entry point of
kvec_oracle.c, which cites the reference lines it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libkvec_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    args = ["make", "-C", _HERE]
    if force:
        args.append("-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = C.CDLL(_SO)
        _declare(_lib)
    return _lib


P = C.c_void_p
I = C.c_int
I64 = C.c_int64


def _declare(L):
    sig = {
        "kvo_gf16_tables": (None, [P, P]),
        "kvo_gf8_tables": (None, [P, P]),
        "kvo_gf8_mul": (C.c_uint8, [C.c_uint8, C.c_uint8]),
        "kvo_gf8_inv": (C.c_uint8, [C.c_uint8]),
        "kvo_rs8_cauchy": (I, [I, I, P]),
        "kvo_xor_encode": (None, [P, P, I, I64]),
        "kvo_xor_reconstruct": (None, [P, P, P, I64, I, P, I]),
        "kvo_pack_kv": (None, [P, P, P, I, I]),
        "kvo_unpack_kv": (None, [P, P, I, I]),
        "kvo_gs_pack": (None, [P, P, P, I, I, I, I]),
        "kvo_gs_parity": (None, [P, I, I, I]),
        "kvo_gs_recover": (None, [P, I, I, I, I, I]),
        "kvo_gs_load_full": (None, [P, P, I, I, I, I]),
        "kvo_gs_pack_row": (I, [P, P, P, I64, I, I]),
        "kvo_rs16_encode": (None, [P, P, I, I, I64, P, P]),
        "kvo_rs16_reconstruct": (I, [P, I64, I, I, P, I, P, P, P]),
        "kvo_rdp_encode": (I, [P, I, P, P, I, I64]),
        "kvo_rdp_decode": (I, [P, I, I, I64, I, I]),
        "kvo_rdp_encode_striped": (I, [P, I, P, P, I, I64, I64]),
        "kvo_rdp_decode_striped": (I, [P, I, I, I64, I64, I, I]),
        "kvo_rs8_encode": (I, [P, I, P, I, I64]),
        "kvo_rs8_decode": (I, [P, I, I, I64, P, I]),
        "kvo_kv_gather": (I, [P, I64, I, I64, I, P, I, I, I, I, P]),
        "kvo_num_threads": (I, []),
        "kvo_set_num_threads": (None, [I]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _ptrs(arrs):
    return (C.c_void_p * len(arrs))(*[_p(a) for a in arrs])


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} failed with code {rc}")


def num_threads() -> int:
    return lib().kvo_num_threads()


def set_num_threads(n: int) -> None:
    lib().kvo_set_num_threads(int(n))


# ----------------------------- Galois fields -----------------------------
def gf16_tables():
    ex = np.zeros(2 * 65535, np.uint16)
    lg = np.zeros(65536, np.uint16)
    lib().kvo_gf16_tables(_p(ex), _p(lg))
    return ex, lg


def gf8_tables():
    ex = np.zeros(510, np.uint8)
    lg = np.zeros(256, np.uint8)
    lib().kvo_gf8_tables(_p(ex), _p(lg))
    return ex, lg


def gf8_mul(a: int, b: int) -> int:
    return int(lib().kvo_gf8_mul(a, b))


def gf8_inv(a: int) -> int:
    return int(lib().kvo_gf8_inv(a))


def rs8_cauchy(k: int, m: int) -> np.ndarray:
    c = np.zeros((m, k), np.uint8)
    _check(lib().kvo_rs8_cauchy(k, m, _p(c)), "rs8_cauchy")
    return c


# ----------------------------- gs: XOR -----------------------------
def xor_encode(data_padded: np.ndarray, data_shards: int, shard_size: int) -> np.ndarray:
    shards = np.zeros((data_shards + 1, shard_size), np.uint8)
    lib().kvo_xor_encode(_p(data_padded), _p(shards), data_shards, shard_size)
    return shards


def xor_reconstruct(shards: np.ndarray, shard_size: int, data_shards: int, missing):
    """In place on ``shards`` like the reference call at benchmark/xor/main.py:174-177.
    Returns the ``recovered_missing`` row."""
    miss = np.asarray(missing, np.int32)
    rec_missing = np.zeros((1, shard_size), np.uint8)
    lib().kvo_xor_reconstruct(_p(shards), _p(shards), _p(rec_missing), shard_size,
                              data_shards, _p(miss) if miss.size else None, int(miss.size))
    return rec_missing


def pack_kv(k16: np.ndarray, v16: np.ndarray, n: int, seq_len: int) -> np.ndarray:
    out = np.zeros(4 * n * seq_len, np.uint8)
    lib().kvo_pack_kv(_p(k16), _p(v16), _p(out), n, seq_len)
    return out


def unpack_kv(kv_bytes: np.ndarray, n: int, seq_len: int) -> np.ndarray:
    out = np.zeros(2 * n * seq_len, np.uint16)
    lib().kvo_unpack_kv(_p(kv_bytes), _p(out), n, seq_len)
    return out


# ----------------------------- gs: RDP -----------------------------
def gs_pack(K_TN, V_TN, shards, nd, S, T, n):
    lib().kvo_gs_pack(_p(K_TN), _p(V_TN), _p(shards), nd, S, T, n)


def gs_parity(shards, nd, S, star_base):
    lib().kvo_gs_parity(_p(shards), nd, S, star_base)


def gs_recover(shards, nd, S, star_base, miss_a, miss_b):
    lib().kvo_gs_recover(_p(shards), nd, S, star_base, miss_a, miss_b)


def gs_load_full(shards, nd, S, T, n) -> np.ndarray:
    out = np.zeros(2 * T * n, np.uint16)
    lib().kvo_gs_load_full(_p(shards), _p(out), nd, S, T, n)
    return out


def gs_pack_row(k, v, rows, row):
    _check(lib().kvo_gs_pack_row(_p(k), _p(v), _p(rows), k.size, row, rows.shape[1]),
           "gs_pack_row")


def gs_backup(K_TN: np.ndarray, V_TN: np.ndarray, nd: int, star_base: int = 0):
    """Whole fused_backup_full_kv (benchmark/rdp/main.py:44-92 + kernel.cu:366-395)
    on [T, n] uint16 arrays; returns the [(nd+2), S] shard matrix."""
    T, n = K_TN.shape
    total = 2 * T * n
    pad = (nd - total % nd) % nd
    S = (total + pad) // nd
    shards = np.zeros((nd + 2, S), np.uint16)
    gs_pack(np.ascontiguousarray(K_TN), np.ascontiguousarray(V_TN), shards, nd, S, T, n)
    gs_parity(shards, nd, S, star_base)
    return shards


# ----------------------------- gs: RS16 -----------------------------
def rs16_encode(data_padded, k, m, S, ex, lg) -> np.ndarray:
    shards = np.zeros((k + m, S), np.uint16)
    lib().kvo_rs16_encode(_p(data_padded), _p(shards), k, m, S, _p(ex), _p(lg))
    return shards


def rs16_reconstruct(shards, S, k, m, missing_data, parity_used, ex, lg):
    md = np.asarray(missing_data, np.int32)
    pu = np.asarray(parity_used, np.int32)
    _check(lib().kvo_rs16_reconstruct(_p(shards), S, k, m, _p(md) if md.size else None,
                                      int(md.size), _p(pu) if pu.size else None,
                                      _p(ex), _p(lg)), "rs16_reconstruct")


# ----------------------------- spec: RDP -----------------------------
def rdp_encode(data, p: int, unit: int = 0, out=None):
    """data: list of k shard arrays of (p-1)*R bytes (shaped [(p-1), R] or
    flat).  unit = 0: p-1 row planes of R bytes; else stripes of (p-1)*unit
    bytes (rows of min(unit, R - s*unit) bytes).  Returns (P, Q) shaped like
    data[0], written into ``out`` = (P, Q) when given."""
    k = len(data)
    R = data[0].size // (p - 1)
    if out is None:
        P_ = np.zeros(data[0].shape, np.uint8)
        Q_ = np.zeros(data[0].shape, np.uint8)
    else:
        P_, Q_ = out
    _check(lib().kvo_rdp_encode_striped(_ptrs(data), k, _p(P_), _p(Q_), p, R, int(unit)),
           "rdp_encode")
    return P_, Q_


def rdp_decode(cols, p: int, e0: int, e1: int = -1, unit: int = 0):
    """cols: k data + P + Q shard arrays (as rdp_encode); erased ones are
    rewritten in place."""
    k = len(cols) - 2
    R = cols[0].size // (p - 1)
    _check(lib().kvo_rdp_decode_striped(_ptrs(cols), k, p, R, int(unit), e0, e1), "rdp_decode")


# ----------------------------- spec: RS8 -----------------------------
def rs8_encode(data, m: int, out=None):
    k = len(data)
    S = data[0].size
    par = [np.zeros(S, np.uint8) for _ in range(m)] if out is None else out
    _check(lib().kvo_rs8_encode(_ptrs(data), k, _ptrs(par), m, S), "rs8_encode")
    return par


def rs8_decode(shards, k: int, m: int, erased):
    S = shards[0].size
    er = np.asarray(list(erased), np.int32)
    _check(lib().kvo_rs8_decode(_ptrs(shards), k, m, S, _p(er) if er.size else None,
                                int(er.size)), "rs8_decode")


# ----------------------------- paged gather -----------------------------
def kv_gather(pool: np.ndarray, page_table: np.ndarray, page_tokens: int, tok_off: int,
              T: int) -> np.ndarray:
    """pool: [L, pool_pages, page_tokens, 2, tok_bytes] uint8;
    page_table: [B, pps] int32.  Returns stream [L, B, T, 2, tok_bytes]."""
    L, pool_pages, pt_, two, tb = pool.shape
    assert pt_ == page_tokens and two == 2
    B, pps = page_table.shape
    out = np.zeros((L, B, T, 2, tb), np.uint8)
    pt = np.ascontiguousarray(page_table, np.int32)
    _check(lib().kvo_kv_gather(_p(pool), pool_pages, L, tb, page_tokens, _p(pt), B, pps,
                               tok_off, T, _p(out)), "kv_gather")
    return out


# ----------------------------- chunked coding -----------------------------
# No reference function: the reference codes each prefill step's KV on the
# serving path (bench_ghostserve_rdp.py:334-392, gather at :445-458).  These
# compose the gather, RDP and RS8 oracles above with the chunk layout.
def chunk_width(chunk_stream_bytes: int, k: int, p: int, record_bytes: int) -> int:
    """Smallest multiple of record_bytes whose k*(p-1) cells hold the chunk."""
    cells = k * (p - 1)
    per = -(-chunk_stream_bytes // cells)
    return -(-per // record_bytes) * record_bytes


def chunk_cells(stream: np.ndarray, k: int, p: int, width: int) -> np.ndarray:
    """One chunk's stream, zero padded to k*(p-1)*width bytes, as its k data
    shard pieces [k, (p-1)*width]."""
    flat = np.zeros(k * (p - 1) * width, np.uint8)
    flat[: stream.size] = stream.reshape(-1)
    return flat.reshape(k, (p - 1) * width)


def chunked_encode(pool: np.ndarray, page_table: np.ndarray, page_tokens: int,
                   chunk_tokens: int, n_chunks: int, k: int, p: int, m: int, unit: int = 0):
    """Whole-sequence stripes of a paged pool coded chunk by chunk.

    Chunk c (positions c*chunk_tokens.. of every sequence) is gathered, zero
    padded and cut into k pieces of (p-1)*width bytes; piece j is data shard
    j's region c, at byte c*(p-1)*width.  Each region is its own RDP stripe set
    (rows of width bytes, stripe unit ``unit``), coded with RDP(p) and the m RS
    parities.  Returns (width, data [k flat shards], P, Q, rs [m flat shards])."""
    tb = pool.shape[-1]
    rec = 2 * tb
    L = pool.shape[0]
    B = page_table.shape[0]
    width = chunk_width(L * B * chunk_tokens * rec, k, p, rec)
    n = (p - 1) * width
    data = [np.zeros(n_chunks * n, np.uint8) for _ in range(k)]
    P_ = np.zeros(n_chunks * n, np.uint8)
    Q_ = np.zeros(n_chunks * n, np.uint8)
    rs = [np.zeros(n_chunks * n, np.uint8) for _ in range(m)]
    for c in range(n_chunks):
        s = kv_gather(pool, page_table, page_tokens, c * chunk_tokens, chunk_tokens)
        cells = chunk_cells(s, k, p, width)
        reg = slice(c * n, (c + 1) * n)
        for j in range(k):
            data[j][reg] = cells[j]
        rdp_encode([d[reg] for d in data], p, unit, out=(P_[reg], Q_[reg]))
        rs8_encode([d[reg] for d in data], m, out=[x[reg] for x in rs])
    return width, data, P_, Q_, rs
