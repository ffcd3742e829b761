"""Independent Galois-field arithmetic for the tests.

Products are computed by carry-less (shift-and-XOR) multiplication followed by
polynomial reduction, with no log/exp tables, so a table-building mistake in
the oracle or the kernels cannot cancel out here.
"""
import numpy as np


def clmul_mod(a, b, poly: int, bits: int):
    """Vectorised carry-less product of a and b reduced modulo poly (degree bits)."""
    a = np.asarray(a, np.uint64)
    b = np.asarray(b, np.uint64)
    acc = np.zeros(np.broadcast(a, b).shape, np.uint64)
    for i in range(bits):
        acc ^= np.where((b >> np.uint64(i)) & np.uint64(1), a << np.uint64(i), np.uint64(0))
    for i in range(2 * bits - 2, bits - 1, -1):
        hit = (acc >> np.uint64(i)) & np.uint64(1)
        acc ^= np.where(hit, np.uint64(poly) << np.uint64(i - bits), np.uint64(0))
    return acc


def gf8_mul_table() -> np.ndarray:
    """256 x 256 table of products in GF(2^8) modulo 0x11D."""
    a = np.arange(256, dtype=np.uint64)[:, None]
    b = np.arange(256, dtype=np.uint64)[None, :]
    return clmul_mod(a, b, 0x11D, 8).astype(np.uint8)


def gf16_mul(a, b):
    return clmul_mod(a, b, 0x1100B, 16).astype(np.uint16)


def gf16_pow2(e: int) -> int:
    """alpha^e in GF(2^16)/0x1100B by square-and-multiply on clmul."""
    r, x = 1, 2
    e %= 65535
    while e:
        if e & 1:
            r = int(gf16_mul(r, x))
        x = int(gf16_mul(x, x))
        e >>= 1
    return r


def gf8_inv_brute(M8, a: int) -> int:
    row = M8[a]
    hits = np.nonzero(row == 1)[0]
    return int(hits[0]) if hits.size else 0


def gf8_rank(M8, A: np.ndarray) -> int:
    """Rank of a matrix over GF(2^8) by elimination with the brute-force table."""
    A = A.copy().astype(np.uint8)
    rows, cols = A.shape
    rank = 0
    for c in range(cols):
        piv = next((r for r in range(rank, rows) if A[r, c]), None)
        if piv is None:
            continue
        A[[rank, piv]] = A[[piv, rank]]
        inv = gf8_inv_brute(M8, int(A[rank, c]))
        A[rank] = M8[inv][A[rank]]
        for r in range(rows):
            if r != rank and A[r, c]:
                A[r] ^= M8[int(A[r, c])][A[rank]]
        rank += 1
    return rank


def gf2_rank(rows):
    """Rank over GF(2) of a list of python-int bit rows."""
    basis = []
    for v in rows:
        for b in basis:
            v = min(v, v ^ b)
        if v:
            basis.append(v)
    return len(basis)
