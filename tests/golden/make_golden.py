"""Writes the small golden vectors under tests/golden/ from the CPU oracle.

The reference ships no test vectors for any codec, so these freeze the
oracle's outputs (each oracle function is pinned to the mathematics by
tests/test_oracle.py): a later change to the oracle that alters a byte fails
tests/test_golden.py, and the GPU kernels are compared with the same files.

Inputs are stored next to the outputs, so the fixtures do not depend on any
random generator.  Run from the repository root:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as ora  # noqa: E402


def u8(rng, *shape):
    return rng.integers(0, 256, shape, dtype=np.uint8)


def u16(rng, *shape):
    return rng.integers(0, 65536, shape, dtype=np.uint16)


def main():
    rng = np.random.default_rng(20260501)
    out = {}

    # gs XOR (benchmark/xor/kernel.cu): encode, then reconstruct data row 2
    nd, S = 4, 1000
    data = u8(rng, nd * S)
    shards = ora.xor_encode(data, nd, S)
    rec = shards.copy()
    rec[2] = 0
    rec_missing = ora.xor_reconstruct(rec, S, nd, [2])
    out["xor"] = dict(data=data, shards=shards, rec_missing=rec_missing, nd=nd, S=S)

    # gs star-diagonal RDP (benchmark/rdp/kernel.cu): backup, then recover(1, 3)
    T, n, nd, sb = 9, 13, 5, 3
    K = u16(rng, T, n)
    V = u16(rng, T, n)
    sh = ora.gs_backup(K, V, nd, sb)
    rc = sh.copy()
    ora.gs_recover(rc, nd, sh.shape[1], sb, 1, 3)
    out["gs_rdp"] = dict(K=K, V=V, shards=sh, recovered=rc, nd=nd, star_base=sb)

    # gs RS over GF(2^16) (benchmark/rs/kernel.cu): encode, reconstruct data {0, 2}
    k, m, S = 4, 2, 37
    ex, lg = ora.gf16_tables()
    d16 = u16(rng, k * S)
    sh16 = ora.rs16_encode(d16, k, m, S, ex, lg)
    er16 = sh16.copy()
    er16[0] = 0
    er16[2] = 0
    ora.rs16_reconstruct(er16, S, k, m, [0, 2], [0, 1], ex, lg)
    out["rs16"] = dict(data=d16, shards=sh16, reconstructed=er16, k=k, m=m, S=S)

    # spec RDP p = 7, k = 6 and p = 5, k = 3 (shortened)
    for p, k, R in ((7, 6, 64), (5, 3, 48)):
        dd = [u8(rng, p - 1, R) for _ in range(k)]
        P, Q = ora.rdp_encode(dd, p)
        out[f"rdp_p{p}k{k}"] = dict(data=np.stack(dd), P=P, Q=Q, p=p)

    # spec RS(6,2) and RS(5,3) over GF(2^8)/0x11D, Cauchy
    for k, m in ((6, 2), (5, 3)):
        dd = [u8(rng, 96) for _ in range(k)]
        par = ora.rs8_encode(dd, m)
        out[f"rs8_k{k}m{m}"] = dict(data=np.stack(dd), parity=np.stack(par),
                                   cauchy=ora.rs8_cauchy(k, m))

    # paged gather and chunked RDP(7) + RS(5,3) of a tiny fp8-like pool
    L, B, pps, pt, tb = 2, 2, 4, 4, 32
    npages = B * pps + 1
    pool = u8(rng, L, npages, pt, 2, tb)
    table = rng.permutation(npages)[: B * pps].astype(np.int32).reshape(B, pps)
    stream = ora.kv_gather(pool, table, pt, 3, 9)
    out["paged"] = dict(pool=pool, table=table, page_tokens=pt, tok_off=3, tokens=9,
                        stream=stream)
    # chunked: 256-byte records, 32-token chunks -> rows of 1280 bytes, so each
    # chunk region holds two stripes of the 1024-byte unit (rows 1024 and 256)
    L, B, pps, pt, tb, unit = 2, 2, 4, 16, 128, 1024
    npages = B * pps + 1
    cpool = u8(rng, L, npages, pt, 2, tb)
    ctable = rng.permutation(npages)[: B * pps].astype(np.int32).reshape(B, pps)
    W, cdata, cP, cQ, crs = ora.chunked_encode(cpool, ctable, pt, 32, 2, 5, 7, 3, unit)
    out["chunked"] = dict(pool=cpool, table=ctable, page_tokens=pt, chunk_tokens=32, n_chunks=2,
                          unit=unit, width=W, data=np.stack(cdata), P=cP, Q=cQ, rs=np.stack(crs))

    for name, arrs in out.items():
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"),
                            **{k: np.asarray(v) for k, v in arrs.items()})
        print(name, sum(np.asarray(v).nbytes for v in arrs.values()), "bytes")


if __name__ == "__main__":
    main()
