"""Reed-Solomon over GF(2^16), signature-compatible with benchmark/rs/main.py.

``rs_kernel`` stands in for the pybind module ``rs_kernel16``
(benchmark/rs/kernel.cu:314-320).  Encode and reconstruct bytes are those of
the reference.  Differences that change no output byte:
  * init_gf_tables() is built once (in C) and cached, and the device copies of
    the tables are cached per device, instead of a 65,535-step Python loop and
    two host-to-device copies on every call.
  * K||V is packed straight into the padded data tensor.
  * Negative or repeated shard indices are rejected (the reference would write
    outside the shard tensor, or solve a singular system).
"""
from __future__ import annotations

import functools

import numpy as np
import torch

from . import _lib, spec

GF_SIZE = 1 << 16
GF_ORDER = GF_SIZE - 1


def _stream(t: torch.Tensor) -> int:
    return _lib.stream_handle(t.device)


def _u16(t: torch.Tensor) -> torch.Tensor:
    if t.element_size() != 2:
        raise TypeError("expected a 2-byte tensor")
    return t


class _RsKernel:
    """The reference module ``rs_kernel16``."""

    @staticmethod
    def pack_fp16_pair_to_u16(k, v, out):
        _lib.require_cuda(k, v, out, what="pack_fp16_pair_to_u16 tensor")
        _lib.call("kvec_rs16_pack", _u16(k).data_ptr(), _u16(v).data_ptr(), _u16(out).data_ptr(),
                  int(k.numel()), int(v.numel()), _stream(out))

    @staticmethod
    def u16_to_fp16_split(*args, **kwargs):
        # keyword names of the reference binding: in, k_out, v_out, N_k, N_v
        names = ["in", "k_out", "v_out", "N_k", "N_v"]
        a = dict(zip(names, args))
        a.update(kwargs)
        in_, k_out, v_out, N_k, N_v = (a[x] for x in names)
        _lib.require_cuda(in_, k_out, v_out, what="u16_to_fp16_split tensor")
        _lib.call("kvec_rs16_split", _u16(in_).data_ptr(), _u16(k_out).data_ptr(),
                  _u16(v_out).data_ptr(), int(N_k), int(N_v), _stream(in_))

    @staticmethod
    def encode_rs_u16(data_padded, shards, data_shards, parity_shards, shard_size, gf_exp, gf_log):
        _lib.require_cuda(data_padded, shards, gf_exp, gf_log, what="encode_rs_u16 tensor")
        _lib.call("kvec_rs16_encode", data_padded.data_ptr(), shards.data_ptr(), int(data_shards),
                  int(parity_shards), int(shard_size), gf_exp.data_ptr(), gf_log.data_ptr(),
                  _stream(shards))

    @staticmethod
    def reconstruct_rs_u16_inplace(shards, shard_size, data_shards, parity_shards, missing_data,
                                   parity_used, gf_exp, gf_log):
        _lib.require_cuda(shards, gf_exp, gf_log, what="reconstruct_rs_u16_inplace tensor")
        if missing_data.dtype != torch.int32 or parity_used.dtype != torch.int32:
            raise RuntimeError("indices must be int32")
        m = int(missing_data.numel())
        if m > 16:
            raise RuntimeError("m (missing data shards) must be <= 16")
        _lib.call("kvec_rs16_reconstruct", shards.data_ptr(), int(shard_size), int(data_shards),
                  int(parity_shards), missing_data.data_ptr() if m else None, m,
                  parity_used.data_ptr() if m else None, gf_exp.data_ptr(), gf_log.data_ptr(),
                  _stream(shards))


rs_kernel = _RsKernel()


@functools.lru_cache(maxsize=1)
def _tables_host():
    ex = np.zeros(2 * GF_ORDER, dtype=np.uint16)
    lg = np.zeros(GF_SIZE, dtype=np.uint16)
    _lib.call("kvec_gf16_tables", ex.ctypes.data, lg.ctypes.data)
    ex.setflags(write=False)
    lg.setflags(write=False)
    return ex, lg


def init_gf_tables():
    """benchmark/rs/main.py:39-54: (gf_exp uint16[131070], gf_log uint16[65536])
    for GF(2^16) with primitive polynomial 0x1100B."""
    ex, lg = _tables_host()
    return ex.copy(), lg.copy()


_dev_tables = {}


def device_gf_tables(device):
    key = str(torch.device(device))
    if key not in _dev_tables:
        ex, lg = _tables_host()
        _dev_tables[key] = (torch.from_numpy(ex.copy()).to(device=device, dtype=torch.uint16),
                            torch.from_numpy(lg.copy()).to(device=device, dtype=torch.uint16))
    return _dev_tables[key]


def shard_size_and_pad(total_symbols: int, num_data_shards: int):
    """benchmark/rs/main.py:57-60."""
    pad = (-total_symbols) % num_data_shards
    shard_size = (total_symbols + pad) // num_data_shards
    return shard_size, pad


SCHEMES = ("ghostserve", "spec")


def forward_encode_kv(keys: torch.Tensor, values: torch.Tensor, num_data_shards: int,
                      num_parity_shards: int, scheme: str = "ghostserve"):
    """benchmark/rs/main.py:63-137: returns (shards [(k+m), S] uint16, meta).
    scheme="spec": RS over GF(2^8)/0x11D with the Cauchy parity block (bytes
    of the same rows) instead of GF(2^16); S is then rounded up to a multiple
    of 8 words (16-byte rows)."""
    if scheme not in SCHEMES:
        raise ValueError(f"scheme must be one of {SCHEMES}, not {scheme!r}")
    assert keys.element_size() == 2 and values.element_size() == 2 and keys.dtype == values.dtype
    device = keys.device
    assert device.type == "cuda"
    B, H, T, D = keys.shape
    N_k = keys.numel()
    N_v = values.numel()
    total = N_k + N_v
    assert total > 0, "Empty KV tensors"
    assert num_data_shards > 0 and num_parity_shards >= 0

    shard_sz, pad = shard_size_and_pad(total, num_data_shards)
    if scheme == "spec":
        shard_sz = -(-shard_sz // 8) * 8
        pad = num_data_shards * shard_sz - total
    total_shards = num_data_shards + num_parity_shards
    assert shard_sz > 0
    # K || V and the zero padding go straight into the shard tensor's data rows
    # (the reference packs into a separate data_padded and the encode copies
    # it over); the encode then reads the rows in place and writes the parity
    # rows.  The shard bytes are the same.
    shards = torch.empty((total_shards, shard_sz), dtype=torch.uint16, device=device)
    data_rows = shards.view(-1)[: num_data_shards * shard_sz]
    if pad:
        data_rows.view(torch.int16)[total:].zero_()
    rs_kernel.pack_fp16_pair_to_u16(keys.contiguous().view(-1), values.contiguous().view(-1),
                                    data_rows)
    if scheme == "spec":
        rows = shards.view(torch.uint8).view(total_shards, -1)
        spec.rs8_encode([rows[i] for i in range(num_data_shards)],
                        [rows[num_data_shards + i] for i in range(num_parity_shards)])
    else:
        gf_exp, gf_log = device_gf_tables(device)
        rs_kernel.encode_rs_u16(data_rows, shards, num_data_shards, num_parity_shards, shard_sz,
                                gf_exp, gf_log)
    meta = {
        "B": B, "H": H, "T": T, "D": D,
        "N_k": N_k, "N_v": N_v,
        "total": total,
        "pad": pad,
        "shard_sz": shard_sz,
        "num_data": num_data_shards,
        "num_parity": num_parity_shards,
        "dtype": keys.dtype,
        "scheme": scheme,
    }
    return shards, meta


def backwards_decode_kv(shards: torch.Tensor, meta: dict, missing_shards):
    """benchmark/rs/main.py:140-206: rebuild missing data shards in place from
    the first surviving parities, then split K, V.  Returns (K, V).  For meta
    of scheme "spec" every missing shard (data or parity, at most m) is
    rebuilt by the GF(2^8) decode."""
    device = shards.device
    num_data = meta["num_data"]
    num_parity = meta["num_parity"]
    shard_sz = meta["shard_sz"]
    if any(int(i) < 0 for i in missing_shards):
        raise ValueError("missing shard indices must be >= 0")
    if len(set(missing_shards)) != len(list(missing_shards)):
        raise ValueError("missing shard indices must be distinct")

    missing_data = sorted([i for i in missing_shards if i < num_data])
    missing_par = sorted([i - num_data for i in missing_shards
                          if num_data <= i < num_data + num_parity])
    avail_par = [p for p in range(num_parity) if p not in missing_par]
    if len(missing_data) > len(avail_par):
        raise RuntimeError("Not enough parity shards to reconstruct the missing data shards.")

    if meta.get("scheme", "ghostserve") == "spec":
        if len(set(missing_shards)) > num_parity:
            raise RuntimeError("Not enough parity shards to reconstruct the missing shards.")
        if missing_shards:
            rows = shards.view(torch.uint8).view(num_data + num_parity, -1)
            spec.rs8_decode([rows[i] for i in range(num_data + num_parity)], num_data,
                            [int(i) for i in missing_shards])
        missing_data = []
    gf_exp, gf_log = device_gf_tables(device)
    if missing_data:
        if len(missing_data) > 16:
            raise RuntimeError("Reconstruction supports at most 16 missing data shards at once.")
        missing_data_t = torch.tensor(missing_data, dtype=torch.int32, device=device)
        parity_used_t = torch.tensor(avail_par[:len(missing_data)], dtype=torch.int32,
                                     device=device)
        rs_kernel.reconstruct_rs_u16_inplace(shards, shard_sz, num_data, num_parity,
                                             missing_data_t, parity_used_t, gf_exp, gf_log)

    data_area = shards[:num_data].contiguous().view(-1)[:meta["total"]]
    dtype = meta.get("dtype", torch.float16)
    K = torch.empty(meta["N_k"], dtype=dtype, device=device)
    V = torch.empty(meta["N_v"], dtype=dtype, device=device)
    rs_kernel.u16_to_fp16_split(data_area, K, V, meta["N_k"], meta["N_v"])
    B, H, T, D = meta["B"], meta["H"], meta["T"], meta["D"]
    return K.view(B, H, T, D), V.view(B, H, T, D)
