"""ctypes binding of libkvec.so (the C ABI declared in include/kvec.h).

torch is imported before the library is opened on purpose: torch ships its own
HIP runtime with the same soname (libamdhip64.so.7), and opening libkvec after
torch makes the dynamic linker bind libkvec to that same runtime, so the
hipStream_t handles torch hands out are valid inside libkvec.

There is no fallback: if libkvec.so is missing or fails to load, every entry
point raises.
"""
from __future__ import annotations

import ctypes as C
import os

import torch  # noqa: F401  (must precede CDLL, see module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkvec.so")

_vp = C.c_void_p
_i = C.c_int
_i64 = C.c_int64
_pp = C.POINTER(C.c_void_p)

class PagedKV(C.Structure):
    """struct kvec_paged_kv of include/kvec.h."""
    _fields_ = [
        ("pool", C.c_void_p),
        ("pool_pages", C.c_int64),
        ("layers", C.c_int),
        ("token_bytes", C.c_int64),
        ("page_tokens", C.c_int),
        ("page_table", C.c_void_p),
        ("batch", C.c_int),
        ("pages_per_seq", C.c_int),
        ("tok_off", C.c_int),
        ("tokens", C.c_int),
    ]


_kvp = C.POINTER(PagedKV)


class ChunkStripe(C.Structure):
    """struct kvec_chunk_stripe of include/kvec.h."""
    _fields_ = [
        ("data", C.POINTER(C.c_void_p)),
        ("k", C.c_int),
        ("P", C.c_void_p),
        ("Q", C.c_void_p),
        ("p", C.c_int),
        ("rs", C.POINTER(C.c_void_p)),
        ("m", C.c_int),
        ("row_bytes", C.c_int64),
        ("region_off", C.c_int64),
        ("width", C.c_int64),
        ("unit_bytes", C.c_int64),
    ]


_csp = C.POINTER(ChunkStripe)

# name -> (restype, argtypes); mirrors include/kvec.h
SIGNATURES = {
    "kvec_version": (_i, []),
    "kvec_strerror": (C.c_char_p, [_i]),
    "kvec_last_error": (C.c_char_p, []),
    "kvec_rdp_encode": (_i, [_pp, _i, _vp, _vp, _i, _i64, _i64, _vp]),
    "kvec_rdp_decode": (_i, [_pp, _i, _i, _i64, _i64, _i, _i, _vp]),
    "kvec_rdp_row_bytes": (_i64, [_i64, _i, _i, _i64]),
    "kvec_rs8_cauchy": (_i, [_i, _i, _vp]),
    "kvec_rs8_encode": (_i, [_pp, _i, _pp, _i, _i64, _vp]),
    "kvec_rs8_decode": (_i, [_pp, _i, _i, _i64, _vp, _i, _vp]),
    "kvec_kv_stream_bytes": (_i64, [_kvp]),
    "kvec_kv_gather": (_i, [_kvp, _vp, _vp]),
    "kvec_kv_gather_split": (_i, [_kvp, _vp, _vp, _vp]),
    "kvec_kv_scatter": (_i, [_kvp, _vp, _vp, _vp]),
    "kvec_rdp_encode_paged": (_i, [_kvp, _pp, _i, _vp, _vp, _i, _i64, _i64, _vp]),
    "kvec_rdp_decode_paged": (_i, [_kvp, _vp, _pp, _i, _vp, _vp, _i, _i64, _i64, _i, _i, _vp]),
    "kvec_chunk_width": (_i64, [_i64, _i, _i, _i64]),
    "kvec_chunk_encode_paged": (_i, [_kvp, _csp, _vp]),
    "kvec_chunk_decode_paged": (_i, [_kvp, _vp, _csp, _vp, _i, _vp]),
    "kvec_xor_encode": (_i, [_vp, _vp, _i, _i64, _vp]),
    "kvec_xor_encode_kv": (_i, [_vp, _vp, _i64, _vp, _i, _i64, _vp]),
    "kvec_xor_recover_kv": (_i, [_vp, _vp, _i, _i64, _i64, _i, _vp]),
    "kvec_xor_reconstruct": (_i, [_vp, _vp, _vp, _i64, _i, _vp, _i, _vp]),
    "kvec_pack_kv": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "kvec_unpack_kv": (_i, [_vp, _vp, _i, _i, _vp]),
    "kvec_gs_rdp_backup": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "kvec_gs_rdp_recover": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "kvec_gs_pack_row": (_i, [_vp, _vp, _vp, _i64, _i, _i64, _vp]),
    "kvec_gs_rdp_parity": (_i, [_vp, _i, _i, _i, _vp]),
    "kvec_hook_step": (_i, [_kvp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _pp]),
    "kvec_rs16_pack": (_i, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "kvec_rs16_split": (_i, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "kvec_rs16_encode": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "kvec_rs16_reconstruct": (_i, [_vp, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _vp]),
    "kvec_gf16_tables": (_i, [_vp, _vp]),
}

# major number of the include/kvec.h these signatures mirror (KVEC_VERSION / 10000)
ABI_MAJOR = 1

_lib = None


class KvecError(RuntimeError):
    """A libkvec call returned a non-zero status."""


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        ver = L.kvec_version()
        if ver // 10000 != ABI_MAJOR:
            raise RuntimeError(f"{LIB_PATH} has ABI version {ver}; these bindings need major "
                               f"version {ABI_MAJOR} (rebuild with __graft_entry__.build())")
        _lib = L
    return _lib


def call(name: str, *args) -> int:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().kvec_last_error().decode(errors="replace")
        raise KvecError(f"{name} failed ({lib().kvec_strerror(rc).decode()}): {msg}")
    return rc


def ptr_array(tensors) -> C.Array:
    return (C.c_void_p * len(tensors))(*[int(t.data_ptr()) for t in tensors])


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return int(torch.cuda.current_stream(device).cuda_stream)


def require_cuda(*tensors, what: str = "tensor") -> None:
    for t in tensors:
        if not t.is_cuda:
            raise ValueError(f"{what} must be a GPU (HIP) tensor")
        if not t.is_contiguous():
            raise ValueError(f"{what} must be contiguous")
