"""MI355X-native KV-cache erasure coding (GhostServe's coding hot path).

Hand-written gfx950 HIP kernels behind the C ABI of ``libkvec.so``
(include/kvec.h), with Python entry points that keep the reference's names and
signatures:

  xor         XOR single parity           (benchmark/xor/main.py)
  rdp         star-diagonal P/Q "RDP"     (benchmark/rdp/main.py)
  rs          Reed-Solomon over GF(2^16)  (benchmark/rs/main.py)
  rdp_kv_ops  the serving plugin's inline extension (bench_ghostserve_rdp.py)
  spec        textbook RDP over a prime p, RS over GF(2^8) (stripe configs)
  paged       paged KV pool <-> coding stream; fused gather + RDP encode
  chunked     per-prefill-chunk RDP + RS coding of a paged (e.g. fp8) cache
  offload     parity copies to pinned host memory on a side stream
  serving     forward_extend hook: per-step KV delta parity, JSONL metrics

Import the package with ``importlib.import_module("26mlsys-ae-ghostserve_amd")``
(the directory name is not a Python identifier).
"""
from . import _lib, chunked, offload, paged, rdp, rdp_kv_ops, rs, serving, spec, xor  # noqa: F401

__all__ = ["xor", "rdp", "rs", "rdp_kv_ops", "spec", "paged", "chunked", "offload", "serving"]
