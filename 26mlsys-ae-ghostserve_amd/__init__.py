"""MI355X-native KV-cache erasure coding (GhostServe's coding hot path).

Hand-written gfx950 HIP kernels behind the C ABI of ``libkvec.so``
(include/kvec.h), with Python entry points that keep the reference's names and
signatures:

  spec        textbook RDP over a prime p, RS over GF(2^8) (stripe configs)

Import the package with ``importlib.import_module("26mlsys-ae-ghostserve_amd")``
(the directory name is not a Python identifier).
"""
from . import _lib, spec  # noqa: F401

__all__ = ["spec"]
