"""The generated gfx950 code never writes a VGPR that holds the data of a
store of more than 64 bits within 2 instructions of that store (the
store-data wait states of the CDNA3 family).  The compiler enforces them only
for stores without an SGPR soffset, so the kernels' stores are written to take
an immediate soffset; this test compiles every kernel file to assembly and
checks the property on every such store."""
import concurrent.futures as cf
import glob
import os
import re
import shutil
import subprocess

import pytest

from conftest import ROOT

CSRC = os.path.join(ROOT, "26mlsys-ae-ghostserve_amd", "csrc")
# every kernel file, so that new kernels are covered as they are added
FILES = sorted(os.path.basename(f) for f in glob.glob(os.path.join(CSRC, "*.hip")))
WAIT = 2
STORE = re.compile(r"^\s*(buffer|global|flat|scratch)_store_dwordx[34]\s+(.*)")


def _regs(tok):
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def store_data_overwrites(asm: str, wait: int = WAIT):
    """(kernel, line, gap) for every VALU write of a >64-bit store's data VGPRs
    fewer than `wait` instructions (s_nop N counting N+1) after the store."""
    out, kern = [], None
    lines = asm.splitlines()
    for i, line in enumerate(lines):
        m = re.match(r"^(_Z\S+):", line)
        if m:
            kern = m.group(1)
        s = STORE.match(line)
        if not s:
            continue
        ops = [o.strip() for o in s.group(2).split(",")]
        data = _regs(ops[0] if s.group(1) == "buffer" else ops[1])
        j, gap = i + 1, 0
        while j < len(lines) and gap < wait:
            t = lines[j].strip()
            j += 1
            if not t or t.startswith((";", ".")):
                continue
            if t.startswith("s_nop"):
                parts = t.split()
                gap += (int(parts[1], 0) + 1) if len(parts) > 1 else 1
                continue
            if t.startswith("v_") and _regs(t.split()[1].rstrip(",")) & data:
                out.append((kern, i + 1, gap))
                break
            gap += 1
    return out


def test_scanner_finds_back_to_back_overwrite():
    asm = "\n".join([
        "_Zk:",
        "\tbuffer_store_dwordx4 v[4:7], v52, s[12:15], s4 offen nt",
        "\tv_xor_b32_e32 v7, v47, v7",
        "\tbuffer_store_dwordx4 v[8:11], v52, s[12:15], 0 offen nt",
        "\ts_nop 1",
        "\tv_mov_b32_e32 v8, 0",
        "\tglobal_store_dwordx4 v[0:1], v[12:15], off",
        "\tv_add_u32_e32 v20, v1, v2",
        "\tv_mov_b32_e32 v13, 0",
    ])
    assert store_data_overwrites(asm) == [("_Zk", 2, 0), ("_Zk", 7, 1)]


def _asm(name, tmp):
    hipcc = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    out = os.path.join(tmp, name + ".s")
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "--cuda-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", CSRC, "-I", os.path.join(ROOT, "include"), os.path.join(CSRC, name), "-o", out]
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    return open(out).read()


def test_kernels_keep_store_data_wait_states(tmp_path):
    if not (os.environ.get("HIPCC") or shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not available")
    with cf.ThreadPoolExecutor(len(FILES)) as ex:
        asms = dict(zip(FILES, ex.map(lambda f: _asm(f, str(tmp_path)), FILES)))
    bad = {f: store_data_overwrites(a)[:5] for f, a in asms.items() if store_data_overwrites(a)}
    assert not bad, bad
    # the files whose kernels issue 128-bit (or 96-bit) stores were all scanned
    wide = {f for f, a in asms.items() if any(STORE.match(line) for line in a.splitlines())}
    assert {"rdp_spec.hip", "paged.hip", "chunk.hip", "rs8_spec.hip", "gs_xor_rdp.hip", "gs_rs16.hip",
            "copy.hip"} <= wide, wide
