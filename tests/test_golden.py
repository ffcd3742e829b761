"""The committed golden vectors (tests/golden/*.npz, written by
tests/golden/make_golden.py from the oracle): the oracle still reproduces them
(CPU), and every HIP kernel produces them from the stored inputs (GPU)."""
import os

import numpy as np
import pytest
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ------------------------------------------------------------------ oracle (CPU)
def test_oracle_reproduces_xor(ora):
    g = load("xor")
    nd, S = int(g["nd"]), int(g["S"])
    sh = ora.xor_encode(g["data"], nd, S)
    assert np.array_equal(sh, g["shards"])
    rec = sh.copy()
    rec[2] = 0
    assert np.array_equal(ora.xor_reconstruct(rec, S, nd, [2]), g["rec_missing"])


def test_oracle_reproduces_gs_rdp(ora):
    g = load("gs_rdp")
    nd, sb = int(g["nd"]), int(g["star_base"])
    sh = ora.gs_backup(g["K"], g["V"], nd, sb)
    assert np.array_equal(sh, g["shards"])
    ora.gs_recover(sh, nd, sh.shape[1], sb, 1, 3)
    assert np.array_equal(sh, g["recovered"])


def test_oracle_reproduces_rs16(ora):
    g = load("rs16")
    k, m, S = int(g["k"]), int(g["m"]), int(g["S"])
    ex, lg = ora.gf16_tables()
    sh = ora.rs16_encode(g["data"], k, m, S, ex, lg)
    assert np.array_equal(sh, g["shards"])
    sh[0] = 0
    sh[2] = 0
    ora.rs16_reconstruct(sh, S, k, m, [0, 2], [0, 1], ex, lg)
    assert np.array_equal(sh, g["reconstructed"])


@pytest.mark.parametrize("name", ["rdp_p7k6", "rdp_p5k3"])
def test_oracle_reproduces_rdp(ora, name):
    g = load(name)
    P, Q = ora.rdp_encode([np.ascontiguousarray(x) for x in g["data"]], int(g["p"]))
    assert np.array_equal(P, g["P"]) and np.array_equal(Q, g["Q"])


@pytest.mark.parametrize("name", ["rs8_k6m2", "rs8_k5m3"])
def test_oracle_reproduces_rs8(ora, name):
    g = load(name)
    k, m = g["cauchy"].shape[1], g["cauchy"].shape[0]
    assert np.array_equal(ora.rs8_cauchy(k, m), g["cauchy"])
    par = ora.rs8_encode([np.ascontiguousarray(x) for x in g["data"]], m)
    assert np.array_equal(np.stack(par), g["parity"])


def test_oracle_reproduces_paged_and_chunked(ora):
    g = load("paged")
    s = ora.kv_gather(g["pool"], g["table"], int(g["page_tokens"]), int(g["tok_off"]),
                      int(g["tokens"]))
    assert np.array_equal(s, g["stream"])
    c = load("chunked")
    W, data, P, Q, rs = ora.chunked_encode(c["pool"], c["table"], int(c["page_tokens"]),
                                           int(c["chunk_tokens"]), int(c["n_chunks"]), 5, 7, 3,
                                           int(c["unit"]))
    assert W == int(c["width"])
    assert np.array_equal(np.stack(data), c["data"])
    assert np.array_equal(P, c["P"]) and np.array_equal(Q, c["Q"])
    assert np.array_equal(np.stack(rs), c["rs"])


# ------------------------------------------------------------------ HIP kernels
def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


@pytest.mark.gpu
def test_gpu_xor_golden(pkg, gpu):
    g = load("xor")
    nd, S = int(g["nd"]), int(g["S"])
    sh = torch.zeros((nd + 1, S), dtype=torch.uint8, device=gpu)
    pkg.xor.xor_kernel.encode_xor(dev(g["data"], gpu), sh, nd, S)
    assert np.array_equal(sh.cpu().numpy(), g["shards"])
    sh[2].zero_()
    rm = torch.empty((1, S), dtype=torch.uint8, device=gpu)
    pkg.xor.xor_kernel.reconstruct_xor(sh, sh, rm, S, nd,
                                       torch.tensor([2], dtype=torch.int32, device=gpu))
    assert np.array_equal(rm.cpu().numpy(), g["rec_missing"])
    assert np.array_equal(sh.cpu().numpy(), g["shards"])


@pytest.mark.gpu
def test_gpu_gs_rdp_golden(pkg, gpu):
    g = load("gs_rdp")
    nd, sb = int(g["nd"]), int(g["star_base"])
    T, n = g["K"].shape
    want = g["shards"]
    S = want.shape[1]
    sh = torch.zeros((nd + 2, S), dtype=torch.uint16, device=gpu)
    pkg.rdp.rdp_kernel.fused_backup_full_kv(dev(g["K"], gpu), dev(g["V"], gpu), sh, nd, S, T, n, sb)
    assert np.array_equal(sh.cpu().numpy(), want)
    out = torch.empty(2 * T * n, dtype=torch.uint16, device=gpu)
    pkg.rdp.rdp_kernel.fused_recovery_full_kv(sh, out, nd, S, T, n, sb, 1, 3)
    assert np.array_equal(sh.cpu().numpy(), g["recovered"])


@pytest.mark.gpu
def test_gpu_rs16_golden(pkg, gpu):
    g = load("rs16")
    k, m, S = int(g["k"]), int(g["m"]), int(g["S"])
    ex, lg = pkg.rs.device_gf_tables(gpu)
    sh = torch.zeros((k + m, S), dtype=torch.uint16, device=gpu)
    pkg.rs.rs_kernel.encode_rs_u16(dev(g["data"], gpu), sh, k, m, S, ex, lg)
    assert np.array_equal(sh.cpu().numpy(), g["shards"])
    sh[0].zero_()
    sh[2].zero_()
    i32 = lambda v: torch.tensor(v, dtype=torch.int32, device=gpu)  # noqa: E731
    pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(sh, S, k, m, i32([0, 2]), i32([0, 1]), ex, lg)
    assert np.array_equal(sh.cpu().numpy(), g["reconstructed"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["rdp_p7k6", "rdp_p5k3"])
def test_gpu_rdp_golden(pkg, gpu, name):
    g = load(name)
    p = int(g["p"])
    data = [dev(x.reshape(-1), gpu) for x in g["data"]]
    P = torch.empty_like(data[0])
    Q = torch.empty_like(data[0])
    pkg.spec.rdp_encode(data, P, Q, p)
    assert np.array_equal(P.cpu().numpy().reshape(g["P"].shape), g["P"])
    assert np.array_equal(Q.cpu().numpy().reshape(g["Q"].shape), g["Q"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["rs8_k6m2", "rs8_k5m3"])
def test_gpu_rs8_golden(pkg, gpu, name):
    g = load(name)
    data = [dev(x, gpu) for x in g["data"]]
    par = [torch.empty_like(data[0]) for _ in range(g["parity"].shape[0])]
    pkg.spec.rs8_encode(data, par)
    assert np.array_equal(torch.stack(par).cpu().numpy(), g["parity"])
    assert np.array_equal(pkg.spec.rs8_cauchy(len(data), len(par)), g["cauchy"])


@pytest.mark.gpu
def test_gpu_paged_and_chunked_golden(pkg, gpu):
    g = load("paged")
    pool = dev(g["pool"], gpu).unsqueeze(4)          # [L, pages, pt, 2, 1, tb]
    table = dev(g["table"], gpu)
    kv = pkg.paged.PagedKV(pool, table, int(g["tok_off"]), int(g["tokens"]))
    assert np.array_equal(kv.gather().cpu().numpy(), g["stream"].reshape(-1))
    c = load("chunked")
    pool = dev(c["pool"], gpu).unsqueeze(4)
    table = dev(c["table"], gpu)
    ct, nc = int(c["chunk_tokens"]), int(c["n_chunks"])
    kv0 = pkg.chunked.chunk_kv(pool, table, 0, ct)
    st = pkg.chunked.ChunkedStripes(kv0.stream_bytes(), 2 * kv0.token_bytes, nc, gpu, k=5, p=7,
                                    m=3, keep_data=True, unit_bytes=int(c["unit"]))
    assert st.width == int(c["width"])
    for ci in range(nc):
        st.encode(pkg.chunked.chunk_kv(pool, table, ci, ct), ci)
    got = lambda t: t.cpu().numpy()  # noqa: E731
    assert np.array_equal(np.stack([got(t) for t in st.data]), c["data"])
    assert np.array_equal(got(st.P), c["P"]) and np.array_equal(got(st.Q), c["Q"])
    assert np.array_equal(np.stack([got(t) for t in st.rs]), c["rs"])
