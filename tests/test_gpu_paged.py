"""Paged KV gather / scatter and the fused gather + RDP encode, against the
oracle (whose gather is pinned to numpy indexing of pool[slots, kv])."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def make_pool(gpu, L, B, pps, page_tokens, H, D, dtype, seed, extra_pages=3):
    g = torch.Generator(device="cpu").manual_seed(seed)
    npages = B * pps + extra_pages
    pool = torch.randn(L, npages, page_tokens, 2, H, D, generator=g).to(dtype)
    perm = torch.randperm(npages, generator=g)[: B * pps].view(B, pps).to(torch.int32)
    return pool, perm


def pool_bytes(pool):
    L, npages, pt, two, H, D = pool.shape
    return pool.contiguous().view(torch.uint8).numpy().reshape(L, npages, pt, 2, -1)


@pytest.mark.parametrize("L,B,pps,pt,H,D,dtype,tok_off,T", [
    (2, 3, 4, 16, 1, 128, torch.bfloat16, 0, 64),
    (3, 2, 6, 16, 2, 64, torch.float16, 16, 50),
    (2, 2, 8, 4, 1, 128, torch.float8_e4m3fn, 5, 17),
    (1, 1, 2, 1, 1, 8, torch.bfloat16, 1, 1),
])
def test_gather_scatter_match_oracle(pkg, ora, gpu, L, B, pps, pt, H, D, dtype, tok_off, T):
    pool, table = make_pool(gpu, L, B, pps, pt, H, D, dtype, seed=L * 10 + B)
    want = ora.kv_gather(pool_bytes(pool), table.numpy(), pt, tok_off, T)
    kv = pkg.paged.PagedKV(pool.to(gpu), table.to(gpu), tok_off, T)
    assert kv.stream_bytes() == want.size
    got = kv.gather()
    assert np.array_equal(got.cpu().numpy(), want.reshape(-1))
    # scatter of a modified stream writes exactly the chunk's token slots
    new = torch.randint(0, 256, (want.size,), dtype=torch.uint8)
    kv.scatter(new.to(gpu))
    after = pool_bytes(kv.pool.cpu())
    exp = pool_bytes(pool).copy()
    newv = new.numpy().reshape(L, B, T, 2, -1)
    for b in range(B):
        for t in range(T):
            tt = tok_off + t
            page = int(table[b, tt // pt])
            for kvi in range(2):
                exp[:, page, tt % pt, kvi] = newv[:, b, t, kvi]
    assert np.array_equal(after, exp)


@pytest.mark.parametrize("p,k", [(7, 6), (5, 4), (7, 3), (3, 2), (11, 10), (13, 9)])
def test_fused_gather_rdp_encode(pkg, ora, gpu, p, k):
    L, B, pps, pt, H, D = 4, 3, 5, 16, 1, 128
    pool, table = make_pool(gpu, L, B, pps, pt, H, D, torch.bfloat16, seed=p * k)
    kv = pkg.paged.PagedKV(pool.to(gpu), table.to(gpu), 0, pps * pt)
    R = pkg.paged.rdp_row_bytes_for(kv, k, p)
    assert R % (2 * kv.token_bytes) == 0
    n = (p - 1) * R
    data = [torch.full((n,), 0x77, dtype=torch.uint8, device=gpu) for _ in range(k)]
    P = torch.empty(n, dtype=torch.uint8, device=gpu)
    Q = torch.empty(n, dtype=torch.uint8, device=gpu)
    pkg.paged.rdp_encode_paged(kv, data, P, Q, p, R)
    stream = ora.kv_gather(pool_bytes(pool), table.numpy(), pt, 0, pps * pt).reshape(-1)
    padded = np.zeros(k * n, np.uint8)
    padded[: stream.size] = stream
    want_data = [padded[j * n:(j + 1) * n].reshape(p - 1, R) for j in range(k)]
    Pw, Qw = ora.rdp_encode(want_data, p)
    for j in range(k):
        assert np.array_equal(data[j].cpu().numpy().reshape(p - 1, R), want_data[j]), j
    assert np.array_equal(P.cpu().numpy().reshape(p - 1, R), Pw)
    assert np.array_equal(Q.cpu().numpy().reshape(p - 1, R), Qw)
    # and the same bytes as gather followed by the unfused encode
    d2 = pkg.spec.split_stream(kv.gather(), k, n)
    P2, Q2 = torch.empty_like(P), torch.empty_like(Q)
    pkg.spec.rdp_encode(d2, P2, Q2, p, R)
    assert torch.equal(P2, P) and torch.equal(Q2, Q)


def test_invalid_page_reads_zero(pkg, gpu):
    L, B, pps, pt, H, D = 1, 1, 2, 4, 1, 16
    pool, table = make_pool(gpu, L, B, pps, pt, H, D, torch.float16, seed=5)
    table[0, 1] = 10 ** 6
    kv = pkg.paged.PagedKV(pool.to(gpu), table.to(gpu), 0, 8)
    s = kv.gather().cpu().numpy().reshape(L, B, 8, 2, -1)
    assert not s[:, 0, 4:].any()
    assert s[:, 0, :4].any()


# p = 13 with k >= 10 is not built (its kernel would spill registers): the
# call fails with an error and writes nothing.
def test_paged_encode_unbuilt_config_raises(pkg, gpu):
    L, B, pps, pt, H, D = 2, 2, 4, 16, 1, 128
    pool, table = make_pool(gpu, L, B, pps, pt, H, D, torch.bfloat16, seed=3)
    kv = pkg.paged.PagedKV(pool.to(gpu), table.to(gpu), 0, pps * pt)
    p, k = 13, 10
    R = pkg.paged.rdp_row_bytes_for(kv, k, p)
    n = (p - 1) * R
    data = [torch.full((n,), 0x77, dtype=torch.uint8, device=gpu) for _ in range(k)]
    P = torch.full((n,), 0x55, dtype=torch.uint8, device=gpu)
    Q = torch.full((n,), 0x55, dtype=torch.uint8, device=gpu)
    with pytest.raises(RuntimeError, match="not built"):
        pkg.paged.rdp_encode_paged(kv, data, P, Q, p, R)
    torch.cuda.synchronize()
    assert bool((P == 0x55).all()) and bool((Q == 0x55).all())
    assert all(bool((d == 0x77).all()) for d in data)
