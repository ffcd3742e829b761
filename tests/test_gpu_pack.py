"""The reference's standalone XOR pack/unpack (xor_kernel.pack_kv / unpack_kv,
benchmark/xor/kernel.cu:93-146, called at benchmark/xor/main.py:80 and :194)
and the copy / zero-fill kernels behind every fallback path, on the GPU
through the C ABI, against the oracle."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bits16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _kv(B, H, T, D, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    k = torch.randn(B, H, T, D, generator=g).to(dtype)
    v = torch.randn(B, H, T, D, generator=g).to(dtype)
    return k, v


# (B, H, T, D): one 256 KiB shard of the XOR k=4 stripe (512 tokens x 1 head x
# 128 bf16, K||V), the whole k=4 stripe (4 x 256 KiB: 2048 tokens), odd n and
# T, the reference demo's shape
@pytest.mark.parametrize("B,H,T,D", [(1, 1, 512, 128), (1, 1, 2048, 128), (1, 3, 7, 1), (2, 1, 5, 3),
                                     (1, 8, 512, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_unpack_match_oracle(pkg, ora, gpu, B, H, T, D, dtype):
    k, v = _kv(B, H, T, D, dtype, seed=B * 100 + H * 10 + T)
    n, seq_len = B * H * D, T
    kd, vd = k.to(gpu), v.to(gpu)
    kv_bytes = torch.full((4 * n * seq_len,), 0xCD, dtype=torch.uint8, device=gpu)
    pkg.xor.xor_kernel.pack_kv(kd, vd, kv_bytes, n, seq_len)
    want = ora.pack_kv(_bits16(k), _bits16(v), n, seq_len)
    got = kv_bytes.cpu().numpy()
    assert np.array_equal(got, want)
    # little-endian byte pairs: K region, then V region
    kb = _bits16(k).reshape(-1)
    assert np.array_equal(got[0:2 * n * seq_len:2], (kb & 0xFF).astype(np.uint8))
    assert np.array_equal(got[1:2 * n * seq_len:2], (kb >> 8).astype(np.uint8))
    out = torch.full((2 * n * seq_len,), 7, dtype=dtype, device=gpu)
    pkg.xor.xor_kernel.unpack_kv(kv_bytes, out, n, seq_len)
    torch.cuda.synchronize()
    assert np.array_equal(_bits16(out), ora.unpack_kv(want, n, seq_len))
    assert torch.equal(out[: n * seq_len].view(k.shape).cpu(), k)
    assert torch.equal(out[n * seq_len:].view(v.shape).cpu(), v)


@pytest.mark.parametrize("shift", [0, 2, 6, 14])
def test_pack_unpack_misaligned_views(pkg, ora, gpu, shift):
    """Tensors that start `shift` bytes past a 16-byte boundary take the copy
    kernel's funnel path (source and destination misaligned differently)."""
    n, seq_len = 5, 37
    words = n * seq_len
    k, v = _kv(1, 1, seq_len, n, torch.float16, seed=shift)
    base_k = torch.zeros(words + 16, dtype=torch.float16, device=gpu)
    base_v = torch.zeros(words + 16, dtype=torch.float16, device=gpu)
    kd = base_k[shift // 2: shift // 2 + words]
    vd = base_v[(shift // 2 + 3) % 8: (shift // 2 + 3) % 8 + words]
    kd.copy_(k.reshape(-1).to(gpu))
    vd.copy_(v.reshape(-1).to(gpu))
    buf = torch.full((4 * words + 32,), 0xEE, dtype=torch.uint8, device=gpu)
    kvb = buf[5: 5 + 4 * words]
    pkg.xor.xor_kernel.pack_kv(kd, vd, kvb, n, seq_len)
    want = ora.pack_kv(_bits16(k), _bits16(v), n, seq_len)
    host = buf.cpu().numpy()
    assert np.array_equal(host[5: 5 + 4 * words], want)
    assert (host[:5] == 0xEE).all() and (host[5 + 4 * words:] == 0xEE).all()
    out_base = torch.zeros(2 * words + 16, dtype=torch.float16, device=gpu)
    out = out_base[1: 1 + 2 * words]
    pkg.xor.xor_kernel.unpack_kv(kvb, out, n, seq_len)
    torch.cuda.synchronize()
    assert np.array_equal(_bits16(out), ora.unpack_kv(want, n, seq_len))
    ob = out_base.cpu()
    assert ob[0].item() == 0 and not ob[1 + 2 * words:].any()


@pytest.mark.parametrize("N_k,N_v,off_in,off_out", [(1, 0, 0, 0), (7, 9, 1, 3), (8, 8, 0, 0),
                                                    (1000, 333, 5, 2), (65536 + 3, 17, 7, 1)])
def test_rs16_pack_split_copy_kernel(pkg, gpu, N_k, N_v, off_in, off_out):
    """pack_fp16_pair_to_u16 / u16_to_fp16_split (benchmark/rs/kernel.cu:225-263)
    through the copy kernel at word offsets that misalign every operand."""
    g = torch.Generator(device="cpu").manual_seed(N_k + N_v)
    kh = torch.randint(0, 1 << 16, (N_k,), generator=g, dtype=torch.int32).to(torch.int16)
    vh = torch.randint(0, 1 << 16, (N_v,), generator=g, dtype=torch.int32).to(torch.int16)
    kb = torch.zeros(N_k + 8, dtype=torch.int16, device=gpu)
    vb = torch.zeros(N_v + 8, dtype=torch.int16, device=gpu)
    kd, vd = kb[off_in: off_in + N_k], vb[off_out: off_out + N_v]
    kd.copy_(kh.to(gpu))
    vd.copy_(vh.to(gpu))
    ob = torch.full((N_k + N_v + 8,), -1, dtype=torch.int16, device=gpu)
    out = ob[off_out: off_out + N_k + N_v]
    pkg.rs.rs_kernel.pack_fp16_pair_to_u16(kd, vd, out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), torch.cat([kh, vh]))
    assert (ob[:off_out] == -1).all() and (ob[off_out + N_k + N_v:] == -1).all()
    k2 = torch.zeros(N_k + 1, dtype=torch.int16, device=gpu)[1:]
    v2 = torch.zeros(N_v, dtype=torch.int16, device=gpu)
    pkg.rs.rs_kernel.u16_to_fp16_split(out, k2, v2, N_k, N_v)
    torch.cuda.synchronize()
    assert torch.equal(k2.cpu(), kh) and torch.equal(v2.cpu(), vh)


def test_pack_rejects_overlap(pkg, gpu):
    buf = torch.zeros(4096, dtype=torch.uint8, device=gpu)
    k = buf[:512].view(torch.float16)
    v = buf[512:1024].view(torch.float16)
    with pytest.raises(RuntimeError, match="overlap"):
        pkg.xor.xor_kernel.pack_kv(k, v, buf[256:256 + 2048], 256, 1)
