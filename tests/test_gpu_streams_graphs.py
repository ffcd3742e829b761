"""Launches captured in a HIP graph, and launches on concurrent streams, give
the bytes of eager launches: the library keeps no state between calls and
launches on the stream it is given (torch's current stream, which is the
capturing stream inside torch.cuda.graph).  Every graph replay follows eager
work that changes its inputs, with a synchronization between replays, and is
checked against an eager launch of the same call."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bytes(n, gpu, seed):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    return torch.randint(0, 256, (n,), generator=g, device=gpu, dtype=torch.uint8)


def _capture(fn):
    """Warm up on a side stream (as capture requires), then capture fn."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


def test_rdp_encode_in_hip_graph(pkg, gpu):
    p, k, R = 7, 6, 64 * 1024
    data = [_bytes((p - 1) * R, gpu, i) for i in range(k)]
    P = torch.empty((p - 1) * R, dtype=torch.uint8, device=gpu)
    Q = torch.empty_like(P)
    Pe, Qe = torch.empty_like(P), torch.empty_like(Q)
    graph = _capture(lambda: pkg.spec.rdp_encode(data, P, Q, p=p))
    for rep in range(4):
        for d in data:
            d.random_(0, 256)
        torch.cuda.synchronize()
        graph.replay()
        pkg.spec.rdp_encode(data, Pe, Qe, p=p)
        torch.cuda.synchronize()
        assert torch.equal(P, Pe) and torch.equal(Q, Qe), rep


def test_plugin_step_parity_in_hip_graph(pkg, gpu):
    """compute_rdp_parity on the plugin's per-step rows (8 + 2 rows of
    2 x 2048 tokens x 128 words), as a serving loop would capture it."""
    nd, S = 8, 2 * 2048 * 128
    rows = torch.zeros((nd + 2, S), dtype=torch.uint16, device=gpu)
    ref = torch.zeros_like(rows)
    graph = _capture(lambda: pkg.rdp_kv_ops.compute_rdp_parity(rows, nd, S, 3))
    for rep in range(4):
        rows[:nd].view(torch.uint8).random_(0, 256)
        torch.cuda.synchronize()
        graph.replay()
        ref.copy_(rows)
        ref[nd:].zero_()
        pkg.rdp_kv_ops.compute_rdp_parity(ref, nd, S, 3)
        torch.cuda.synchronize()
        assert torch.equal(rows, ref), rep


def test_encodes_on_concurrent_streams(pkg, gpu):
    """Two stripe sets encoded over and over on two streams at once, with
    their inputs rewritten on each stream between encodes."""
    p, k, R = 7, 6, 128 * 1024
    sets = []
    for s in range(2):
        data = [_bytes((p - 1) * R, gpu, 10 * s + i) for i in range(k)]
        P = torch.empty((p - 1) * R, dtype=torch.uint8, device=gpu)
        sets.append((data, P, torch.empty_like(P)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    for rep in range(5):
        for (data, P, Q), st in zip(sets, streams):
            with torch.cuda.stream(st):
                for d in data:
                    d.add_(rep + 1)
                pkg.spec.rdp_encode(data, P, Q, p=p)
    torch.cuda.synchronize()
    for data, P, Q in sets:
        Pe, Qe = torch.empty_like(P), torch.empty_like(Q)
        pkg.spec.rdp_encode(data, Pe, Qe, p=p)
        torch.cuda.synchronize()
        assert torch.equal(P, Pe) and torch.equal(Q, Qe)


def test_xor_and_rs16_encodes_in_hip_graph(pkg, gpu):
    """encode_xor and encode_rs_u16 (each with its data-row copy) captured in
    one graph on row sizes that end in partial tiles."""
    nd, Sb = 6, 8192 * 5 + 37
    k, m, S = 6, 2, 8192 * 3 + 5
    ex, lg = pkg.rs.device_gf_tables(gpu)
    xd = _bytes(nd * Sb, gpu, 1)
    xs = torch.empty((nd + 1, Sb), dtype=torch.uint8, device=gpu)
    rd = _bytes(k * S * 2, gpu, 2).view(torch.uint16)
    rsh = torch.empty((k + m, S), dtype=torch.uint16, device=gpu)
    xe, re = torch.empty_like(xs), torch.empty_like(rsh)

    def both(xs_, rsh_):
        pkg.xor.xor_kernel.encode_xor(xd, xs_, nd, Sb)
        pkg.rs.rs_kernel.encode_rs_u16(rd, rsh_, k, m, S, ex, lg)

    graph = _capture(lambda: both(xs, rsh))
    for rep in range(4):
        xd.random_(0, 256)
        rd.view(torch.uint8).random_(0, 256)
        torch.cuda.synchronize()
        graph.replay()
        both(xe, re)
        torch.cuda.synchronize()
        assert torch.equal(xs, xe) and torch.equal(rsh, re), rep


@pytest.mark.parametrize("lost,used", [((1, 4), (0, 1)), ((2,), (1,))])
def test_rs16_reconstruct_in_hip_graph(pkg, gpu, lost, used):
    """reconstruct_rs_u16_inplace (the one-shot tile kernel) captured once, for
    two lost rows and for one; before each replay the tensor is re-encoded
    from new data and the lost rows are overwritten."""
    k, m, S = 6, 2, 44741
    ex, lg = pkg.rs.device_gf_tables(gpu)
    data = _bytes(k * S * 2, gpu, 3).view(torch.uint16)
    sh = torch.empty((k + m, S), dtype=torch.uint16, device=gpu)
    md = torch.tensor(lost, dtype=torch.int32, device=gpu)
    pu = torch.tensor(used, dtype=torch.int32, device=gpu)
    pkg.rs.rs_kernel.encode_rs_u16(data, sh, k, m, S, ex, lg)
    graph = _capture(lambda: pkg.rs.rs_kernel.reconstruct_rs_u16_inplace(sh, S, k, m, md, pu, ex, lg))
    for rep in range(4):
        data.view(torch.uint8).random_(0, 256)
        pkg.rs.rs_kernel.encode_rs_u16(data, sh, k, m, S, ex, lg)
        want = sh.clone()
        for r in lost:
            sh[r].fill_(0x1111 * (r + 1) + rep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(sh, want), rep


def test_fused_backup_in_hip_graph(pkg, gpu):
    """fused_backup_full_kv (pack K || V into the rows + star-diagonal P/Q)
    captured and replayed on new K and V."""
    T, n, nd, sb = 64, 301, 6, 5        # 4 padding words after K || V
    S = -(-2 * T * n // nd)
    K = torch.empty((T, n), dtype=torch.int16, device=gpu)
    V = torch.empty_like(K)
    sh = torch.zeros((nd + 2, S), dtype=torch.uint16, device=gpu)
    ref = torch.zeros_like(sh)
    graph = _capture(lambda: pkg.rdp.rdp_kernel.fused_backup_full_kv(K, V, sh, nd, S, T, n, sb))
    for rep in range(4):
        K.view(torch.uint8).random_(0, 256)
        V.view(torch.uint8).random_(0, 256)
        torch.cuda.synchronize()
        graph.replay()
        pkg.rdp.rdp_kernel.fused_backup_full_kv(K, V, ref, nd, S, T, n, sb)
        torch.cuda.synchronize()
        assert torch.equal(sh, ref), rep
