// rdp_spec.hip -- textbook RDP (Corbett et al., FAST 2004) over a prime p.
//
// Geometry: every shard is its own HBM buffer, cut into stripes of p-1 rows
// (RdpGeom, kvec_internal.h: rows of U bytes, a shorter last stripe; U = 0 is
// one stripe of p-1 row planes).  Byte offset o of a stripe's rows is an
// independent RDP instance.  Rows of 16-64 KiB measured fastest: the time
// follows the distance between the rows one column's cells come from (15 MB
// apart with row planes: 8 % slower).  A thread owns one 16-byte lane offset
// and streams all k*(p-1) cells of its stripe column through registers, so
// each data byte is read from HBM once and each parity byte is written once.  The diagonal of a cell is a compile-time constant after
// unrolling, so the "shift" of the diagonal parity costs no data movement at
// all: it is only a choice of accumulator register.
//
// Decode is a fixed GF(2) linear map per erasure pattern.  It is solved at
// compile time (constexpr Gauss-Jordan over the code's row/diagonal equations)
// for the built (p, k) configurations, so the kernel is a straight-line XOR
// network over the surviving cells; other configurations take the same map as
// a kernel argument.
#include "rdp_plan.h"

namespace kvec {

// ---------------------------------------------------------------- encode
// A thread owns one 16-byte lane offset; a block is one wave, so each load
// instruction reads 1 KiB contiguous from one stripe row.  Memory-level
// parallelism comes from each thread requesting many cells before folding any
// of them in: the cells of rdp_group(p, k) shards (all k*(p-1) cells for p <= 7) are
// issued back to back, and a scheduling barrier keeps the compiler from
// interleaving the XORs with them, which it otherwise does to lower register
// use, waiting on each load in turn.  Two waves per SIMD leave room for the
// 36 in-flight cells of p = 7 (144 VGPRs) beside the 12 accumulators.
constexpr int kBS = 64;

// Shards whose cells are requested together: every shard while their cells
// and the 2(p-1) accumulators fit in about 200 VGPRs.
constexpr int rdp_group(int P, int K) {
    const int g = (50 - 2 * (P - 1)) / (P - 1);
    return g < 1 ? 1 : (g > K ? K : g);
}

template <int P, int K, bool BUF>
__global__ __launch_bounds__(kBS) __attribute__((amdgpu_waves_per_eu(1, 2))) void rdp_encode_kernel(
        RdpPtrs d, uint8_t* __restrict__ Pp, uint8_t* __restrict__ Qp, RdpGeom geo, uint64_t nb) {
    constexpr int ROWS = P - 1, G = rdp_group(P, K);
    const RdpWave w = rdp_wave(geo, ROWS, blockIdx.x, threadIdx.x);
    if (w.within >= w.g) return;
    const uint32_t off = w.within;
    RdpAcc<P> pr[ROWS], q[ROWS];
#pragma unroll
    for (int j0 = 0; j0 < K; j0 += G) {
        u32x4 x[G][ROWS];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (j0 + g >= K) break;
            const ShardView<BUF> sv(d.p[j0 + g], nb);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) x[g][r] = sv.load(w.base + r * w.g, off);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int j = j0 + g;
            if (j >= K) break;
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                pr[r].add(x[g][r]);
                const int dg = (r + j) % P;
                if (dg != P - 1) q[dg].add(x[g][r]);
            }
        }
        // keep the next group's loads behind this fold (bounds register use):
        // a compiler memory barrier for the IR passes, a scheduling barrier
        // for the machine scheduler
        if constexpr (G < K) {
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    const ShardView<BUF> sp(Pp, nb), sq(Qp, nb);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const u32x4 pv = pr[r].get();
        sp.store(w.base + r * w.g, off, pv);
        // The P cell of row r lies on diagonal (r + p - 1) % p = r - 1.
        if (r >= 1) q[r - 1].add(pv);
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) sq.store(w.base + r * w.g, off, q[r].get());
}

// ---------------------------------------------------------------- decode
// Same shape as the encode: every surviving cell the plan needs (36 for a
// p = 7 pair) is requested before the XOR network runs.  The network follows
// the pattern's schedule (rdp_plan.h): each output extends an earlier one by
// the cells where their maps differ.
template <int P, int K, int E0, int E1, bool BUF>
__global__ __launch_bounds__(kBS) __attribute__((amdgpu_waves_per_eu(1, 2))) void rdp_decode_kernel(
        RdpPtrs sh, RdpGeom geo, uint64_t nb) {
    constexpr int ROWS = P - 1;
    constexpr int NC = (K + 2) * ROWS;
    constexpr RdpPlan plan = make_rdp_plan(P, K, E0, E1);
    static_assert(plan.ok, "RDP erasure pattern not decodable");
    const RdpWave w = rdp_wave(geo, ROWS, blockIdx.x, threadIdx.x);
    if (w.within >= w.g) return;
    const uint32_t off = w.within;
    u32x4 x[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (!((plan.need[c >> 6] >> (c & 63)) & 1)) continue;
        x[c] = ShardView<BUF>(sh.p[c / ROWS], nb).load(w.base + (c % ROWS) * w.g, off);
    }
    __builtin_amdgcn_sched_barrier(0);
    constexpr RdpSched sch = make_rdp_sched(plan);
    u32x4 acc[plan.nout];
#pragma unroll
    for (int i = 0; i < plan.nout; ++i) {
        const int o = sch.order[i];
        Xor3Acc a(sch.base[o] < 0 ? u32x4{0, 0, 0, 0} : acc[sch.base[o]]);
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if ((sch.dmask[o][c >> 6] >> (c & 63)) & 1) a.add(x[c]);
        acc[o] = a.get();
    }
#pragma unroll
    for (int o = 0; o < plan.nout; ++o) {
        const int c = plan.out_cell[o];
        ShardView<BUF>(sh.p[c / ROWS], nb).store(w.base + (c % ROWS) * w.g, off, acc[o]);
    }
}

// The decode map by input cell, for the generic kernel: each cell the outputs
// need, with the set of outputs (bit o) that XOR it in.  Built on the host
// from the plan's per-output masks.
constexpr int kRdpMaxCells = kRdpMaxShards * kRdpMaxRows;
static_assert(kRdpMaxOut <= 32, "output sets are 32-bit masks");
struct RdpCellMap {
    int ncell, nout;
    int out_cell[kRdpMaxOut];
    uint8_t cell[kRdpMaxCells];
    uint32_t outs[kRdpMaxCells];
};

inline RdpCellMap rdp_cell_map(const RdpPlan& plan) {
    RdpCellMap cm{};
    cm.nout = plan.nout;
    for (int o = 0; o < plan.nout; ++o) cm.out_cell[o] = plan.out_cell[o];
    for (int c = 0; c < kRdpMaxCells; ++c) {
        uint32_t outs = 0;
        for (int o = 0; o < plan.nout; ++o)
            if ((plan.mask[o][c >> 6] >> (c & 63)) & 1) outs |= 1u << o;
        if (outs) {
            cm.cell[cm.ncell] = uint8_t(c);
            cm.outs[cm.ncell++] = outs;
        }
    }
    return cm;
}

// Same map for any (p, k) and any shard size.  Each needed cell is loaded
// once, BATCH at a time so that BATCH are in flight, and folded into every
// output that uses it (wave-uniform tests of its output set); the 2 ROWS
// outputs accumulate in registers.  Sized per p, so that small codes keep
// more loads in flight.
template <int ROWS, int BATCH>
__global__ __launch_bounds__(kBS) void rdp_decode_generic_kernel(RdpPtrs sh, RdpCellMap cm, RdpGeom geo) {
    constexpr int NOUT = 2 * ROWS;
    static_assert(NOUT <= kRdpMaxOut, "outputs of one stripe");
    const RdpWave w = rdp_wave(geo, ROWS, blockIdx.x, threadIdx.x);
    if (w.within >= w.g) return;
    const uint64_t off = w.base + w.within;
    u32x4 acc[NOUT];
#pragma unroll
    for (int o = 0; o < NOUT; ++o) acc[o] = u32x4{0, 0, 0, 0};
    for (int i0 = 0; i0 < cm.ncell; i0 += BATCH) {
        u32x4 x[BATCH];
#pragma unroll
        for (int t = 0; t < BATCH; ++t) {
            x[t] = u32x4{0, 0, 0, 0};
            if (i0 + t < cm.ncell) {
                const int c = cm.cell[i0 + t];
                x[t] = ld16(sh.p[c / ROWS] + uint64_t(c % ROWS) * w.g + off);
            }
        }
#pragma unroll
        for (int t = 0; t < BATCH; ++t) {
            const uint32_t outs = i0 + t < cm.ncell ? cm.outs[i0 + t] : 0u;
#pragma unroll
            for (int o = 0; o < NOUT; ++o)
                if ((outs >> o) & 1) acc[o] ^= x[t];
        }
    }
#pragma unroll
    for (int o = 0; o < NOUT; ++o) {
        if (o < cm.nout) {
            const int c = cm.out_cell[o];
            st_stream(sh.p[c / ROWS] + uint64_t(c % ROWS) * w.g, off, acc[o]);
        }
    }
}

typedef void (*GenericDecFn)(RdpPtrs, RdpCellMap, RdpGeom);

static GenericDecFn generic_decode_fn(int p) {
    switch (p) {
        case 3: return &rdp_decode_generic_kernel<2, 16>;
        case 5: return &rdp_decode_generic_kernel<4, 16>;
        case 7: return &rdp_decode_generic_kernel<6, 16>;
        case 11: return &rdp_decode_generic_kernel<10, 8>;
        case 13: return &rdp_decode_generic_kernel<12, 12>;
        default: return nullptr;
    }
}

// ---------------------------------------------------------------- dispatch
typedef void (*EncFn)(RdpPtrs, uint8_t*, uint8_t*, RdpGeom, uint64_t);
typedef void (*DecFn)(RdpPtrs, RdpGeom, uint64_t);

template <int P, bool BUF, int K = 1>
EncFn pick_encode(int k) {
    if constexpr (K > P - 1) {
        return nullptr;
    } else {
        if (k == K) return &rdp_encode_kernel<P, K, BUF>;
        return pick_encode<P, BUF, K + 1>(k);
    }
}

template <bool BUF>
static EncFn encode_fn(int p, int k) {
    switch (p) {
        case 3: return pick_encode<3, BUF>(k);
        case 5: return pick_encode<5, BUF>(k);
        case 7: return pick_encode<7, BUF>(k);
        case 11: return pick_encode<11, BUF>(k);
        case 13: return pick_encode<13, BUF>(k);
        default: return nullptr;
    }
}

template <int P, int K, bool BUF, int E0, int E1>
DecFn pick_decode_pair(int e1) {
    if constexpr (E1 > K + 1) {
        return nullptr;
    } else {
        if (e1 == E1) return &rdp_decode_kernel<P, K, E0, E1, BUF>;
        return pick_decode_pair<P, K, BUF, E0, E1 + 1>(e1);
    }
}

template <int P, int K, bool BUF, int E0 = 0>
DecFn pick_decode(int e0, int e1) {
    if constexpr (E0 > K + 1) {
        return nullptr;
    } else {
        if (e0 == E0) {
            if (e1 < 0) return &rdp_decode_kernel<P, K, E0, -1, BUF>;
            return pick_decode_pair<P, K, BUF, E0, E0 + 1>(e1);
        }
        return pick_decode<P, K, BUF, E0 + 1>(e0, e1);
    }
}

// Compile-time XOR networks are built for the full-width codes p = 3, 5, 7,
// through buffer resources (shards below 4 GiB) or flat addresses (larger);
// everything else takes the generic kernel.
template <bool BUF>
static DecFn decode_fn_t(int p, int k, int e0, int e1) {
    if (p == 7 && k == 6) return pick_decode<7, 6, BUF>(e0, e1);
    if (p == 5 && k == 4) return pick_decode<5, 4, BUF>(e0, e1);
    if (p == 3 && k == 2) return pick_decode<3, 2, BUF>(e0, e1);
    return nullptr;
}

static DecFn decode_fn(int p, int k, int e0, int e1, bool buf) {
    return buf ? decode_fn_t<true>(p, k, e0, e1) : decode_fn_t<false>(p, k, e0, e1);
}

static int check_geom(int k, int p, int64_t row_bytes, int64_t unit_bytes, const char* fn) {
    if (!is_prime(p) || p < 3) return set_error(KVEC_EINVAL, "%s: p=%d is not an odd prime", fn, p);
    if (p > kRdpMaxP) return set_error(KVEC_EUNSUPPORTED, "%s: p=%d > %d", fn, p, kRdpMaxP);
    if (k < 1 || k > p - 1) return set_error(KVEC_EINVAL, "%s: k=%d not in [1, p-1=%d]", fn, k, p - 1);
    if (row_bytes < 0 || row_bytes % 16 != 0)
        return set_error(KVEC_EINVAL, "%s: row_bytes=%lld must be a non-negative multiple of 16", fn,
                         (long long)row_bytes);
    if (row_bytes >= (int64_t(1) << 32))
        return set_error(KVEC_EUNSUPPORTED, "%s: row_bytes=%lld must be < 4 GiB", fn, (long long)row_bytes);
    if (unit_bytes < 0 || unit_bytes % kRdpWaveBytes != 0)
        return set_error(KVEC_EINVAL, "%s: unit_bytes=%lld must be 0 or a positive multiple of %u", fn,
                         (long long)unit_bytes, kRdpWaveBytes);
    return KVEC_OK;
}

}  // namespace kvec

using namespace kvec;

extern "C" int kvec_rdp_encode(const void* const* data, int k, void* P, void* Q, int p,
                               int64_t row_bytes, int64_t unit_bytes, void* stream) {
    int rc = check_geom(k, p, row_bytes, unit_bytes, "kvec_rdp_encode");
    if (rc) return rc;
    if (!data || !P || !Q) return set_error(KVEC_EINVAL, "kvec_rdp_encode: null pointer");
    RdpPtrs d{};
    for (int j = 0; j < k; ++j) {
        if (!data[j] || !aligned16(data[j]))
            return set_error(KVEC_EINVAL, "kvec_rdp_encode: data[%d] null or not 16-byte aligned", j);
        d.p[j] = (uint8_t*)data[j];
    }
    if (!aligned16(P) || !aligned16(Q))
        return set_error(KVEC_EINVAL, "kvec_rdp_encode: P/Q not 16-byte aligned");
    if (row_bytes == 0) return KVEC_OK;
    const uint64_t nb = uint64_t(p - 1) * uint64_t(row_bytes);
    {
        Span w[2] = {{P, nb, "P", -1}, {Q, nb, "Q", -1}};
        Span r[kRdpMaxShards];
        for (int j = 0; j < k; ++j) r[j] = Span{data[j], nb, "data", j};
        if ((rc = check_no_alias(w, 2, r, k, "kvec_rdp_encode"))) return rc;
    }
    const bool buf = fits_buffer(nb);
    EncFn fn = buf ? encode_fn<true>(p, k) : encode_fn<false>(p, k);
    if (!fn) return set_error(KVEC_EUNSUPPORTED, "kvec_rdp_encode: p=%d k=%d not built", p, k);
    const RdpGeom geo = make_rdp_geom(uint64_t(row_bytes), uint64_t(unit_bytes));
    hipLaunchKernelGGL(fn, dim3(unsigned(rdp_waves(geo))), dim3(kBS), 0, as_stream(stream), d,
                       (uint8_t*)P, (uint8_t*)Q, geo, nb);
    return check_launch("kvec_rdp_encode");
}

extern "C" int kvec_rdp_decode(void* const* shards, int k, int p, int64_t row_bytes, int64_t unit_bytes,
                               int e0, int e1, void* stream) {
    int rc = check_geom(k, p, row_bytes, unit_bytes, "kvec_rdp_decode");
    if (rc) return rc;
    if (!shards) return set_error(KVEC_EINVAL, "kvec_rdp_decode: null shard array");
    if (e0 < -1 || e0 > k + 1 || e1 < -1 || e1 > k + 1)
        return set_error(KVEC_EINVAL, "kvec_rdp_decode: erased index out of [-1, %d]", k + 1);
    RdpPtrs s{};
    for (int j = 0; j < k + 2; ++j) {
        if (!shards[j] || !aligned16(shards[j]))
            return set_error(KVEC_EINVAL, "kvec_rdp_decode: shard %d null or not 16-byte aligned", j);
        s.p[j] = (uint8_t*)shards[j];
    }
    // canonical pattern: a < b, or (a, -1)
    int a = e0, b = e1;
    if (a == b) b = -1;
    if (a < 0) { a = b; b = -1; }
    if (b >= 0 && b < a) { int t = a; a = b; b = t; }
    if (a < 0 || row_bytes == 0) return KVEC_OK;
    const uint64_t nb = uint64_t(p - 1) * uint64_t(row_bytes);
    {
        // the rebuilt shards must not share a byte with any other shard
        Span w[2], r[kRdpMaxShards];
        int nw = 0, nr = 0;
        for (int j = 0; j < k + 2; ++j)
            (j == a || j == b ? w[nw++] : r[nr++]) = Span{shards[j], nb, "shard", j};
        if ((rc = check_no_alias(w, nw, r, nr, "kvec_rdp_decode"))) return rc;
    }
    const RdpGeom geo = make_rdp_geom(uint64_t(row_bytes), uint64_t(unit_bytes));
    const dim3 grid(unsigned(rdp_waves(geo))), block(kBS);
    DecFn fn = decode_fn(p, k, a, b, fits_buffer(nb));
    if (fn) {
        hipLaunchKernelGGL(fn, grid, block, 0, as_stream(stream), s, geo, nb);
    } else {
        RdpPlan plan = make_rdp_plan(p, k, a, b);
        if (!plan.ok)
            return set_error(KVEC_EDECODE, "kvec_rdp_decode: pattern (%d, %d) not decodable", a, b);
        GenericDecFn gfn = generic_decode_fn(p);
        if (!gfn) return set_error(KVEC_EUNSUPPORTED, "kvec_rdp_decode: p=%d", p);
        hipLaunchKernelGGL(gfn, grid, block, 0, as_stream(stream), s, rdp_cell_map(plan), geo);
    }
    return check_launch("kvec_rdp_decode");
}

extern "C" int64_t kvec_rdp_row_bytes(int64_t stream_bytes, int k, int p, int64_t granule) {
    if (stream_bytes < 0 || k < 1 || p < 3 || granule < 16 || granule % 16 != 0) return -1;
    const int64_t cells = int64_t(k) * (p - 1);
    const int64_t per = (stream_bytes + cells - 1) / cells;
    return (per + granule - 1) / granule * granule;
}
