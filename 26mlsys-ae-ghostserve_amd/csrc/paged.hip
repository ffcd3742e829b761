// paged.hip -- paged KV pool <-> coding stream, and the fused gather + RDP
// encode.
//
// Pool: [layers][pool_pages][page_tokens][2 (K,V)][token_bytes], the token
// layout the reference's delta gather reads (kv_pool[slots, 0/1],
// bench_ghostserve_rdp.py:440-458), grouped in pages.  The page table maps
// (sequence b, logical page) to a pool page.  The coding stream of a chunk of
// `tokens` positions starting at tok_off holds the chunk's token records in
// order, [layers][batch][tokens][2][token_bytes], so every page contributes
// whole contiguous runs of records and a wave's 1 KiB of stream is one
// contiguous 1 KiB of a pool page.  Addressing: paged_geom.h.
#include "paged_geom.h"
#include "rdp_plan.h"

namespace kvec {

constexpr int kGBS = 256;

// stream[s] = pool cell, one 16-byte cell per thread
__global__ __launch_bounds__(kGBS) void kv_gather_kernel(PagedGeom g, uint8_t* __restrict__ out,
                                                         uint32_t ncells) {
    const uint32_t c = blockIdx.x * kGBS + threadIdx.x;
    if (c >= ncells) return;
    const uint32_t w = fdiv(c, g.div_cells);
    const uint32_t inner = (c - w * g.div_cells.d) * 16;
    st_stream(out, uint64_t(c) * 16, cell_load(g, w, inner));
}

// The K halves of the chunk's records to outK and the V halves to outV, each
// in record order (the delta gather kv_pool[slots, 0] / kv_pool[slots, 1] of
// bench_ghostserve_rdp.py:445-458, laid out as the [K | V] parity row of
// pack_row_from_block, :105-118).  tb = token_bytes, a multiple of 16, so no
// cell straddles the halves; the destination is selected without a branch.
__global__ __launch_bounds__(kGBS) void kv_gather_split_kernel(PagedGeom g, uint8_t* __restrict__ outK,
                                                               uint8_t* __restrict__ outV,
                                                               uint32_t ncells, uint32_t tb) {
    const uint32_t c = blockIdx.x * kGBS + threadIdx.x;
    if (c >= ncells) return;
    const uint32_t w = fdiv(c, g.div_cells);
    const uint32_t inner = (c - w * g.div_cells.d) * 16;
    const bool v = inner >= tb;
    st_stream(v ? outV : outK, uint64_t(w) * tb + (v ? inner - tb : inner), cell_load(g, w, inner));
}

// pool cell = stream[s] (inverse; padding slots and invalid pages are skipped)
__global__ __launch_bounds__(kGBS) void kv_scatter_kernel(PagedGeom g, const uint8_t* __restrict__ in,
                                                          uint32_t ncells) {
    const uint32_t c = blockIdx.x * kGBS + threadIdx.x;
    if (c >= ncells) return;
    const uint32_t w = fdiv(c, g.div_cells);
    const uint32_t inner = (c - w * g.div_cells.d) * 16;
    cell_store(g, w, inner, ld_stream(in, uint64_t(c) * 16));
}

// ------------------------------------------------- fused gather + RDP encode
// Cell (shard j, row r, byte o of stripe s's rows) is stream byte
// j*(p-1)*R + s*(p-1)*U + r*g_s + o (stripe geometry: kvec_internal.h); with
// R, U and so g_s multiples of the record size, its record is
// j*(recs per shard) + (s*(p-1)*U + r*g_s)/rec + o/rec.
// Each cell is loaded from the pool once, stored to its data shard and folded
// into P and Q in registers.  A thread owns one lane offset and a block is one
// wave.  Shards go in groups of paged_group(p, k) (18 cells for p = 7): the
// group's page-table entries are all requested, then all its cells, then the
// cells are stored and folded; scheduling barriers keep each phase's loads
// together (left to itself the compiler interleaves them with their uses and
// waits on each in turn).  Groups of 3 shards measured fastest for p = 7
// (whole-stripe groups, 2-shard groups and groups whose page-table loads ride
// with the previous group's cells were 1-3 % slower).
constexpr int kFBS = 64;
static_assert(kFBS * 16 == kRdpWaveBytes, "one wave per 1 KiB of a stripe row");

constexpr int paged_group(int P, int K) {
    const int g = 18 / (P - 1);
    return g < 1 ? 1 : (g > K ? K : g);
}

template <int P, int K>
__global__ __launch_bounds__(kFBS) __attribute__((amdgpu_waves_per_eu(1, 2))) void rdp_encode_paged_kernel(
        PagedGeom g, Ptrs<16> d, uint8_t* __restrict__ Pp, uint8_t* __restrict__ Qp, RdpGeom geo,
        uint32_t nb, uint32_t recs_per_shard) {
    constexpr int ROWS = P - 1, G = paged_group(P, K);
    const RdpWave w = rdp_wave(geo, ROWS, blockIdx.x, threadIdx.x);
    if (w.within >= w.g) return;
    const uint32_t off = w.within;
    const uint32_t w0 = fdiv(off, g.div_rec);
    const uint32_t inner = off - w0 * g.div_rec.d;
    // per lane: the record of (shard 0, row 0); row r adds r * g_rec records
    const uint32_t lane_rec = fdiv(uint32_t(w.base), g.div_rec) + w0;
    const uint32_t g_rec = fdiv(uint32_t(w.g), g.div_rec);
    auto rec = [&](int j, int r) { return uint32_t(j) * recs_per_shard + uint32_t(r) * g_rec + lane_rec; };
    const uint32_t rb = uint32_t(w.base), rg = uint32_t(w.g);
    RdpAcc<P> pr[ROWS], q[ROWS];
#pragma unroll
    for (int j0 = 0; j0 < K; j0 += G) {
        CellRef ref[G][ROWS];
#pragma unroll
        for (int gg = 0; gg < G; ++gg)
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
                if (j0 + gg < K) ref[gg][r] = cell_ref(g, rec(j0 + gg, r));
        __builtin_amdgcn_sched_barrier(0);
        u32x4 x[G][ROWS];
#pragma unroll
        for (int gg = 0; gg < G; ++gg)
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
                if (j0 + gg < K) x[gg][r] = cell_load_ref(g, ref[gg][r], inner);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            const int j = j0 + gg;
            if (j >= K) break;
            const ShardView<true> sv(d.p[j], nb);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                sv.store(rb + r * rg, off, x[gg][r]);
                pr[r].add(x[gg][r]);
                const int dg = (r + j) % P;
                if (dg != P - 1) q[dg].add(x[gg][r]);
            }
        }
        // Keep the next group's loads (page-table entries included) behind
        // this fold: a compiler memory barrier for the IR passes, which would
        // otherwise hoist every group's page-table loads to the top, and a
        // scheduling barrier for the machine scheduler.
        if constexpr (G < K) {
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // The P cell of row r lies on diagonal (r + p - 1) % p = r - 1.
    const ShardView<true> sp(Pp, nb), sq(Qp, nb);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const u32x4 pv = pr[r].get();
        sp.store(rb + r * rg, off, pv);
        if (r >= 1) q[r - 1].add(pv);
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) sq.store(rb + r * rg, off, q[r].get());
}

// ------------------------------------------------- fused RDP decode into the pool
// The inverse of the fused encode: up to two lost shards of the stripe set
// are rebuilt, lost data cells straight into their pool pages (and into the
// data shard buffers when the caller keeps them), lost P / Q cells into the
// parity buffers.  Surviving data cells are read from the pool (the pool is
// the primary copy of the data) or, when the caller passes the data shard
// buffers, from those; padding cells past the stream read as zero and are
// never stored.
//
// p = 7, k = 6 without data buffers (the KV chunk stripes) runs the
// erasure pattern's XOR map solved at compile time, in the shape of the
// fused encode: every needed cell's page-table entry is requested, then every
// cell, then the straight-line network; anything else runs the map from the
// kernel argument, one output at a time (re-read inputs hit the cache).
template <int P, int K, int E0, int E1>
__global__ __launch_bounds__(kFBS) __attribute__((amdgpu_waves_per_eu(1, 2))) void rdp_decode_paged_kernel(
        PagedGeom g, uint8_t* __restrict__ Pp, uint8_t* __restrict__ Qp, RdpGeom geo, uint32_t nb,
        uint32_t recs_per_shard) {
    constexpr int ROWS = P - 1, NC = (K + 2) * ROWS;
    constexpr RdpPlan plan = make_rdp_plan(P, K, E0, E1);
    static_assert(plan.ok, "RDP erasure pattern not decodable");
    constexpr RdpSched sch = make_rdp_sched(plan);
    const RdpWave w = rdp_wave(geo, ROWS, blockIdx.x, threadIdx.x);
    if (w.within >= w.g) return;
    const uint32_t off = w.within;
    const uint32_t w0 = fdiv(off, g.div_rec);
    const uint32_t inner = off - w0 * g.div_rec.d;
    const uint32_t lane_rec = fdiv(uint32_t(w.base), g.div_rec) + w0;
    const uint32_t g_rec = fdiv(uint32_t(w.g), g.div_rec);
    auto rec = [&](int c) {
        return uint32_t(c / ROWS) * recs_per_shard + uint32_t(c % ROWS) * g_rec + lane_rec;
    };
    auto needed = [&](int c) { return (plan.need[c >> 6] >> (c & 63)) & 1; };
    const uint32_t rb = uint32_t(w.base), rg = uint32_t(w.g);
    CellRef ref[NC], refo[plan.nout];
#pragma unroll
    for (int c = 0; c < K * ROWS; ++c)
        if (needed(c)) ref[c] = cell_ref(g, rec(c));
#pragma unroll
    for (int o = 0; o < plan.nout; ++o)
        if (plan.out_cell[o] < K * ROWS) refo[o] = cell_ref(g, rec(plan.out_cell[o]));
    __builtin_amdgcn_sched_barrier(0);
    const ShardView<true> sp(Pp, nb), sq(Qp, nb);
    u32x4 x[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (!needed(c)) continue;
        const int s = c / ROWS, r = c % ROWS;
        x[c] = s < K ? cell_load_ref(g, ref[c], inner) : (s == K ? sp : sq).load(rb + r * rg, off);
    }
    __builtin_amdgcn_sched_barrier(0);
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
        const int c = plan.out_cell[o], s = c / ROWS, r = c % ROWS;
        if (s < K) cell_store_ref(g, refo[o], inner, acc[o]);
        else (s == K ? sp : sq).store(rb + r * rg, off, acc[o]);
    }
}

__global__ __launch_bounds__(kFBS) void rdp_decode_paged_generic(PagedGeom g, Ptrs<16> d, uint8_t* Pp,
                                                                 uint8_t* Qp, RdpGeom geo, int rows, int k,
                                                                 RdpPlan plan, uint32_t recs_per_shard) {
    const RdpWave w = rdp_wave(geo, rows, blockIdx.x, threadIdx.x);
    if (w.within >= w.g) return;
    const uint32_t off = w.within;
    const uint32_t w0 = fdiv(off, g.div_rec);
    const uint32_t inner = off - w0 * g.div_rec.d;
    const uint32_t lane_rec = fdiv(uint32_t(w.base), g.div_rec) + w0;
    const uint32_t g_rec = fdiv(uint32_t(w.g), g.div_rec);
    const bool bufs = d.p[0] != nullptr;
    auto place = [&](int s, int r) { return w.base + uint64_t(r) * w.g + off; };
    for (int o = 0; o < plan.nout; ++o) {
        u32x4 acc = {0, 0, 0, 0};
        for (int wd = 0; wd < kRdpNW; ++wd) {
            uint64_t msk = plan.mask[o][wd];
            while (msk) {
                const int c = wd * 64 + __builtin_ctzll(msk);
                msk &= msk - 1;
                const int s = c / rows, r = c - s * rows;
                if (s < k)
                    acc ^= bufs ? ld16(d.p[s] + place(s, r))
                                : cell_load(g, uint32_t(s) * recs_per_shard + uint32_t(r) * g_rec + lane_rec,
                                            inner);
                else
                    acc ^= ld16((s == k ? Pp : Qp) + place(s, r));
            }
        }
        const int c = plan.out_cell[o], s = c / rows, r = c - s * rows;
        if (s < k) {
            cell_store(g, uint32_t(s) * recs_per_shard + uint32_t(r) * g_rec + lane_rec, inner, acc);
            if (bufs) st_stream(d.p[s], place(s, r), acc);
        } else {
            st_stream(s == k ? Pp : Qp, place(s, r), acc);
        }
    }
}

typedef void (*PagedDecFn)(PagedGeom, uint8_t*, uint8_t*, RdpGeom, uint32_t, uint32_t);

template <int E0, int E1>
PagedDecFn pick_paged_dec76(int e1) {
    if constexpr (E1 > 7) {
        return nullptr;
    } else {
        if (e1 == E1) return &rdp_decode_paged_kernel<7, 6, E0, E1>;
        return pick_paged_dec76<E0, E1 + 1>(e1);
    }
}

template <int E0 = 0>
PagedDecFn paged_dec76(int e0, int e1) {
    if constexpr (E0 > 7) {
        return nullptr;
    } else {
        if (e0 == E0) {
            if (e1 < 0) return &rdp_decode_paged_kernel<7, 6, E0, -1>;
            return pick_paged_dec76<E0, E0 + 1>(e1);
        }
        return paged_dec76<E0 + 1>(e0, e1);
    }
}

typedef void (*PagedEncFn)(PagedGeom, Ptrs<16>, uint8_t*, uint8_t*, RdpGeom, uint32_t, uint32_t);

template <int P, int K = 1>
PagedEncFn pick_paged(int k) {
    // p = 13 with k >= 10 would need more registers than a wave has and spill
    // to scratch (spilled code has produced wrong bytes on this hardware), so
    // those codes are not built here.
    if constexpr (K > P - 1 || (P == 13 && K >= 10)) {
        return nullptr;
    } else {
        if (k == K) return &rdp_encode_paged_kernel<P, K>;
        return pick_paged<P, K + 1>(k);
    }
}

static PagedEncFn paged_fn(int p, int k) {
    switch (p) {
        case 3: return pick_paged<3>(k);
        case 5: return pick_paged<5>(k);
        case 7: return pick_paged<7>(k);
        case 11: return pick_paged<11>(k);
        case 13: return pick_paged<13>(k);
        default: return nullptr;
    }
}

}  // namespace kvec

using namespace kvec;

extern "C" int64_t kvec_kv_stream_bytes(const kvec_paged_kv* kv) {
    if (!kv) return -1;
    return int64_t(kv->layers) * kv->batch * int64_t(kv->tokens) * 2 * kv->token_bytes;
}

extern "C" int kvec_kv_gather(const kvec_paged_kv* kv, void* out, void* stream) {
    PagedGeom g;
    int rc = make_geom(kv, &g, "kvec_kv_gather");
    if (rc) return rc;
    if (!out || !aligned16(out)) return set_error(KVEC_EINVAL, "kvec_kv_gather: output null or misaligned");
    const uint32_t ncells = uint32_t(g.recs_total * g.rec / 16);
    if (ncells == 0) return KVEC_OK;
    const Span w[1] = {{out, uint64_t(ncells) * 16, "out", -1}}, r[2] = {pool_span(kv), table_span(kv)};
    if ((rc = check_no_alias(w, 1, r, 2, "kvec_kv_gather"))) return rc;
    hipLaunchKernelGGL(kv_gather_kernel, dim3(blocks_for(ncells, kGBS)), dim3(kGBS), 0,
                       as_stream(stream), g, (uint8_t*)out, ncells);
    return check_launch("kvec_kv_gather");
}

extern "C" int kvec_kv_gather_split(const kvec_paged_kv* kv, void* out_k, void* out_v, void* stream) {
    PagedGeom g;
    int rc = make_geom(kv, &g, "kvec_kv_gather_split");
    if (rc) return rc;
    if (!out_k || !out_v || !aligned16(out_k) || !aligned16(out_v))
        return set_error(KVEC_EINVAL, "kvec_kv_gather_split: output null or misaligned");
    const uint32_t ncells = uint32_t(g.recs_total * g.rec / 16);
    if (ncells == 0) return KVEC_OK;
    const uint64_t half = uint64_t(ncells) * 8;
    const Span w[2] = {{out_k, half, "out_k", -1}, {out_v, half, "out_v", -1}},
               r[2] = {pool_span(kv), table_span(kv)};
    if ((rc = check_no_alias(w, 2, r, 2, "kvec_kv_gather_split"))) return rc;
    hipLaunchKernelGGL(kv_gather_split_kernel, dim3(blocks_for(ncells, kGBS)), dim3(kGBS), 0,
                       as_stream(stream), g, (uint8_t*)out_k, (uint8_t*)out_v, ncells,
                       uint32_t(kv->token_bytes));
    return check_launch("kvec_kv_gather_split");
}

extern "C" int kvec_kv_scatter(const kvec_paged_kv* kv, void* pool, const void* in, void* stream) {
    PagedGeom g;
    int rc = make_geom(kv, &g, "kvec_kv_scatter");
    if (rc) return rc;
    if (!pool || pool != kv->pool) return set_error(KVEC_EINVAL, "kvec_kv_scatter: pool must be kv->pool");
    if (!in || !aligned16(in)) return set_error(KVEC_EINVAL, "kvec_kv_scatter: input null or misaligned");
    const uint32_t ncells = uint32_t(g.recs_total * g.rec / 16);
    if (ncells == 0) return KVEC_OK;
    const Span w[1] = {pool_span(kv)}, r[2] = {{in, uint64_t(ncells) * 16, "in", -1}, table_span(kv)};
    if ((rc = check_no_alias(w, 1, r, 2, "kvec_kv_scatter"))) return rc;
    hipLaunchKernelGGL(kv_scatter_kernel, dim3(blocks_for(ncells, kGBS)), dim3(kGBS), 0,
                       as_stream(stream), g, (const uint8_t*)in, ncells);
    return check_launch("kvec_kv_scatter");
}

extern "C" int kvec_rdp_encode_paged(const kvec_paged_kv* kv, void* const* data, int k, void* P,
                                     void* Q, int p, int64_t row_bytes, int64_t unit_bytes, void* stream) {
    PagedGeom g;
    int rc = make_geom(kv, &g, "kvec_rdp_encode_paged");
    if (rc) return rc;
    if (!is_prime(p) || p < 3 || p > 13 || k < 1 || k > p - 1)
        return set_error(KVEC_EINVAL, "kvec_rdp_encode_paged: p=%d k=%d", p, k);
    if (row_bytes <= 0 || row_bytes % (2 * kv->token_bytes))
        return set_error(KVEC_EINVAL,
                         "kvec_rdp_encode_paged: row_bytes=%lld must be a multiple of 2*token_bytes",
                         (long long)row_bytes);
    if (unit_bytes < 0 || unit_bytes % kRdpWaveBytes || unit_bytes % (2 * kv->token_bytes))
        return set_error(KVEC_EINVAL,
                         "kvec_rdp_encode_paged: unit_bytes=%lld must be 0 or a multiple of 1024 and "
                         "of 2*token_bytes", (long long)unit_bytes);
    if (!fits_buffer(uint64_t(p - 1) * uint64_t(row_bytes)))
        return set_error(KVEC_EUNSUPPORTED, "kvec_rdp_encode_paged: shards must be < 4 GiB");
    const uint64_t stream_bytes = g.recs_total * g.rec;
    if (uint64_t(k) * (p - 1) * uint64_t(row_bytes) < stream_bytes)
        return set_error(KVEC_EINVAL, "kvec_rdp_encode_paged: k*(p-1)*row_bytes < stream bytes");
    if (uint64_t(k) * (p - 1) * uint64_t(row_bytes) / g.rec >= (uint64_t(1) << 32))
        return set_error(KVEC_EUNSUPPORTED, "kvec_rdp_encode_paged: stripe too large for 32-bit records");
    if (!data || !P || !Q || !aligned16(P) || !aligned16(Q))
        return set_error(KVEC_EINVAL, "kvec_rdp_encode_paged: null or misaligned parity");
    Ptrs<16> d{};
    for (int j = 0; j < k; ++j) {
        if (!data[j] || !aligned16(data[j]))
            return set_error(KVEC_EINVAL, "kvec_rdp_encode_paged: data[%d] null or misaligned", j);
        d.p[j] = (uint8_t*)data[j];
    }
    const uint64_t nb = uint64_t(p - 1) * uint64_t(row_bytes);
    {
        Span w[kRdpMaxShards];
        const Span r[2] = {pool_span(kv), table_span(kv)};
        for (int j = 0; j < k; ++j) w[j] = Span{data[j], nb, "data", j};
        w[k] = Span{P, nb, "P", -1};
        w[k + 1] = Span{Q, nb, "Q", -1};
        if ((rc = check_no_alias(w, k + 2, r, 2, "kvec_rdp_encode_paged"))) return rc;
    }
    PagedEncFn fn = paged_fn(p, k);
    if (!fn) return set_error(KVEC_EUNSUPPORTED, "kvec_rdp_encode_paged: p=%d k=%d not built", p, k);
    const RdpGeom geo = make_rdp_geom(uint64_t(row_bytes), uint64_t(unit_bytes));
    hipLaunchKernelGGL(fn, dim3(unsigned(rdp_waves(geo))), dim3(kFBS), 0, as_stream(stream), g, d,
                       (uint8_t*)P, (uint8_t*)Q, geo, uint32_t(nb), uint32_t(nb / g.rec));
    return check_launch("kvec_rdp_encode_paged");
}

extern "C" int kvec_rdp_decode_paged(const kvec_paged_kv* kv, void* pool, void* const* data, int k,
                                     void* P, void* Q, int p, int64_t row_bytes, int64_t unit_bytes,
                                     int e0, int e1, void* stream) {
    PagedGeom g;
    int rc = make_geom(kv, &g, "kvec_rdp_decode_paged");
    if (rc) return rc;
    if (!pool || pool != kv->pool)
        return set_error(KVEC_EINVAL, "kvec_rdp_decode_paged: pool must be kv->pool");
    if (!is_prime(p) || p < 3 || p > 13 || k < 1 || k > p - 1)
        return set_error(KVEC_EINVAL, "kvec_rdp_decode_paged: p=%d k=%d", p, k);
    if (row_bytes <= 0 || row_bytes % (2 * kv->token_bytes))
        return set_error(KVEC_EINVAL,
                         "kvec_rdp_decode_paged: row_bytes=%lld must be a multiple of 2*token_bytes",
                         (long long)row_bytes);
    if (unit_bytes < 0 || unit_bytes % kRdpWaveBytes || unit_bytes % (2 * kv->token_bytes))
        return set_error(KVEC_EINVAL,
                         "kvec_rdp_decode_paged: unit_bytes=%lld must be 0 or a multiple of 1024 and "
                         "of 2*token_bytes", (long long)unit_bytes);
    if (!fits_buffer(uint64_t(p - 1) * uint64_t(row_bytes)))
        return set_error(KVEC_EUNSUPPORTED, "kvec_rdp_decode_paged: shards must be < 4 GiB");
    const uint64_t stream_bytes = g.recs_total * g.rec;
    if (uint64_t(k) * (p - 1) * uint64_t(row_bytes) < stream_bytes)
        return set_error(KVEC_EINVAL, "kvec_rdp_decode_paged: k*(p-1)*row_bytes < stream bytes");
    if (uint64_t(k) * (p - 1) * uint64_t(row_bytes) / g.rec >= (uint64_t(1) << 32))
        return set_error(KVEC_EUNSUPPORTED, "kvec_rdp_decode_paged: stripe too large for 32-bit records");
    if (!P || !Q || !aligned16(P) || !aligned16(Q))
        return set_error(KVEC_EINVAL, "kvec_rdp_decode_paged: null or misaligned parity");
    if (e0 < -1 || e0 > k + 1 || e1 < -1 || e1 > k + 1)
        return set_error(KVEC_EINVAL, "kvec_rdp_decode_paged: erased index out of [-1, %d]", k + 1);
    Ptrs<16> d{};
    if (data) {
        for (int j = 0; j < k; ++j) {
            if (!data[j] || !aligned16(data[j]))
                return set_error(KVEC_EINVAL, "kvec_rdp_decode_paged: data[%d] null or misaligned", j);
            d.p[j] = (uint8_t*)data[j];
        }
    }
    int a = e0, b = e1;
    if (a == b) b = -1;
    if (a < 0) { a = b; b = -1; }
    if (b >= 0 && b < a) { int t = a; a = b; b = t; }
    if (a < 0) return KVEC_OK;
    const uint64_t nb = uint64_t(p - 1) * uint64_t(row_bytes);
    {
        // the pool, P, Q and the data shards are each read and may be
        // rewritten, so none may share a byte with another
        Span w[kRdpMaxShards + 1];
        const Span r[1] = {table_span(kv)};
        int nw = 0;
        w[nw++] = pool_span(kv);
        w[nw++] = Span{P, nb, "P", -1};
        w[nw++] = Span{Q, nb, "Q", -1};
        if (data)
            for (int j = 0; j < k; ++j) w[nw++] = Span{data[j], nb, "data", j};
        if ((rc = check_no_alias(w, nw, r, 1, "kvec_rdp_decode_paged"))) return rc;
    }
    const RdpGeom geo = make_rdp_geom(uint64_t(row_bytes), uint64_t(unit_bytes));
    const dim3 grid(unsigned(rdp_waves(geo))), block(kFBS);
    const uint32_t rps = uint32_t(nb / g.rec);
    PagedDecFn fn = (p == 7 && k == 6 && !data) ? paged_dec76(a, b) : nullptr;
    if (fn) {
        hipLaunchKernelGGL(fn, grid, block, 0, as_stream(stream), g, (uint8_t*)P, (uint8_t*)Q, geo,
                           uint32_t(nb), rps);
    } else {
        RdpPlan plan = make_rdp_plan(p, k, a, b);
        if (!plan.ok)
            return set_error(KVEC_EDECODE, "kvec_rdp_decode_paged: pattern (%d, %d) not decodable", a, b);
        hipLaunchKernelGGL(rdp_decode_paged_generic, grid, block, 0, as_stream(stream), g, d, (uint8_t*)P,
                           (uint8_t*)Q, geo, p - 1, k, plan, rps);
    }
    return check_launch("kvec_rdp_decode_paged");
}
