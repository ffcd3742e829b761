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
// contiguous 1 KiB of a pool page.
//
// A stream byte s maps to (record w = s / record_bytes, inner byte); w to
// (layer, b, t) by two invariant-divisor divisions; the slot comes from the
// page table.  token_bytes is a multiple of 16, so a 16-byte cell never
// straddles two records.  Page-table entries outside [0, pool_pages) read as
// zero pages (the kernels never address outside the pool).
#include "kvec_internal.h"

namespace kvec {

struct PagedGeom {
    const uint8_t* pool;
    uint8_t* pool_w;            // same pool, for the scatter
    const int32_t* table;       // [batch][pps]
    uint64_t layer_stride;      // pool_pages * page_tokens * record bytes
    uint64_t recs_total;        // layers * batch * tokens
    uint32_t rec, pps, tok_off, page_shift, pool_pages;
    FastDiv div_rec, div_t, div_b, div_cells;  // div_cells: record_bytes / 16
};

// Source address of the 16-byte stream cell in record w at byte `inner`;
// nullptr for padding records and invalid page-table entries.
__device__ __forceinline__ const uint8_t* cell_src(const PagedGeom& g, uint32_t w, uint32_t inner) {
    if (w >= g.recs_total) return nullptr;
    const uint32_t lb = fdiv(w, g.div_t);
    const uint32_t t = w - lb * g.div_t.d + g.tok_off;
    const uint32_t layer = fdiv(lb, g.div_b);
    const uint32_t b = lb - layer * g.div_b.d;
    const int32_t page = g.table[uint64_t(b) * g.pps + (t >> g.page_shift)];
    if (page < 0 || uint32_t(page) >= g.pool_pages) return nullptr;
    const uint64_t slot = (uint64_t(uint32_t(page)) << g.page_shift) | (t & ((1u << g.page_shift) - 1));
    return g.pool + uint64_t(layer) * g.layer_stride + slot * g.rec + inner;
}

__device__ __forceinline__ uint8_t* cell_dst(const PagedGeom& g, uint32_t w, uint32_t inner) {
    return const_cast<uint8_t*>(cell_src(g, w, inner)) - g.pool + g.pool_w;
}

constexpr int kGBS = 256;

// stream[s] = pool cell, one 16-byte cell per thread
__global__ __launch_bounds__(kGBS) void kv_gather_kernel(PagedGeom g, uint8_t* __restrict__ out,
                                                         uint32_t ncells) {
    const uint32_t c = blockIdx.x * kGBS + threadIdx.x;
    if (c >= ncells) return;
    const uint32_t w = fdiv(c, g.div_cells);
    const uint32_t inner = (c - w * g.div_cells.d) * 16;
    const uint8_t* src = cell_src(g, w, inner);
    const u32x4 v = src ? ld_stream(src, 0) : u32x4{0, 0, 0, 0};
    st_stream(out, uint64_t(c) * 16, v);
}

// pool cell = stream[s] (inverse; padding slots and invalid pages are skipped)
__global__ __launch_bounds__(kGBS) void kv_scatter_kernel(PagedGeom g, const uint8_t* __restrict__ in,
                                                          uint32_t ncells) {
    const uint32_t c = blockIdx.x * kGBS + threadIdx.x;
    if (c >= ncells) return;
    const uint32_t w = fdiv(c, g.div_cells);
    const uint32_t inner = (c - w * g.div_cells.d) * 16;
    if (!cell_src(g, w, inner)) return;
    st_stream(cell_dst(g, w, inner), 0, ld_stream(in, uint64_t(c) * 16));
}

// ------------------------------------------------- fused gather + RDP encode
// Stream cell (shard j, row r, lane offset o) is stream byte (j*(p-1) + r)*R + o;
// with R a multiple of the record size its record is (j*(p-1) + r)*(R/rec) + o/rec.
// The cell is loaded from the pool once, stored to its data shard and folded
// into P and Q in registers.
constexpr int kFBS = 128;

template <int P, int K>
__global__ __launch_bounds__(kFBS) void rdp_encode_paged_kernel(PagedGeom g, Ptrs<16> d,
                                                                uint8_t* __restrict__ Pp,
                                                                uint8_t* __restrict__ Qp, uint64_t R,
                                                                uint32_t recs_per_row, uint32_t nvec) {
    constexpr int ROWS = P - 1;
    const uint32_t u = blockIdx.x * kFBS + threadIdx.x;
    if (u >= nvec) return;
    const uint32_t off = u << 4;
    const uint32_t w0 = fdiv(off, g.div_rec);
    const uint32_t inner = off - w0 * g.rec;
    const uint64_t nb = ROWS * R;
    u32x4 pr[ROWS], q[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        pr[r] = u32x4{0, 0, 0, 0};
        q[r] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const ShardView<true> sv(d.p[j], nb);
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint32_t w = (j * ROWS + r) * recs_per_row + w0;
            const uint8_t* src = cell_src(g, w, inner);
            const u32x4 x = src ? ld_stream(src, 0) : u32x4{0, 0, 0, 0};
            sv.store(r * R, off, x);
            pr[r] ^= x;
            const int dg = (r + j) % P;
            if (dg != P - 1) q[dg] ^= x;
        }
    }
#pragma unroll
    for (int r = 1; r < ROWS; ++r) q[r - 1] ^= pr[r];
    const ShardView<true> sp(Pp, nb), sq(Qp, nb);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        sp.store(r * R, off, pr[r]);
        sq.store(r * R, off, q[r]);
    }
}

typedef void (*PagedEncFn)(PagedGeom, Ptrs<16>, uint8_t*, uint8_t*, uint64_t, uint32_t, uint32_t);

template <int P, int K = 1>
PagedEncFn pick_paged(int k) {
    if constexpr (K > P - 1) {
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

static int make_geom(const kvec_paged_kv* kv, PagedGeom* g, const char* fn) {
    if (!kv) return set_error(KVEC_EINVAL, "%s: null descriptor", fn);
    if (!kv->pool || !kv->page_table) return set_error(KVEC_EINVAL, "%s: null pool or page table", fn);
    if (kv->layers < 1 || kv->batch < 1 || kv->tokens < 0 || kv->tok_off < 0 || kv->pool_pages < 1 ||
        kv->pages_per_seq < 1)
        return set_error(KVEC_EINVAL, "%s: bad sizes", fn);
    if (kv->token_bytes < 16 || kv->token_bytes % 16 || kv->token_bytes > (int64_t(1) << 28))
        return set_error(KVEC_EINVAL, "%s: token_bytes=%lld must be a positive multiple of 16", fn,
                         (long long)kv->token_bytes);
    if (kv->page_tokens < 1 || (kv->page_tokens & (kv->page_tokens - 1)))
        return set_error(KVEC_EINVAL, "%s: page_tokens=%d must be a power of two", fn, kv->page_tokens);
    if (int64_t(kv->tok_off) + kv->tokens > int64_t(kv->pages_per_seq) * kv->page_tokens)
        return set_error(KVEC_EINVAL, "%s: tokens past the page table", fn);
    if (!aligned16(kv->pool)) return set_error(KVEC_EINVAL, "%s: pool not 16-byte aligned", fn);
    const uint64_t rec = 2 * uint64_t(kv->token_bytes);
    const uint64_t recs = uint64_t(kv->layers) * kv->batch * uint64_t(kv->tokens);
    if (recs >= (uint64_t(1) << 32) || uint64_t(kv->layers) * kv->batch >= (uint64_t(1) << 32) ||
        kv->pool_pages >= (int64_t(1) << 31) || recs * rec / 16 >= (uint64_t(1) << 32))
        return set_error(KVEC_EUNSUPPORTED, "%s: chunk too large for 32-bit cell indices", fn);
    g->pool = (const uint8_t*)kv->pool;
    g->pool_w = (uint8_t*)kv->pool;
    g->table = kv->page_table;
    g->layer_stride = uint64_t(kv->pool_pages) * kv->page_tokens * rec;
    g->recs_total = recs;
    g->rec = uint32_t(rec);
    g->pps = uint32_t(kv->pages_per_seq);
    g->tok_off = uint32_t(kv->tok_off);
    int sh = 0;
    while ((1 << sh) < kv->page_tokens) ++sh;
    g->page_shift = uint32_t(sh);
    g->pool_pages = uint32_t(kv->pool_pages);
    g->div_rec = make_fastdiv(g->rec);
    g->div_t = make_fastdiv(uint32_t(kv->tokens ? kv->tokens : 1));
    g->div_b = make_fastdiv(uint32_t(kv->batch));
    g->div_cells = make_fastdiv(g->rec / 16);
    return KVEC_OK;
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
    hipLaunchKernelGGL(kv_gather_kernel, dim3(blocks_for(ncells, kGBS)), dim3(kGBS), 0,
                       as_stream(stream), g, (uint8_t*)out, ncells);
    return check_launch("kvec_kv_gather");
}

extern "C" int kvec_kv_scatter(const kvec_paged_kv* kv, void* pool, const void* in, void* stream) {
    PagedGeom g;
    int rc = make_geom(kv, &g, "kvec_kv_scatter");
    if (rc) return rc;
    if (!pool || pool != kv->pool) return set_error(KVEC_EINVAL, "kvec_kv_scatter: pool must be kv->pool");
    if (!in || !aligned16(in)) return set_error(KVEC_EINVAL, "kvec_kv_scatter: input null or misaligned");
    const uint32_t ncells = uint32_t(g.recs_total * g.rec / 16);
    if (ncells == 0) return KVEC_OK;
    hipLaunchKernelGGL(kv_scatter_kernel, dim3(blocks_for(ncells, kGBS)), dim3(kGBS), 0,
                       as_stream(stream), g, (const uint8_t*)in, ncells);
    return check_launch("kvec_kv_scatter");
}

extern "C" int kvec_rdp_encode_paged(const kvec_paged_kv* kv, void* const* data, int k, void* P,
                                     void* Q, int p, int64_t row_bytes, void* stream) {
    PagedGeom g;
    int rc = make_geom(kv, &g, "kvec_rdp_encode_paged");
    if (rc) return rc;
    if (!is_prime(p) || p < 3 || p > 13 || k < 1 || k > p - 1)
        return set_error(KVEC_EINVAL, "kvec_rdp_encode_paged: p=%d k=%d", p, k);
    if (row_bytes <= 0 || row_bytes % (2 * kv->token_bytes))
        return set_error(KVEC_EINVAL,
                         "kvec_rdp_encode_paged: row_bytes=%lld must be a multiple of 2*token_bytes",
                         (long long)row_bytes);
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
    PagedEncFn fn = paged_fn(p, k);
    const uint32_t nvec = uint32_t(row_bytes / 16);
    const uint32_t spr = uint32_t(row_bytes / g.rec);
    hipLaunchKernelGGL(fn, dim3(blocks_for(nvec, kFBS)), dim3(kFBS), 0, as_stream(stream), g, d,
                       (uint8_t*)P, (uint8_t*)Q, uint64_t(row_bytes), spr, nvec);
    return check_launch("kvec_rdp_encode_paged");
}
