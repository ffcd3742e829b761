// paged_geom.h -- addressing of a paged KV pool, shared by the gather,
// scatter and fused coding kernels.
//
// Pool: [layers][pool_pages][page_tokens][2 (K,V)][token_bytes].  The coding
// stream of a chunk of `tokens` positions starting at tok_off holds the
// chunk's token records in order, [layers][batch][tokens][2][token_bytes].
// A stream byte s maps to (record w = s / record_bytes, inner byte); w to
// (layer, b, t) by two invariant-divisor divisions; the slot comes from the
// page table.  token_bytes is a multiple of 16, so a 16-byte cell never
// straddles two records.  Page-table entries outside [0, pool_pages) read as
// zero pages (the kernels never address outside the pool).
#pragma once

#include "kvec_internal.h"

namespace kvec {

struct PagedGeom {
    const uint8_t* pool;
    uint8_t* pool_w;            // same pool, for the scatter
    const int32_t* table;       // [batch][pps]
    uint64_t layer_stride;      // pool_pages * page_tokens * record bytes
    uint32_t layer_recs;        // pool_pages * page_tokens
    uint64_t recs_total;        // layers * batch * tokens
    uint32_t rec, pps, tok_off, page_shift, pool_pages;
    FastDiv div_rec, div_t, div_b, div_cells;  // div_cells: record_bytes / 16
};

// Byte offset in the pool of the 16-byte stream cell in record w at byte
// `inner`.  Branch-free, so that a thread's many cell loads can all be in
// flight at once: a padding record (w >= recs_total) or an invalid page-table
// entry yields the offset of a cell of pool page 0 and valid = false.
__device__ __forceinline__ uint64_t cell_offset(const PagedGeom& g, uint32_t w, uint32_t inner,
                                                bool& valid) {
    valid = w < g.recs_total;
    const uint32_t ww = valid ? w : 0u;
    const uint32_t lb = fdiv(ww, g.div_t);
    const uint32_t t = ww - lb * g.div_t.d + g.tok_off;
    const uint32_t layer = fdiv(lb, g.div_b);
    const uint32_t b = lb - layer * g.div_b.d;
    const uint32_t page = uint32_t(g.table[b * g.pps + (t >> g.page_shift)]);
    valid = valid && page < g.pool_pages;
    const uint32_t pg = valid ? page : 0u;
    const uint64_t slot = (uint64_t(pg) << g.page_shift) | (t & ((1u << g.page_shift) - 1));
    return uint64_t(layer) * g.layer_stride + slot * g.rec + inner;
}

// 16 zero bytes that invalid cells are read from: choosing the address before
// the load (instead of zeroing the loaded value after it) keeps the validity
// test off the load's critical path, so a thread's cell loads issue back to back.
__device__ __attribute__((aligned(16))) uint32_t kZeroCell[4] = {0, 0, 0, 0};  // never written

// The cell's 16 bytes (zero for padding records and invalid pages).
__device__ __forceinline__ u32x4 cell_load(const PagedGeom& g, uint32_t w, uint32_t inner) {
    bool valid;
    const uint64_t off = cell_offset(g, w, inner, valid);
    const uint8_t* a = valid ? g.pool + off : reinterpret_cast<const uint8_t*>(kZeroCell);
    return ld_stream(a, 0);
}

// Split access for kernels that keep several cells in flight per thread:
// cell_ref issues the page-table load of a cell and keeps, in two VGPRs, the
// entry and the cell's record index with page 0 (its layer and in-page token),
// kNoCell for padding records; cell_load_ref / cell_store_ref finish the access.
// Issuing the refs of a later row before the cells of an earlier one keeps both
// kinds of load in flight.  Everything stays per lane: no wave-uniform values
// are held across the phases (spilled SGPRs have given run-to-run different
// results in these kernels).
constexpr uint32_t kNoCell = 0xFFFFFFFFu;

struct CellRef {
    uint32_t base;  // layer * layer_recs + in-page token, or kNoCell
    uint32_t page;  // page-table entry (any value; checked on use)
};

__device__ __forceinline__ CellRef cell_ref(const PagedGeom& g, uint32_t w) {
    const bool valid = w < g.recs_total;
    const uint32_t ww = valid ? w : 0u;
    const uint32_t lb = fdiv(ww, g.div_t);
    const uint32_t t = ww - lb * g.div_t.d + g.tok_off;
    const uint32_t layer = fdiv(lb, g.div_b);
    const uint32_t b = lb - layer * g.div_b.d;
    const uint32_t page = uint32_t(g.table[b * g.pps + (t >> g.page_shift)]);
    return CellRef{valid ? layer * g.layer_recs + (t & ((1u << g.page_shift) - 1)) : kNoCell, page};
}

// cell_ref for the lanes of one wave whose records are rec0 + d, with rec0
// wave-uniform and 0 <= d <= dmax per lane (the 16-byte cells of one 1 KiB
// stream piece).  When the whole run lies in one sequence's tokens of one
// layer and before the padding, the record's (layer, sequence, token) is
// decomposed once for the wave in scalar registers and each lane only adds
// its token offset; otherwise every lane decomposes its own record.
__device__ __forceinline__ CellRef cell_ref_run(const PagedGeom& g, uint32_t rec0, uint32_t d,
                                                uint32_t dmax) {
    const uint32_t lb = fdiv(rec0, g.div_t);
    const uint32_t t0 = rec0 - lb * g.div_t.d;
    const uint32_t nrec = uint32_t(g.recs_total);  // < 2^32 (make_geom)
    if (t0 + dmax < g.div_t.d && nrec > dmax && rec0 < nrec - dmax) {
        const uint32_t layer = fdiv(lb, g.div_b);
        const uint32_t b = lb - layer * g.div_b.d;
        const uint32_t t = t0 + g.tok_off + d;
        const int32_t* row = g.table + b * g.pps;
        return CellRef{layer * g.layer_recs + (t & ((1u << g.page_shift) - 1)), uint32_t(row[t >> g.page_shift])};
    }
    return cell_ref(g, rec0 + d);
}

__device__ __forceinline__ bool cell_valid(const PagedGeom& g, const CellRef& c) {
    return c.base != kNoCell && c.page < g.pool_pages;
}

__device__ __forceinline__ uint64_t cell_ref_offset(const PagedGeom& g, const CellRef& c, uint32_t inner) {
    return uint64_t(c.base + (c.page << g.page_shift)) * g.rec + inner;
}

__device__ __forceinline__ u32x4 cell_load_ref(const PagedGeom& g, const CellRef& c, uint32_t inner) {
    const uint8_t* a = cell_valid(g, c) ? g.pool + cell_ref_offset(g, c, inner)
                                        : reinterpret_cast<const uint8_t*>(kZeroCell);
    return ld_stream(a, 0);
}

__device__ __forceinline__ void cell_store_ref(const PagedGeom& g, const CellRef& c, uint32_t inner,
                                               u32x4 v) {
    if (cell_valid(g, c)) st_stream(g.pool_w, cell_ref_offset(g, c, inner), v);
}

// Write the cell (padding records and invalid pages are skipped).
__device__ __forceinline__ void cell_store(const PagedGeom& g, uint32_t w, uint32_t inner, u32x4 v) {
    bool valid;
    const uint64_t off = cell_offset(g, w, inner, valid);
    if (valid) st_stream(g.pool_w, off, v);
}

// The whole pool and the page table, for the alias checks (after make_geom).
inline Span pool_span(const kvec_paged_kv* kv) {
    return Span{kv->pool, uint64_t(kv->layers) * uint64_t(kv->pool_pages) * uint64_t(kv->page_tokens) * 2 *
                              uint64_t(kv->token_bytes),
                "pool", -1};
}
inline Span table_span(const kvec_paged_kv* kv) {
    return Span{kv->page_table, uint64_t(kv->batch) * uint64_t(kv->pages_per_seq) * 4, "page_table", -1};
}

inline int make_geom(const kvec_paged_kv* kv, PagedGeom* g, const char* fn) {
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
        kv->pool_pages >= (int64_t(1) << 31) || recs * rec / 16 >= (uint64_t(1) << 32) ||
        int64_t(kv->batch) * kv->pages_per_seq >= (int64_t(1) << 31) ||
        uint64_t(kv->layers) * uint64_t(kv->pool_pages) * uint64_t(kv->page_tokens) >= kNoCell)
        return set_error(KVEC_EUNSUPPORTED, "%s: chunk too large for 32-bit cell indices", fn);
    g->pool = (const uint8_t*)kv->pool;
    g->pool_w = (uint8_t*)kv->pool;
    g->table = kv->page_table;
    g->layer_stride = uint64_t(kv->pool_pages) * kv->page_tokens * rec;
    g->layer_recs = uint32_t(uint64_t(kv->pool_pages) * kv->page_tokens);
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
