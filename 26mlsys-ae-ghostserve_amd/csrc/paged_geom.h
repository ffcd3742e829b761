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
