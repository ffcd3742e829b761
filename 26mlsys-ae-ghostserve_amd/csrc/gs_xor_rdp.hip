// gs_xor_rdp.hip -- the reference's XOR and star-diagonal "RDP" codes,
// bit-exact, on its packed [(rows), S] shard tensors.
//
//   XOR  benchmark/xor/kernel.cu:17-88 (+ pack/unpack :93-146 as copies)
//   RDP  benchmark/rdp/kernel.cu:32-345 and bench_ghostserve_rdp.py:105-150
//
// The column work runs on the tile engine (tile_engine.h).  The diagonal
// parity Q[d] = XOR_r D_r[(d - r) mod S] skips each row's star word in the
// same pass: the lane whose window holds it masks it before the XOR.
#include "tile_engine.h"

namespace kvec {

// ----------------------------------------------------------------- XOR rows
// out[c] = XOR of in rows {lo..hi-1} \ {skip}, plus row `extra` when >= 0.
struct RowSet {
    int lo, hi, skip, extra;
};

__device__ __forceinline__ u32x4 xor_rows_window(const uint8_t* in, uint64_t Sb, RowSet rs,
                                                 uint64_t c0) {
    u32x4 acc = {0, 0, 0, 0};
    for (int r = rs.lo; r < rs.hi; ++r)
        if (r != rs.skip) acc ^= load_window16(in + uint64_t(r) * Sb + c0);
    if (rs.extra >= 0) acc ^= load_window16(in + uint64_t(rs.extra) * Sb + c0);
    return acc;
}

__device__ __forceinline__ u32x4 xor_rows_partial(const uint8_t* in, uint64_t Sb, RowSet rs,
                                                  uint64_t c0, uint32_t n) {
    u32x4 acc = {0, 0, 0, 0};
    for (uint32_t i = 0; i < n; ++i) {
        uint8_t b = 0;
        for (int r = rs.lo; r < rs.hi; ++r)
            if (r != rs.skip) b ^= in[uint64_t(r) * Sb + c0 + i];
        if (rs.extra >= 0) b ^= in[uint64_t(rs.extra) * Sb + c0 + i];
        acc = set_byte(acc, i, b);
    }
    return acc;
}

// Whether a whole tile of `rs` can take the batched path with ND rows: rows
// 0..ND-1 (encode, or P recomputed), or rows 0..ND minus one data row (a data
// row rebuilt from P), in an `in` tensor of in_bytes < 2^31 (0: never).
template <int ND>
__device__ __forceinline__ bool xor_rows_batchable(RowSet rs, uint32_t in_bytes) {
    if (ND == 0 || in_bytes == 0 || rs.lo != 0 || rs.hi != ND) return false;
    return (rs.skip < 0 && rs.extra < 0) || (rs.skip >= 0 && rs.skip < ND && rs.extra == ND);
}

// XOR of the ND rows of one tile with every row's chunk requested at
// once.  Row i of the batch is row i of `in`, or i + 1 from the skipped row
// on.  Each lane loads its aligned chunk of the row; the next chunk, which a
// misaligned window reaches into, is the next lane's (DPP), and lane 63 loads
// it itself (other lanes' edge loads are out of range and read nothing).
// Offsets are taken from `in` rounded down to 16 bytes, so they are never
// negative, and the resource reaches to the end of the last 16-byte chunk
// holding a byte of `in`.  With fc.dst set, the owned chunks are copied as in
// the general path.
template <int ND>
__device__ __forceinline__ u32x4 xor_rows_batched(const uint8_t* in, uint32_t Sb, uint32_t in_bytes,
                                                  RowSet rs, const FlatCopy& fc) {
    const uint32_t b15 = uint32_t(reinterpret_cast<uintptr_t>(in)) & 15;
    const uint8_t* in_al = in - b15;
    const __amdgpu_buffer_rsrc_t rsin = chunk_rsrc(in_al, (b15 + in_bytes + 15) & ~15u);
    const uint32_t t0 = blockIdx.x * uint32_t(kTileBytes);
    const uint32_t lane = threadIdx.x & 63;
    auto row_a = [&](int i) {   // tile start of batch row i, from in_al
        const uint32_t j = uint32_t(i + (rs.skip >= 0 && i >= rs.skip ? 1 : 0));
        return b15 + j * Sb + t0;
    };
    u32x4 lo[ND], e1[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const uint32_t A = row_a(i), sh = A & 15;
        const uint32_t my = A - sh + 16 * threadIdx.x;
        lo[i] = chunk_load(rsin, my);
        e1[i] = chunk_load(rsin, lane == 63 && sh ? my + 16 : kNoLoad);
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const uint32_t A = row_a(i), sh = A & 15;
        const u32x4 hi = from_next_lane_or(lo[i], e1[i]);
        acc ^= sh ? funnel16(lo[i], hi, sh) : lo[i];
        if (fc.dst) {
            const uint8_t* c = in_al + (A - sh) + 16 * threadIdx.x;
            if (sh) copy_chunk(fc, c + 16, hi);
            else copy_chunk(fc, c, lo[i]);
        }
    }
    return acc;
}

// One tile of XOR-of-rows, written to up to two outputs (row base addresses).
// With fc.dst set, rows lo..hi-1 of `in` (the whole flat range of fc, no
// skip) are also copied to fc.dst by the same loads.  NT: non-temporal
// stores of the outputs.
template <int ND, bool NT = false>
__device__ __forceinline__ void xor_rows_tile(const uint8_t* in, uint64_t Sb, uint32_t in_bytes,
                                              RowSet rs, uint8_t* out0, uint8_t* out1,
                                              const FlatCopy& fc, uint8_t* tile) {
    const uint64_t t0 = uint64_t(blockIdx.x) * kTileBytes;
    const uint32_t nbytes = uint32_t(Sb - t0 < uint64_t(kTileBytes) ? Sb - t0 : kTileBytes);
    const uint64_t c0 = t0 + 16 * threadIdx.x;
    u32x4 acc = {0, 0, 0, 0};
    // Rows of at least one full tile take the batched path in every tile: in a
    // partial last tile the lanes past the row's end XOR bytes that are not
    // stored, and their copied chunks carry the next row's bytes (the values
    // its own tile copies) or lie past the copy range.
    const bool batched = Sb >= uint64_t(kTileBytes) && xor_rows_batchable<ND>(rs, in_bytes);
    if (batched) {
        if constexpr (ND > 0) acc = xor_rows_batched<ND>(in, uint32_t(Sb), in_bytes, rs, fc);
    } else if (t0 + kTileBytes <= Sb) {
        // whole tile inside the rows: uniform row windows, loads carry the copy
        const uint32_t off = 16 * threadIdx.x;
        for (int r = rs.lo; r < rs.hi; ++r) {
            if (r == rs.skip) continue;
            const RowWin rw = row_win(in + uint64_t(r) * Sb + t0);
            u32x4 lo, hi;
            win_chunks(rw, off, lo, hi);
            acc ^= win_join(rw, lo, hi);
            if (fc.dst) copy_owned(fc, rw, off, lo, hi);
        }
        if (rs.extra >= 0) acc ^= load_window16(in + uint64_t(rs.extra) * Sb + c0);
    } else if (c0 + 16 <= Sb) {
        acc = xor_rows_window(in, Sb, rs, c0);
    } else if (c0 < Sb) {
        acc = xor_rows_partial(in, Sb, rs, c0, uint32_t(Sb - c0));
    }
    if (fc.dst) {
        if (!batched && t0 + kTileBytes > Sb && c0 < Sb)
            for (int r = rs.lo; r < rs.hi; ++r)
                copy_bytes(fc, uint64_t(r) * Sb + c0, uint64_t(r) * Sb + (c0 + 16 < Sb ? c0 + 16 : Sb));
        if (t0 == 0 && threadIdx.x == 0)
            for (int r = rs.lo; r < rs.hi; ++r) copy_row_head(fc, uint64_t(r) * Sb, Sb);
    }
    *reinterpret_cast<u32x4*>(tile + 16 * threadIdx.x) = acc;
    __syncthreads();
    if (out0) tile_store<NT>(out0 + t0, tile, nbytes);
    if (out1) tile_store<NT>(out1 + t0, tile, nbytes);
}

template <int ND>
__global__ __launch_bounds__(kTB) void xor_rows_kernel(const uint8_t* in, uint64_t Sb, uint32_t in_bytes,
                                                       RowSet rs, uint8_t* out0, uint8_t* out1,
                                                       FlatCopy fc) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[kTileBytes + 16];
    xor_rows_tile<ND>(in, Sb, in_bytes, rs, out0, out1, fc, tile);
}

// benchmark/xor/kernel.cu:47-88 with the missing index read on the device:
// data row m < nd is P ^ the other data rows; m == nd recomputes P; anything
// else leaves every buffer untouched.
template <int ND>
__global__ __launch_bounds__(kTB) void xor_reconstruct_kernel(const uint8_t* enc, uint8_t* rec,
                                                              uint8_t* rec_missing, uint64_t Sb,
                                                              uint32_t in_bytes, int nd,
                                                              const int32_t* missing_idx) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[kTileBytes + 16];
    const int m = __builtin_amdgcn_readfirstlane(missing_idx[0]);
    RowSet rs;
    if (m >= 0 && m < nd)
        rs = RowSet{0, nd, m, nd};
    else if (m == nd)
        rs = RowSet{0, nd, -1, -1};
    else
        return;
    // non-temporal output stores: 121.2 against 130.2 us on the 512 MiB stream
    xor_rows_tile<ND, true>(enc, Sb, in_bytes, rs, rec + uint64_t(m) * Sb, rec_missing,
                            FlatCopy{nullptr, nullptr, 0}, tile);
}

// ------------------------------------------------------- XOR encode from K, V
// forward_encode_kv's pack (benchmark/xor/main.py:69-90: K bytes then V bytes,
// zero padding) and encode_xor (benchmark/xor/kernel.cu:17-41) in one pass:
// data row j of the shard tensor is bytes [j Sb, (j+1) Sb) of the stream
// K || V || zeros, and row ND their XOR.  The host runs it when the shards, K
// and V are 16-byte aligned and K's size kb is a multiple of 16, so every
// aligned 16-byte chunk of the stream lies in K, in V or in the padding: it is
// read through K's and V's buffer resources at once, the other load (and both,
// in the padding) out of range and reading nothing.  Each lane stores, to the
// data rows, the aligned chunk that starts inside its window (as the fused
// copy of xor_rows_batched does) up to the end of the data rows, and the XOR
// goes through LDS to row ND.  Rows hold at least one full tile; in a partial
// last tile the lanes past a row's end store the next row's chunks, the
// values that row's own tile stores.  kb < 2^30 and (ND + 1) Sb < 2^31.
constexpr int kKvTB = 256;                 // 201 against 195 us with 512-thread tiles
constexpr uint32_t kKvTile = 16 * kKvTB;

template <int ND>
__global__ __launch_bounds__(kKvTB) void xor_encode_kv_kernel(const uint8_t* K, const uint8_t* V,
                                                              uint32_t kb, uint8_t* sh, uint32_t Sb) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[kKvTile + 16];
    const uint32_t t0 = blockIdx.x * kKvTile;
    const uint32_t nbytes = Sb - t0 < kKvTile ? Sb - t0 : kKvTile;
    const uint32_t lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rk = chunk_rsrc(K, kb), rv = chunk_rsrc(V, kb);
    const uint32_t data_end = uint32_t(ND) * Sb;
    // the stream's aligned chunk at x (x = kNoLoad: none): x < kb reads K,
    // kb <= x < 2 kb reads V, anything else is out of range in both
    auto stream_chunk = [&](uint32_t x) {
        return chunk_load(rk, x) | chunk_load(rv, x - kb);
    };
    u32x4 lo[ND], e1[ND];
#pragma unroll
    for (int j = 0; j < ND; ++j) {
        const uint32_t A = uint32_t(j) * Sb + t0, m = A & 15, my = A - m + 16 * threadIdx.x;
        lo[j] = stream_chunk(my);
        e1[j] = stream_chunk(lane == 63 && m ? my + 16 : kNoLoad);
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < ND; ++j) {
        const uint32_t A = uint32_t(j) * Sb + t0, m = A & 15, my = A - m + 16 * threadIdx.x;
        const u32x4 hi = from_next_lane_or(lo[j], e1[j]);
        acc ^= m ? funnel16(lo[j], hi, m) : lo[j];
        const uint32_t c = m ? my + 16 : my;   // the chunk that starts in the window
        const u32x4 v = m ? hi : lo[j];
        if (c + 16 <= data_end) {
            st_stream(sh, c, v);
        } else if (c < data_end) {
            const gptr<uint8_t> d = as_global(sh);
            for (uint32_t i = 0; i < data_end - c; ++i) d[c + i] = byte_of(v, int(i));
        }
    }
    *reinterpret_cast<u32x4*>(tile + 16 * threadIdx.x) = acc;
    __syncthreads();
    tile_store<false, kKvTB>(sh + data_end + t0, tile, nbytes);
}

// ----------------------------------------------------------------- gs RDP P/Q
// Words (u16).  P[c] = XOR_r D_r[c]; Qfull[d] = XOR_r D_r[(d - r) mod S].
// Row r starts at byte r*S*2, so its tile is misaligned by mr bytes, and the
// diagonal term of row r is the same row shifted by r words.  Each thread loads
// one aligned 16-byte chunk of each row; the P window (offset mr) and the Q
// window (offset mr - 2r) are byte funnels of that chunk and a neighbour's,
// taken from the adjacent lane by a DPP wave shift (lanes at a wave edge load
// the neighbouring chunk themselves).  Every load is bounded by the tensor,
// whatever the shifts deliver.  Columns whose diagonal wraps (w < nd - 1) and
// the row tail take a per-word path.
//
// The star skip: row r leaves its word at column star_r = (star_base + r) % S
// (C remainder: negative means no skip) out of the diagonal it lies on,
// d = star_r + r (mod S).  That word is the one at position d - w0 of the
// thread's row-r diagonal window, so it is masked there.
// x % S with C semantics (the sign of x), dividing only when x is outside [0, S).
__device__ __forceinline__ int64_t cmod(int64_t x, int64_t S) {
    return (x >= 0 && x < S) ? x : x % S;
}

// v with its bytes 0..n-1 zeroed (n <= 0: v).
__device__ __forceinline__ u32x4 drop_low_bytes(u32x4 v, int n) {
    auto m = [&](int d) {
        const int k = n - 4 * d;   // bytes of dword d to clear
        return k <= 0 ? 0xFFFFFFFFu : (k >= 4 ? 0u : 0xFFFFFFFFu << (8 * k));
    };
    return u32x4{v.x & m(0), v.y & m(1), v.z & m(2), v.w & m(3)};
}

__device__ __forceinline__ u32x4 drop_word(u32x4 v, int64_t k) {
    if (k < 0 || k >= 8) return v;
    const uint32_t m = (k & 1) ? 0x0000FFFFu : 0xFFFF0000u;
    switch (k >> 1) {
        case 0: v.x &= m; break;
        case 1: v.y &= m; break;
        case 2: v.z &= m; break;
        default: v.w &= m; break;
    }
    return v;
}

// Where the data rows' bytes come from.  Without K/V (FUSED false) they are
// the shard rows themselves.  For the fused backup (the pack of
// benchmark/rdp/kernel.cu:32-72, then the parity of :76-107) data-row bytes
// [0, kb) are K_TN, [kb, 2 kb) are V_TN and the rest is the row tensor's own
// padding, which the caller zero-fills and nothing here writes; the kernel
// stores the K/V bytes into the data rows (bytes [0, copy_end)) from the same
// loads.  K and V are equally aligned modulo 16 with their place in the rows,
// so an aligned row chunk is an aligned K or V chunk.
struct GsSource {
    const uint8_t* K;
    const uint8_t* V;
    int64_t kb;         // bytes of K (and of V)
    int64_t copy_end;   // data-row bytes that come from K||V: min(2 kb, nd Sb)
    int64_t rows_end;   // bytes of the whole row tensor, (nd + 2) Sb
};

__device__ __forceinline__ uint8_t gs_src_byte(const GsSource& g, const uint8_t* base, int64_t x) {
    if (x < g.kb) return as_global(g.K)[x];
    if (x < 2 * g.kb) return as_global(g.V)[x - g.kb];
    return x < g.rows_end ? as_global(base)[x] : uint8_t(0);
}

__device__ __forceinline__ uint16_t gs_src_word(const GsSource& g, const uint16_t* sh, int64_t w) {
    const int64_t kw = g.kb / 2;
    if (w < kw) return as_global(reinterpret_cast<const uint16_t*>(g.K))[w];
    if (w < 2 * kw) return as_global(reinterpret_cast<const uint16_t*>(g.V))[w - kw];
    return as_global(sh)[w];
}

// The aligned 16-byte chunk at row offset X assembled byte by byte: only for
// the few chunks next to a K/V/padding boundary.  Bytes before the tensor
// (X < 0) are never used and read as 0.
__device__ __forceinline__ u32x4 gs_src_chunk_bytes(const GsSource& g, const uint8_t* base,
                                                    int64_t X) {
    u32x4 v = {0, 0, 0, 0};
    for (int i = 0; i < 16; ++i)
        if (X + i >= 0) v = set_byte(v, i, gs_src_byte(g, base, X + i));
    return v;
}

// The same 16 bytes for X with base + X 16-byte aligned: one aligned load, or
// two merged where a K/V or V/padding boundary falls inside the chunk; bytes
// before the tensor (X < 0) or past its end read as 0.  K and V are aligned
// like their place in the rows, so each load is the aligned 16-byte chunk
// around a byte of its own tensor and stays in that byte's page.
__device__ __forceinline__ u32x4 gs_src_chunk(const GsSource& g, const uint8_t* base, int64_t X) {
    const int64_t kb = g.kb, first = X < 0 ? 0 : X;
    const int64_t last = X + 15 < g.rows_end - 1 ? X + 15 : g.rows_end - 1;
    if (first > last) return u32x4{0, 0, 0, 0};
    auto src = [&](int64_t x) { return x < kb ? 0 : (x < 2 * kb ? 1 : 2); };
    auto load = [&](int w) {
        return ld16(w == 0 ? g.K + X : (w == 1 ? g.V + (X - kb) : base + X));
    };
    const int ws = src(first), we = src(last);
    u32x4 v;
    if (ws == we) {
        v = load(ws);
    } else if (we == ws + 1) {
        const int n = int((ws == 0 ? kb : 2 * kb) - X);   // bytes from the first source
        const u32x4 a = load(ws);
        v = (a ^ drop_low_bytes(a, n)) | drop_low_bytes(load(we), n);
    } else {
        return gs_src_chunk_bytes(g, base, X);   // both boundaries in one chunk (K under 16 bytes)
    }
    if (X < 0) v = drop_low_bytes(v, int(-X));
    if (X + 16 > g.rows_end) v = v ^ drop_low_bytes(v, int(g.rows_end - X));
    return v;
}

// Store the parts of the chunk at row offset X that lie in [0, lim).
__device__ __forceinline__ void gs_store_chunk(uint8_t* base, int64_t X, u32x4 v, int64_t lim) {
    if (X >= 0 && X + 16 <= lim) {
        st_stream(base, X, v);
        return;
    }
    const gptr<uint8_t> d = as_global(base);
    for (int i = 0; i < 16; ++i)
        if (X + i >= 0 && X + i < lim) d[X + i] = byte_of(v, i);
}

// gs_store_chunk with 32-bit offsets, X >= 0 (row tensors below 2 GiB).
__device__ __forceinline__ void gs_store_chunk32(uint8_t* base, uint32_t X, u32x4 v, uint32_t lim) {
    if (X + 16 <= lim) {
        st_stream(base, X, v);
        return;
    }
    const gptr<uint8_t> d = as_global(base);
    for (int i = 0; i < 16; ++i)
        if (X + i < lim) d[X + i] = byte_of(v, i);
}

// Per data row r < 8: the diagonal its star word lies on, (star_r + r) mod S
// with star_r = (star_base + r) % S, or -1 when the row skips nothing (C
// remainder: a negative star_base gives a negative star_r).  The same for
// every tile, so the host computes it once; the batched path runs only on
// row tensors below 2 GiB, so it fits 32 bits.
struct GsStar {
    int32_t d[8];
};

// P/Q of one tile of a stripe of at least one full tile with ND = nd <= 8
// data rows: each row's chunk, and the edge lanes' neighbour chunks, are all
// requested before the first is used, so a thread has every row in flight at
// once.  In a partial last tile the lanes past the row's end compute words
// that are not stored (their loads read the next row, or zeros past the
// resource); a fused copy from them stores the next row's bytes from the same
// source the owning tile reads them from.
// With nd <= 8 the Q window starts at most 14 bytes before the lane's chunk
// (mr - 2r >= -14), so the previous lane's chunk always covers it.  Without
// K/V the row resource starts at the 16-aligned address at or below the row
// tensor, so every chunk offset is >= 0, the first tile's included.  In the
// first tile only thread 0's Q words wrap: word i < r of row r is row r's word
// S + i - r, and the window read the flat word before the row (row r-1's word
// S + i - r) in its place.  Lanes 1..ND of wave 0 fetch the rows' last 16
// bytes along with their own loads, and thread 0 adds the difference of
// consecutive rows' tails from them.  Returns false, having loaded nothing,
// when the tile needs the general path: a fused tile whose K/V/padding
// boundary falls inside some row's loads, and the fused first tile of a row
// tensor that is not 16-byte aligned (row 0's first chunk would start before K).
template <bool FUSED, int ND>
__device__ __forceinline__ bool gs_pq_batched(uint16_t* sh, uint32_t Sb, uint32_t t0b, int32_t w0,
                                              const GsStar& star, const GsSource& g,
                                              uint32_t rows_bytes, u32x4& p, u32x4& q) {
    const uint8_t* base = reinterpret_cast<const uint8_t*>(sh);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t b15 = uint32_t(reinterpret_cast<uintptr_t>(base)) & 15;
    const uint32_t kb = uint32_t(g.kb), copy_end = uint32_t(g.copy_end);
    if (FUSED && t0b == 0 && b15 != 0) return false;
    // misalignment of row r's tile start, and its lane-0 chunk offset in the
    // rows (-b15 for row 0 of the first tile: the chunk holding byte 0)
    auto row_mr = [&](int r) { return (b15 + uint32_t(r) * Sb + t0b) & 15; };
    auto row_x0 = [&](int r) { return uint32_t(r) * Sb + t0b - row_mr(r); };
    // source of row r's chunks: 0 the rows, 1 K, 2 V, -1 mixed
    // every byte row r's loads cover: the lanes' chunks, lane 0's previous
    // chunk (a window starting before its chunk, not in the first tile) and
    // the last lane's next chunk (a window reaching past its chunk)
    auto row_src = [&](int r) {
        if (!FUSED) return 0;
        const int32_t mr = int32_t(row_mr(r)), sq = mr - 2 * r;
        const int64_t x0 = row_x0(r);
        const int64_t lo = x0 - (sq < 0 && t0b != 0 ? 16 : 0);
        const int64_t hi = x0 + kTileBytes + (mr > 0 || sq > 0 ? 16 : 0);
        if (hi <= int64_t(kb)) return 1;
        if (lo >= int64_t(kb) && hi <= 2 * int64_t(kb)) return 2;
        return lo < 2 * int64_t(kb) ? -1 : 0;
    };
    uint32_t srcs = 0;   // row r's source in bits 2r, 2r+1
    if (FUSED) {
        bool mixed = false;
#pragma unroll
        for (int r = 0; r < ND; ++r) {
            const int sr = row_src(r);
            mixed |= sr < 0;
            srcs |= uint32_t(sr & 3) << (2 * r);
        }
        if (mixed) return false;
    }
    // without K/V the rows from their aligned-down start (offsets + rb)
    const uint32_t rb = FUSED ? 0 : b15;
    const __amdgpu_buffer_rsrc_t rrows = chunk_rsrc(base - rb, rows_bytes + rb);
    // first tile: lane j + 1 of wave 0 fetches the two aligned chunks over the
    // 16 bytes before row j's end (flat offset tx), from the rows or from K or
    // V; a pair across a K/V/padding boundary is read byte by byte.  Without
    // K/V along with the lane's own loads; the fused kernel, which has no
    // scalar registers to spare there, after them.
    const bool tail_lane = ND > 1 && t0b == 0 && threadIdx.x >= 1 && threadIdx.x <= ND;
    const uint32_t tx = threadIdx.x * Sb - 16, tm = (b15 + tx) & 15, ta = tx - tm;
    auto tail_of = [&]() {
        u32x4 t = {0, 0, 0, 0};
        if (tail_lane) {
            const uint8_t* c = base + ta;
            const uint32_t te = ta + (tm ? 32 : 16);
            bool bytes = false;
            if (FUSED && te <= kb) c = g.K + ta;
            else if (FUSED && ta >= kb && te <= 2 * kb) c = g.V + (ta - kb);
            else if (FUSED && ta < 2 * kb) bytes = true;
            if (bytes) {
                t = gs_src_chunk_bytes(g, base, tx);
            } else {
                const u32x4 lo = ld16(c);
                t = tm ? funnel16(lo, ld16(c + 16), tm) : lo;
            }
        }
        return t;
    };
    u32x4 tail = {0, 0, 0, 0};
    if (!FUSED) tail = tail_of();
    u32x4 c0[ND], e1[ND], em[ND];
#pragma unroll
    for (int r = 0; r < ND; ++r) {
        const int src = int(srcs >> (2 * r)) & 3;
        const __amdgpu_buffer_rsrc_t rs =
            src == 1 ? chunk_rsrc(g.K, kb) : (src == 2 ? chunk_rsrc(g.V, kb) : rrows);
        const uint32_t mr = row_mr(r);
        const int s = int(mr) - 2 * r;
        const uint32_t my = row_x0(r) + (src == 2 ? 0u - kb : rb) + 16 * threadIdx.x;
        c0[r] = chunk_load(rs, my);
        e1[r] = chunk_load(rs, lane == 63 && (mr > 0 || s > 0) ? my + 16 : kNoLoad);
        em[r] = chunk_load(rs, lane == 0 && s < 0 && (t0b | threadIdx.x) != 0 ? my - 16 : kNoLoad);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < ND; ++r) {
        const uint32_t mr = row_mr(r);
        const int s = int(mr) - 2 * r;
        // the shifts run with every lane active; the edge lanes keep the
        // chunks they loaded themselves (a per-lane select here was
        // miscompiled: one funnel case read the shifted value from before
        // the select, so lane 0 lost its previous chunk)
        const u32x4 c1 = from_next_lane_or(c0[r], e1[r]), cm = from_prev_lane_or(c0[r], em[r]);
        if (FUSED) {
            // this lane's chunk into the data rows (rows read from the row
            // tensor itself lie past K||V, so their chunks fail the test); the
            // last thread also stores the chunk past the block, which the
            // window's last mr bytes fall in.  A wave's 64 chunks start at
            // position `pre` of a 128-byte line: when pre != 0 its first and
            // last lines are shared with the neighbouring waves, and their
            // chunks go through L2 (the two parts merge there), the others
            // non-temporal.  All non-temporal, the two parts of each such line
            // were written separately: 235 against 219.5 us on the 512 MiB
            // stream (rows misaligned by 86 bytes mod 128).
            const uint32_t X = row_x0(r) + 16 * threadIdx.x;
            const uint32_t pre = uint32_t((reinterpret_cast<uintptr_t>(sh) + row_x0(r)) >> 4) & 7;
            const bool edge = pre != 0 && (lane < 8 - pre || lane >= 64 - pre);
            if (X < copy_end) {
                if (edge && X + 16 <= copy_end) st16(reinterpret_cast<uint8_t*>(sh) + X, c0[r]);
                else gs_store_chunk32(reinterpret_cast<uint8_t*>(sh), X, c0[r], copy_end);
                if (mr > 0 && threadIdx.x == kTB - 1)
                    gs_store_chunk32(reinterpret_cast<uint8_t*>(sh), X + 16, c1, copy_end);
            }
        }
        p ^= mr ? funnel16(c0[r], c1, mr) : c0[r];
        u32x4 qw;
        if (s > 0) qw = funnel16(c0[r], c1, uint32_t(s));
        else if (s == 0) qw = c0[r];
        else qw = funnel16(cm, c0[r], uint32_t(s + 16));
        q ^= star.d[r] < 0 ? qw : drop_word(qw, int64_t(star.d[r]) - w0);
    }
    if constexpr (ND > 1) {
        if (t0b == 0 && threadIdx.x < 64) {
            const u32x4 t = FUSED ? tail_of() : tail;
            // Words 0..r-1 of row r's window are the 2r bytes before the row:
            // its first chunk's first mr bytes (flat bytes of row r-1's end)
            // after zeros (lane 0 loads no previous chunk here).  In their
            // place go row r's last r words.
            u32x4 fix = {0, 0, 0, 0}, prev = lane_value(t, 1);
#pragma unroll
            for (int r = 1; r < ND; ++r) {
                const u32x4 cur = lane_value(t, r + 1);
                const int mr = int(row_mr(r)), z = 2 * r - mr;   // leading zero bytes
                const u32x4 was = drop_low_bytes(funnel16(prev, u32x4{0, 0, 0, 0}, 16 - 2 * r), z);
                const u32x4 f = was ^ funnel16(cur, u32x4{0, 0, 0, 0}, 16 - 2 * r);
                fix ^= star.d[r] < 0 ? f : drop_word(f, int64_t(star.d[r]) - w0);
                prev = cur;
            }
            if (threadIdx.x == 0) q ^= fix;
        }
    }
    return true;
}

template <bool FUSED, int ND>
__global__ __launch_bounds__(kTB) void gs_rdp_parity_kernel(uint16_t* sh, int nd, int64_t S,
                                                            int star_base, GsSource g,
                                                            uint64_t rows_bytes, GsStar star) {
    __shared__ __attribute__((aligned(16))) uint8_t tp[kTileBytes + 16];
    __shared__ __attribute__((aligned(16))) uint8_t tq[kTileBytes + 16];
    const uint8_t* base = reinterpret_cast<const uint8_t*>(sh);
    const uint8_t* end = base + uint64_t(nd + 2) * uint64_t(S) * 2;
    const uint64_t Sb = uint64_t(S) * 2;
    const int64_t w0 = int64_t(blockIdx.x) * (kTileBytes / 2) + 8 * threadIdx.x;
    const uint64_t t0b = uint64_t(blockIdx.x) * kTileBytes;
    const uint32_t nbytes = uint32_t(Sb - t0b < uint64_t(kTileBytes) ? Sb - t0b : kTileBytes);
    const uint32_t lane = threadIdx.x & 63;
    // Lanes with a whole or partial window in the row whose diagonal does not
    // wrap; the partial lane's words past the row end are never stored.
    const bool fast = w0 < S && w0 >= nd - 1;
    u32x4 p = {0, 0, 0, 0}, q = {0, 0, 0, 0};
    // Stripes of at least one full tile: every row requested at once.  The
    // general loop below handles shorter stripes, nd > 8, rows tensors of
    // 2 GiB or more and fused tiles next to a K/V boundary.
    bool batched = false;
    if constexpr (ND > 0) {
        if (rows_bytes && S >= kTileBytes / 2)
            batched = gs_pq_batched<FUSED, ND>(sh, uint32_t(Sb), uint32_t(t0b), int32_t(w0), star, g,
                                               uint32_t(rows_bytes), p, q);
    }
    for (int r = 0; r < (batched ? 0 : nd); ++r) {
        const uint8_t* A0 = base + uint64_t(r) * Sb + t0b;
        const uint32_t mr = uint32_t(reinterpret_cast<uintptr_t>(A0) & 15);
        const int s = int(mr) - 2 * r;   // Q window offset from my, in [-2(nd-1), 15]
        // lane 0's aligned chunk: at row offset X0, read from rp (uniform)
        const int64_t X0 = int64_t(uint64_t(r) * Sb + t0b) - int64_t(mr);
        const uint8_t* rp = A0 - mr;
        bool mixed = false, from_kv = false;
        if (FUSED) {
            // every chunk any lane loads for this row: its own, the edge lanes'
            // neighbours, and the Q window's chunks when it starts more than
            // one chunk back (s < -16)
            const int64_t lo = X0 - 48 - 2 * int64_t(nd), hi = X0 + kTileBytes + 32;
            if (hi <= g.kb) {
                rp = g.K + X0;
                from_kv = true;
            } else if (lo >= g.kb && hi <= 2 * g.kb) {
                rp = g.V + (X0 - g.kb);
                from_kv = true;
            } else if (lo < 2 * g.kb) {
                mixed = true;
            }
        }
        const uint8_t* my = rp + 16 * threadIdx.x;
        const int64_t X = X0 + 16 * int64_t(threadIdx.x);
        // K/V chunks lie inside K/V by the classification above; row chunks
        // past the tensor's end (lanes past the last word) read as zero
        u32x4 c0;
        if (FUSED && mixed) c0 = gs_src_chunk(g, base, X);
        else c0 = (from_kv || my < end) ? ld16(my) : u32x4{0, 0, 0, 0};
        // the shifts run with every lane active (a lane reading a disabled lane
        // gets nothing); lanes at a wave edge then load their neighbour chunk
        u32x4 c1 = from_next_lane(c0), cm = from_prev_lane(c0);
        if (lane == 63 && fast && (mr > 0 || s > 0))
            c1 = (FUSED && mixed) ? gs_src_chunk(g, base, X + 16)
                                  : ((from_kv || my + 16 < end) ? ld16(my + 16) : u32x4{0, 0, 0, 0});
        if (lane == 0 && fast && s < 0)
            cm = (FUSED && mixed) ? gs_src_chunk(g, base, X - 16) : ld16(my - 16);
        if (fast) {
            if (FUSED && (from_kv || mixed)) {
                // This lane's chunk into the data rows.  The window's last mr
                // bytes are in the next chunk: the next lane stores it, unless
                // that lane is past the block or past the row's last word (the
                // row's last lanes store the next chunk themselves; bytes past
                // the row are the next row's, stored with the same values).
                gs_store_chunk(reinterpret_cast<uint8_t*>(sh), X, c0, g.copy_end);
                if (mr > 0 && (threadIdx.x == kTB - 1 || w0 + 16 > S))
                    gs_store_chunk(reinterpret_cast<uint8_t*>(sh), X + 16, c1, g.copy_end);
            }
            p ^= mr ? funnel16(c0, c1, mr) : c0;
            u32x4 qw;
            if (s > 0) {
                qw = funnel16(c0, c1, uint32_t(s));
            } else if (s == 0) {
                qw = c0;
            } else if (s >= -16) {
                qw = funnel16(cm, c0, uint32_t(s + 16));
            } else {
                // rows r >= 9 of wide stripes: the window starts k chunks
                // back (k = floor(s / 16) <= -2), past the neighbour lane
                const int k = (s - 15) / 16;
                const int64_t Xq = X + 16 * k;
                const u32x4 a = (FUSED && mixed) ? gs_src_chunk(g, base, Xq) : ld16(my + 16 * k);
                const u32x4 b = (FUSED && mixed) ? gs_src_chunk(g, base, Xq + 16)
                                                 : ld16(my + 16 * k + 16);
                qw = funnel16(a, b, uint32_t(s - 16 * k));
            }
            const int64_t star = cmod(int64_t(star_base) + r, S);
            q ^= star < 0 ? qw : drop_word(qw, cmod(star + r, S) - w0);
        }
    }
    if (!batched && !fast && w0 < S) {
        const int n = int(S - w0 < 8 ? S - w0 : 8);
        for (int i = 0; i < n; ++i) {
            uint16_t a = 0, b = 0;
            for (int r = 0; r < nd; ++r) {
                const int64_t x = int64_t(r) * S + w0 + i;
                const uint16_t v = FUSED ? gs_src_word(g, sh, x) : sh[x];
                if (FUSED && 2 * x < g.copy_end) as_global(sh)[x] = v;
                a ^= v;
                int64_t c = (w0 + i - r) % S;
                if (c < 0) c += S;
                if (c != cmod(int64_t(star_base) + r, S))
                    b ^= FUSED ? gs_src_word(g, sh, int64_t(r) * S + c) : sh[uint64_t(r) * S + c];
            }
            p = set_byte(set_byte(p, 2 * i, uint8_t(a)), 2 * i + 1, uint8_t(a >> 8));
            q = set_byte(set_byte(q, 2 * i, uint8_t(b)), 2 * i + 1, uint8_t(b >> 8));
        }
    }
    *reinterpret_cast<u32x4*>(tp + 16 * threadIdx.x) = p;
    *reinterpret_cast<u32x4*>(tq + 16 * threadIdx.x) = q;
    __syncthreads();
    uint8_t* out = reinterpret_cast<uint8_t*>(sh);
    tile_store<true>(out + uint64_t(nd) * Sb + t0b, tp, nbytes);
    tile_store<true>(out + uint64_t(nd + 1) * Sb + t0b, tq, nbytes);
}

// ------------------------------------------------------------- gs recovery
// fused_recovery_full_kv in one pass: row t (t >= 0) rebuilt as P ^ the other
// data rows and written back into the shards, and every data row's tile (row
// t's the rebuilt one) written to out, the flat copy-out of the data rows
// clipped to out_len bytes (load_full_kernel, benchmark/rdp/kernel.cu:305-345).
// A block owns one column tile of every row.  Each data row's window is staged
// in an LDS tile and written with tile_store, so every output byte has exactly
// one writer whatever the alignment of out.  Full tiles of stripes with
// nd = ND <= 8 in shards below 2 GiB, and their partial last tile when a row
// holds at least one full tile, request every surviving row's chunk at once
// (the loads of xor_rows_batched, one LDS tile per row); otherwise the rows
// go one at a time through one LDS tile.  Row t itself is never read.
// Stores, as measured on the 512 MiB stream: the copy-out non-temporal (232
// -> 209 us), the rebuilt row plain (non-temporal: 226 us).
template <int ND>
__global__ __launch_bounds__(kTB) void gs_recover_kernel(uint8_t* sh, uint64_t Sb, uint32_t in_bytes,
                                                         int nd, int t, uint8_t* out,
                                                         uint64_t out_len) {
    constexpr int NT = ND > 0 ? ND : 1;
    __shared__ __attribute__((aligned(16))) uint8_t tiles[NT][kTileBytes + 16];
    const uint64_t t0 = uint64_t(blockIdx.x) * kTileBytes;
    const uint32_t nbytes = uint32_t(Sb - t0 < uint64_t(kTileBytes) ? Sb - t0 : kTileBytes);
    const uint64_t c0 = t0 + 16 * threadIdx.x;
    // data row r's tile into out, up to out_len
    auto store_row = [&](int r, const uint8_t* tile) {
        const uint64_t o = uint64_t(r) * Sb + t0;
        if (o < out_len) tile_store<true>(out + o, tile, uint32_t(out_len - o < nbytes ? out_len - o : nbytes));
    };
    if constexpr (ND > 0) {
        // every tile of rows of at least one full tile: in a partial last tile
        // the lanes past the row's end stage bytes that are not stored
        if (Sb >= uint64_t(kTileBytes) && in_bytes) {
            const uint32_t b15 = uint32_t(reinterpret_cast<uintptr_t>(sh)) & 15;
            const __amdgpu_buffer_rsrc_t rs = chunk_rsrc(sh - b15, (b15 + in_bytes + 15) & ~15u);
            const uint32_t lane = threadIdx.x & 63;
            // batch row i: data row i, or i + 1 from row t on (then P last)
            auto row_of = [&](int i) { return i + (t >= 0 && i >= t ? 1 : 0); };
            auto row_a = [&](int i) { return b15 + uint32_t(row_of(i)) * uint32_t(Sb) + uint32_t(t0); };
            u32x4 lo[ND], e1[ND];
#pragma unroll
            for (int i = 0; i < ND; ++i) {
                const uint32_t A = row_a(i), m = A & 15, my = A - m + 16 * threadIdx.x;
                lo[i] = chunk_load(rs, my);
                e1[i] = chunk_load(rs, lane == 63 && m ? my + 16 : kNoLoad);
            }
            __builtin_amdgcn_sched_barrier(0);
            u32x4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < ND; ++i) {
                const uint32_t m = row_a(i) & 15;
                const u32x4 w = m ? funnel16(lo[i], from_next_lane_or(lo[i], e1[i]), m) : lo[i];
                acc ^= w;
                const int j = row_of(i);
                if (j < ND) *reinterpret_cast<u32x4*>(tiles[j] + 16 * threadIdx.x) = w;
            }
            if (t >= 0) *reinterpret_cast<u32x4*>(tiles[t] + 16 * threadIdx.x) = acc;
            __syncthreads();
#pragma unroll
            for (int r = 0; r < ND; ++r) store_row(r, tiles[r]);
            if (t >= 0) tile_store(sh + uint64_t(t) * Sb + t0, tiles[t], nbytes);
            return;
        }
    }
    uint8_t* tl = tiles[0];
    u32x4 acc = {0, 0, 0, 0};
    for (int r = 0; r <= nd; ++r) {   // the data rows, then P
        if (r == t || (r == nd && t < 0)) continue;
        const uint8_t* row = sh + uint64_t(r) * Sb;
        u32x4 w = {0, 0, 0, 0};
        if (c0 + 16 <= Sb) {
            w = load_window16(row + c0);
        } else if (c0 < Sb) {
            for (uint32_t i = 0; i < uint32_t(Sb - c0); ++i) w = set_byte(w, i, row[c0 + i]);
        }
        acc ^= w;
        if (r < nd) {
            *reinterpret_cast<u32x4*>(tl + 16 * threadIdx.x) = w;
            __syncthreads();
            store_row(r, tl);
            __syncthreads();
        }
    }
    if (t >= 0) {
        *reinterpret_cast<u32x4*>(tl + 16 * threadIdx.x) = acc;
        __syncthreads();
        store_row(t, tl);
        tile_store(sh + uint64_t(t) * Sb + t0, tl, nbytes);
    }
}

// ----------------------------------------------------------------- host side
// The batched tile paths take 1..8 rows (ND = the row count; 0: general path
// only) in tensors below 2 GiB, whose out-of-range buffer loads then start
// at 2^31.
typedef void (*XorRowsFn)(const uint8_t*, uint64_t, uint32_t, RowSet, uint8_t*, uint8_t*, FlatCopy);
typedef void (*XorRecFn)(const uint8_t*, uint8_t*, uint8_t*, uint64_t, uint32_t, int, const int32_t*);

template <int ND = 1>
XorRowsFn xor_rows_fn(int rows) {
    if constexpr (ND > 8) {
        return &xor_rows_kernel<0>;
    } else {
        if (rows == ND) return &xor_rows_kernel<ND>;
        return xor_rows_fn<ND + 1>(rows);
    }
}

template <int ND = 1>
XorRecFn xor_rec_fn(int rows) {
    if constexpr (ND > 8) {
        return &xor_reconstruct_kernel<0>;
    } else {
        if (rows == ND) return &xor_reconstruct_kernel<ND>;
        return xor_rec_fn<ND + 1>(rows);
    }
}

inline uint32_t small_bytes(uint64_t n) { return n < (uint64_t(1) << 31) ? uint32_t(n) : 0; }

typedef void (*XorEncKvFn)(const uint8_t*, const uint8_t*, uint32_t, uint8_t*, uint32_t);

template <int ND = 1>
XorEncKvFn xor_encode_kv_fn(int nd) {
    if constexpr (ND > 8) {
        return nullptr;
    } else {
        if (nd == ND) return &xor_encode_kv_kernel<ND>;
        return xor_encode_kv_fn<ND + 1>(nd);
    }
}

typedef void (*GsRecoverFn)(uint8_t*, uint64_t, uint32_t, int, int, uint8_t*, uint64_t);

template <int ND = 1>
GsRecoverFn gs_recover_fn(int nd) {
    if constexpr (ND > 8) {
        return &gs_recover_kernel<0>;
    } else {
        if (nd == ND) return &gs_recover_kernel<ND>;
        return gs_recover_fn<ND + 1>(nd);
    }
}

static int xor_rows(const uint8_t* in, uint64_t Sb, RowSet rs, uint8_t* out0, uint8_t* out1,
                    hipStream_t st, const char* what, FlatCopy fc = FlatCopy{nullptr, nullptr, 0}) {
    if (Sb == 0) return KVEC_OK;
    // rows of `in` the tile reads: lo..hi-1 and extra
    const int top = rs.extra >= rs.hi ? rs.extra + 1 : rs.hi;
    hipLaunchKernelGGL(xor_rows_fn(rs.hi - rs.lo), dim3(blocks_for(int64_t(Sb), kTileBytes)), dim3(kTB),
                       0, st, in, Sb, small_bytes(uint64_t(top) * Sb), rs, out0, out1, fc);
    return check_launch(what);
}

typedef void (*GsParityFn)(uint16_t*, int, int64_t, int, GsSource, uint64_t, GsStar);

template <bool FUSED, int ND = 1>
GsParityFn gs_parity_fn(int nd) {
    if constexpr (ND > 8) {
        return &gs_rdp_parity_kernel<FUSED, 0>;
    } else {
        if (nd == ND) return &gs_rdp_parity_kernel<FUSED, ND>;
        return gs_parity_fn<FUSED, ND + 1>(nd);
    }
}

static int gs_rdp_parity(uint16_t* sh, int nd, int64_t S, int star_base, hipStream_t st,
                         const char* what, const GsSource* fused = nullptr) {
    if (nd <= 0 || S <= 0) return KVEC_OK;  // the reference kernel returns at once
    const dim3 grid(blocks_for(S * 2, kTileBytes));
    // The batched path addresses the rows (and K, V) through buffer resources
    // of up to 15 bytes more than the tensor, whose out-of-range loads must
    // start at 2^31: 0 switches it off.
    const uint64_t rows_bytes = uint64_t(nd + 2) * uint64_t(S) * 2;
    const uint64_t lim = (uint64_t(1) << 31) - 16;
    const bool small = rows_bytes <= lim && (!fused || uint64_t(fused->kb) <= lim);
    const uint64_t rb = small ? rows_bytes : 0;
    GsStar star{};
    for (int r = 0; r < 8; ++r) {
        const int64_t sr = (int64_t(star_base) + r) % S;
        star.d[r] = sr < 0 ? -1 : int32_t((sr + r) % S);
    }
    if (fused)
        hipLaunchKernelGGL(gs_parity_fn<true>(nd), grid, dim3(kTB), 0, st, sh, nd, S, star_base, *fused, rb,
                           star);
    else
        hipLaunchKernelGGL(gs_parity_fn<false>(nd), grid, dim3(kTB), 0, st, sh, nd, S, star_base,
                           GsSource{nullptr, nullptr, 0, 0, 0}, rb, star);
    return check_launch(what);
}

}  // namespace kvec

using namespace kvec;

// =========================== XOR (benchmark/xor/kernel.cu) ===================

// encode_xor_launcher, benchmark/xor/kernel.cu:158-171
extern "C" int kvec_xor_encode(const void* data_padded, void* shards, int data_shards,
                               int64_t shard_size, void* stream) {
    if (!data_padded || !shards) return set_error(KVEC_EINVAL, "kvec_xor_encode: null pointer");
    if (data_shards < 1 || shard_size < 0)
        return set_error(KVEC_EINVAL, "kvec_xor_encode: data_shards=%d shard_size=%lld", data_shards,
                         (long long)shard_size);
    hipStream_t st = as_stream(stream);
    const uint64_t Sb = uint64_t(shard_size);
    if (ranges_overlap(data_padded, Sb * data_shards, (uint8_t*)shards + Sb * data_shards, Sb))
        return set_error(KVEC_EINVAL, "kvec_xor_encode: data overlaps the parity row");
    // The data rows are copied by the parity kernel's own loads when the two
    // buffers are disjoint and equally aligned modulo 16 bytes; else (same
    // buffer: no copy; partial overlap: refused) by a copy first.
    if (Sb && fused_copy_ok(data_padded, shards, Sb * data_shards))
        return xor_rows((const uint8_t*)data_padded, Sb, RowSet{0, data_shards, -1, -1},
                        (uint8_t*)shards + Sb * data_shards, nullptr, st, "kvec_xor_encode",
                        FlatCopy{(const uint8_t*)data_padded, (uint8_t*)shards, Sb * data_shards});
    int rc = copy_d2d(shards, data_padded, Sb * data_shards, st, "kvec_xor_encode");
    if (rc) return rc;
    return xor_rows((const uint8_t*)data_padded, Sb, RowSet{0, data_shards, -1, -1},
                    (uint8_t*)shards + Sb * data_shards, nullptr, st, "kvec_xor_encode");
}

// forward_encode_kv, benchmark/xor/main.py:69-90 (pack_kv of K then V into the
// stream, zero padding) followed by encode_xor, benchmark/xor/kernel.cu:158-171.
extern "C" int kvec_xor_encode_kv(const void* key_input, const void* value_input,
                                  int64_t kv_half_bytes, void* shards, int data_shards,
                                  int64_t shard_size, void* stream) {
    if (data_shards < 1 || shard_size < 0 || kv_half_bytes < 0)
        return set_error(KVEC_EINVAL, "kvec_xor_encode_kv: data_shards=%d shard_size=%lld kv_bytes=%lld",
                         data_shards, (long long)shard_size, (long long)kv_half_bytes);
    const uint64_t Sb = uint64_t(shard_size), kb = uint64_t(kv_half_bytes);
    const uint64_t data_bytes = Sb * uint64_t(data_shards);
    if (2 * kb > data_bytes)
        return set_error(KVEC_EINVAL, "kvec_xor_encode_kv: K and V (%llu bytes) exceed %d rows of %lld",
                         (unsigned long long)(2 * kb), data_shards, (long long)shard_size);
    if (!shards || (kb && (!key_input || !value_input)))
        return set_error(KVEC_EINVAL, "kvec_xor_encode_kv: null pointer");
    if (Sb == 0) return KVEC_OK;
    hipStream_t st = as_stream(stream);
    uint8_t* sh = (uint8_t*)shards;
    const uintptr_t R0 = uintptr_t(sh), R1 = R0 + data_bytes + Sb;
    const uintptr_t Kp = uintptr_t(key_input), Vp = uintptr_t(value_input);
    const bool apart = (Kp + kb <= R0 || Kp >= R1) && (Vp + kb <= R0 || Vp >= R1);
    const bool aligned = ((R0 | Kp | Vp | kb) & 15) == 0;
    XorEncKvFn fn = xor_encode_kv_fn(data_shards);
    if (fn && apart && aligned && Sb >= uint64_t(kKvTile) && kb < (uint64_t(1) << 30) &&
        data_bytes + Sb < (uint64_t(1) << 31)) {
        hipLaunchKernelGGL(fn, dim3(blocks_for(int64_t(Sb), kKvTile)), dim3(kKvTB), 0, st,
                           (const uint8_t*)key_input, (const uint8_t*)value_input, uint32_t(kb), sh,
                           uint32_t(Sb));
        return check_launch("kvec_xor_encode_kv");
    }
    // otherwise the pack, the zero padding, then encode_xor on the rows in place
    int rc = copy_d2d(sh, key_input, kb, st, "kvec_xor_encode_kv");
    if (!rc) rc = copy_d2d(sh + kb, value_input, kb, st, "kvec_xor_encode_kv");
    if (rc) return rc;
    if (data_bytes > 2 * kb) {
        rc = zero_d(sh + 2 * kb, data_bytes - 2 * kb, st, "kvec_xor_encode_kv");
        if (rc) return rc;
    }
    return xor_rows(sh, Sb, RowSet{0, data_shards, -1, -1}, sh + data_bytes, nullptr, st,
                    "kvec_xor_encode_kv");
}

// reconstruct_xor_launcher, benchmark/xor/kernel.cu:173-191
extern "C" int kvec_xor_reconstruct(const void* encoded_data, void* recovered_data,
                                    void* recovered_missing, int64_t shard_size, int data_shards,
                                    const int32_t* missing_indices, int missing_count,
                                    void* stream) {
    if (missing_count != 1) return KVEC_OK;  // the reference kernel is a no-op
    if (!encoded_data || !recovered_data || !recovered_missing || !missing_indices)
        return set_error(KVEC_EINVAL, "kvec_xor_reconstruct: null pointer");
    if (data_shards < 1 || shard_size < 0)
        return set_error(KVEC_EINVAL, "kvec_xor_reconstruct: data_shards=%d shard_size=%lld",
                         data_shards, (long long)shard_size);
    if (shard_size == 0) return KVEC_OK;
    const uint64_t Sb = uint64_t(shard_size);
    hipLaunchKernelGGL(xor_rec_fn(data_shards), dim3(blocks_for(int64_t(Sb), kTileBytes)), dim3(kTB), 0,
                       as_stream(stream), (const uint8_t*)encoded_data, (uint8_t*)recovered_data,
                       (uint8_t*)recovered_missing, Sb, small_bytes(uint64_t(data_shards + 1) * Sb),
                       data_shards, missing_indices);
    return check_launch("kvec_xor_reconstruct");
}

// backwards_decode_kv, benchmark/xor/main.py:159-194: the missing shard rebuilt
// in place (reconstruct_xor) and the first out_bytes of the data rows copied
// out (unpack_kv).  A lost data row: one pass of gs_recover_kernel over the
// byte rows (P is row data_shards).  A lost P: P recomputed, then the copy-out
// pass.  missing < 0: the copy-out pass alone.  With out inside the shard
// tensor, the reconstruct and then a copy (out == shards: no copy; an output
// that overlaps the bytes it copies is refused).
extern "C" int kvec_xor_recover_kv(void* shards, void* out, int data_shards, int64_t shard_size,
                                   int64_t out_bytes, int missing, void* stream) {
    if (!shards || (out_bytes > 0 && !out))
        return set_error(KVEC_EINVAL, "kvec_xor_recover_kv: null pointer");
    if (data_shards < 1 || shard_size < 0 || out_bytes < 0 || missing > data_shards)
        return set_error(KVEC_EINVAL, "kvec_xor_recover_kv: data_shards=%d shard_size=%lld missing=%d",
                         data_shards, (long long)shard_size, missing);
    const uint64_t Sb = uint64_t(shard_size), nbytes = uint64_t(out_bytes);
    if (nbytes > Sb * uint64_t(data_shards))
        return set_error(KVEC_EINVAL, "kvec_xor_recover_kv: %llu output bytes exceed the data rows",
                         (unsigned long long)nbytes);
    if (Sb == 0) return KVEC_OK;
    hipStream_t st = as_stream(stream);
    uint8_t* sh = (uint8_t*)shards;
    const int nd = data_shards;
    const uintptr_t R0 = uintptr_t(sh), R1 = R0 + uint64_t(nd + 1) * Sb;
    const uintptr_t O0 = uintptr_t(out), O1 = O0 + nbytes;
    // An output inside the shard tensor gets the rebuild and then the copy-out;
    // the copy's own source and destination must then be the same bytes or
    // disjoint.
    if (out != shards && ranges_overlap(out, nbytes, sh, nbytes))
        return set_error(KVEC_EINVAL, "kvec_xor_recover_kv: output overlaps the data rows it copies");
    if (missing == nd) {   // P recomputed from the data rows
        int rc = xor_rows(sh, Sb, RowSet{0, nd, -1, -1}, sh + uint64_t(nd) * Sb, nullptr, st,
                          "kvec_xor_recover_kv");
        if (rc) return rc;
    }
    if (nbytes == 0 && missing < 0) return KVEC_OK;
    const int t = missing >= 0 && missing < nd ? missing : -1;
    if (nbytes == 0 || O1 <= R0 || O0 >= R1) {
        if (t < 0 && nbytes == 0) return KVEC_OK;
        hipLaunchKernelGGL(gs_recover_fn(nd), dim3(blocks_for(int64_t(Sb), kTileBytes)), dim3(kTB), 0, st,
                           sh, Sb, small_bytes(uint64_t(nd + 1) * Sb), nd, t, (uint8_t*)out, nbytes);
        return check_launch("kvec_xor_recover_kv");
    }
    if (t >= 0) {
        int rc = xor_rows(sh, Sb, RowSet{0, nd, t, nd}, sh + uint64_t(t) * Sb, nullptr, st,
                          "kvec_xor_recover_kv");
        if (rc) return rc;
    }
    return copy_d2d(out, sh, nbytes, st, "kvec_xor_recover_kv");
}

// pack_kv_launcher, benchmark/xor/kernel.cu:193-207: K bytes then V bytes
// (the little-endian byte split of a 16-bit word is the identity in memory).
extern "C" int kvec_pack_kv(const void* key_input, const void* value_input, void* kv_bytes, int n,
                            int seq_len, void* stream) {
    if (n < 0 || seq_len < 0) return set_error(KVEC_EINVAL, "kvec_pack_kv: n=%d seq_len=%d", n, seq_len);
    const uint64_t bytes = uint64_t(n) * uint64_t(seq_len) * 2;
    if (bytes && (!key_input || !value_input || !kv_bytes))
        return set_error(KVEC_EINVAL, "kvec_pack_kv: null pointer");
    hipStream_t st = as_stream(stream);
    int rc = copy_d2d(kv_bytes, key_input, bytes, st, "kvec_pack_kv");
    if (rc) return rc;
    return copy_d2d((uint8_t*)kv_bytes + bytes, value_input, bytes, st, "kvec_pack_kv");
}

// unpack_kv_launcher, benchmark/xor/kernel.cu:209-223 (stream-ordered; the
// reference also blocks the host until the device is idle).
extern "C" int kvec_unpack_kv(const void* kv_bytes, void* dequant_kv, int n, int seq_len,
                              void* stream) {
    if (n < 0 || seq_len < 0) return set_error(KVEC_EINVAL, "kvec_unpack_kv: n=%d seq_len=%d", n, seq_len);
    const uint64_t bytes = uint64_t(n) * uint64_t(seq_len) * 4;
    if (bytes && (!kv_bytes || !dequant_kv)) return set_error(KVEC_EINVAL, "kvec_unpack_kv: null pointer");
    return copy_d2d(dequant_kv, kv_bytes, bytes, as_stream(stream), "kvec_unpack_kv");
}

// ====================== gs RDP (benchmark/rdp/kernel.cu) =====================

// fused_backup_full_kv_launcher, benchmark/rdp/kernel.cu:366-395: pack the
// token-major K|V words into the data rows (pack_scatter_kernel_full, :32-72,
// drops words past row nd-1), then P and Q (compute_rdp_parity_kernel, :76-107).
extern "C" int kvec_gs_rdp_backup(const void* K_TN, const void* V_TN, void* shards, int nd, int S,
                                  int T, int n, int star_base, void* stream) {
    if (!shards) return set_error(KVEC_EINVAL, "kvec_gs_rdp_backup: null shards");
    hipStream_t st = as_stream(stream);
    if (T > 0 && n > 0 && nd > 0 && S > 0) {
        if (!K_TN || !V_TN) return set_error(KVEC_EINVAL, "kvec_gs_rdp_backup: null K/V");
        const uint64_t tn = uint64_t(T) * uint64_t(n), cap = uint64_t(nd) * uint64_t(S);
        // The pack rides on the parity kernel when K and V are equally aligned
        // modulo 16 with their place in the rows and overlap nothing there.
        const uintptr_t R0 = uintptr_t(shards), Rend = R0 + (cap + 2 * uint64_t(S)) * 2;
        const uintptr_t Kp = uintptr_t(K_TN), Vp = uintptr_t(V_TN);
        const bool apart = (Kp + tn * 2 <= R0 || Kp >= Rend) && (Vp + tn * 2 <= R0 || Vp >= Rend);
        if (apart && ((Kp ^ R0) & 15) == 0 && ((Vp ^ (R0 + tn * 2)) & 15) == 0) {
            const uint64_t kv = 4 * tn, rows = 2 * cap;
            const GsSource g{(const uint8_t*)K_TN, (const uint8_t*)V_TN, int64_t(2 * tn),
                             int64_t(kv < rows ? kv : rows), int64_t(Rend - R0)};
            return gs_rdp_parity((uint16_t*)shards, nd, S, star_base, st, "kvec_gs_rdp_backup", &g);
        }
        const uint64_t nk = tn < cap ? tn : cap;
        const uint64_t nv = 2 * tn < cap ? tn : (cap > tn ? cap - tn : 0);
        int rc = copy_d2d(shards, K_TN, nk * 2, st, "kvec_gs_rdp_backup");
        if (!rc) rc = copy_d2d((uint16_t*)shards + tn, V_TN, nv * 2, st, "kvec_gs_rdp_backup");
        if (rc) return rc;
    }
    return gs_rdp_parity((uint16_t*)shards, nd, S, star_base, st, "kvec_gs_rdp_backup");
}

// fused_recovery_full_kv_launcher, benchmark/rdp/kernel.cu:397-521.  Indices
// outside [0, nd) are dropped (:402-404).  Two distinct data rows a < b: the
// launcher's last two kernels rebuild row a from P (:473-480), overwriting
// every word the ring-walk kernels (:411-470) wrote, and then row b from P
// (:482-490); that second rebuild returns row b's input bytes exactly
// (P ^ a' ^ rest = b), so only row a is rewritten here.  One row: rebuilt
// from P (:492-507).  Then the data rows are copied out (load_full_kernel,
// :305-345), words past row nd-1 reading 0.
extern "C" int kvec_gs_rdp_recover(void* shards, void* out_TN, int nd, int S, int T, int n,
                                   int star_base, int missing_a, int missing_b, void* stream) {
    if (!shards) return set_error(KVEC_EINVAL, "kvec_gs_rdp_recover: null shards");
    hipStream_t st = as_stream(stream);
    int a = (missing_a >= 0 && missing_a < nd) ? missing_a : -1;
    int b = (missing_b >= 0 && missing_b < nd) ? missing_b : -1;
    // Two rows lost: the reference's fill_a_star_from_P (benchmark/rdp/kernel.cu:268-282,
    // launched at :466) reads P and the other rows at column (star_base + a) % S and writes
    // row a there, a the lower row.  A negative remainder (C's %) addresses the row before
    // each one, and before the tensor for row 0: undefined, so refused.  Otherwise that
    // write lands in row a, which rebuild_row_from_P rewrites, and star_base changes no
    // output byte.
    if (a >= 0 && b >= 0 && a != b && S > 0 && (int64_t(star_base) + (a < b ? a : b)) % S < 0)
        return set_error(KVEC_EINVAL,
                         "kvec_gs_rdp_recover: (star_base + a) %% S < 0 for lost rows %d and %d (star_base=%d): "
                         "the reference addresses outside row a", a < b ? a : b, a < b ? b : a, star_base);
    int t = -1;
    if (a >= 0 && b >= 0 && a != b)
        t = a < b ? a : b;
    else if (a >= 0 && b < 0)
        t = a;
    else if (b >= 0 && a < 0)
        t = b;
    const bool copy_out = T > 0 && n > 0 && nd > 0 && S > 0;
    if (copy_out && !out_TN) return set_error(KVEC_EINVAL, "kvec_gs_rdp_recover: null output");
    const uint64_t total = 2 * uint64_t(T > 0 ? T : 0) * uint64_t(n > 0 ? n : 0);
    const uint64_t cap = uint64_t(nd > 0 ? nd : 0) * uint64_t(S > 0 ? S : 0);
    const uint64_t nc = total < cap ? total : cap;
    // An output inside the shard tensor gets the rebuild and then the copy-out;
    // the copy's own source and destination must then be the same bytes or
    // disjoint.
    if (copy_out && out_TN != shards && ranges_overlap(out_TN, nc * 2, shards, nc * 2))
        return set_error(KVEC_EINVAL, "kvec_gs_rdp_recover: output overlaps the data rows it copies");
    if (copy_out) {
        // One pass (rebuild and copy-out) when out overlaps no shard row.
        const uint64_t Sb = uint64_t(S) * 2;
        const uintptr_t R0 = uintptr_t(shards), R1 = R0 + uint64_t(nd + 2) * Sb;
        const uintptr_t O0 = uintptr_t(out_TN), O1 = O0 + total * 2;
        if (O1 <= R0 || O0 >= R1) {
            hipLaunchKernelGGL(gs_recover_fn(nd), dim3(blocks_for(int64_t(Sb), kTileBytes)), dim3(kTB), 0, st,
                               (uint8_t*)shards, Sb, small_bytes(uint64_t(nd + 1) * Sb), nd, t,
                               (uint8_t*)out_TN, nc * 2);
            int rc = check_launch("kvec_gs_rdp_recover");
            if (rc) return rc;
            return zero_d((uint16_t*)out_TN + nc, (total - nc) * 2, st, "kvec_gs_rdp_recover");
        }
    }
    if (t >= 0 && S > 0) {
        const uint64_t Sb = uint64_t(S) * 2;
        uint8_t* base = (uint8_t*)shards;
        int rc = xor_rows(base, Sb, RowSet{0, nd, t, nd}, base + uint64_t(t) * Sb, nullptr, st,
                          "kvec_gs_rdp_recover");
        if (rc) return rc;
    }
    if (copy_out) {
        int rc = copy_d2d(out_TN, shards, nc * 2, st, "kvec_gs_rdp_recover");
        if (rc) return rc;
        return zero_d((uint16_t*)out_TN + nc, (total - nc) * 2, st, "kvec_gs_rdp_recover");
    }
    return KVEC_OK;
}

// pack_row_from_block_launcher, bench_ghostserve_rdp.py:152-175:
// rows[row] = K words then V words.
extern "C" int kvec_gs_pack_row(const void* k_blk, const void* v_blk, void* rows, int64_t words,
                                int row, int64_t S, void* stream) {
    if (words < 0 || S < 2 * words || row < 0)
        return set_error(KVEC_EINVAL, "kvec_gs_pack_row: need S >= 2*words (S=%lld, words=%lld)",
                         (long long)S, (long long)words);
    if (words && (!k_blk || !v_blk || !rows)) return set_error(KVEC_EINVAL, "kvec_gs_pack_row: null pointer");
    hipStream_t st = as_stream(stream);
    uint16_t* rp = (uint16_t*)rows + uint64_t(row) * uint64_t(S);
    int rc = copy_d2d(rp, k_blk, uint64_t(words) * 2, st, "kvec_gs_pack_row");
    if (rc) return rc;
    return copy_d2d(rp + words, v_blk, uint64_t(words) * 2, st, "kvec_gs_pack_row");
}

// compute_rdp_parity_launcher, bench_ghostserve_rdp.py:177-199 (row stride S).
extern "C" int kvec_gs_rdp_parity(void* rows, int nd, int S, int star_base, void* stream) {
    if (!rows) return set_error(KVEC_EINVAL, "kvec_gs_rdp_parity: null rows");
    return gs_rdp_parity((uint16_t*)rows, nd, S, star_base, as_stream(stream), "kvec_gs_rdp_parity");
}
