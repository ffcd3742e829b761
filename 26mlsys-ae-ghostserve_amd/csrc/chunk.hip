// chunk.hip -- chunked coding of a paged KV pool, as prefill chunks arrive.
//
// One pass over a chunk's token records in the pool writes, in the chunk's own
// region of whole-sequence stripes:
//   * (optionally) the k data shards,
//   * textbook RDP(p) row parity P and diagonal parity Q over those k shards
//     (k <= p-1; columns k..p-2 of the code are implicit zeros),
//   * systematic RS(k, m) parity over GF(2^8)/0x11D (Cauchy) over the same k
//     shards.
//
// Layout: every shard of the whole-sequence stripe set holds one region of
// (p-1)*W bytes per chunk; chunk c's region starts at region_off (c*(p-1)*W
// for chunks in order).  A region is a spec RDP stripe set in the striped
// geometry of kvec_internal.h with rows of W bytes and unit U: stripe s has
// p-1 rows of g_s = min(U, W - s*U) bytes, row r at region_off + s*(p-1)*U +
// r*g_s.  Chunk c's stream (its token records in order, paged_geom.h), zero
// padded to k*(p-1)*W bytes, is cut into k shard pieces of (p-1)*W bytes, so
// data byte (shard j, stripe s, row r, offset o) is stream byte
// j*(p-1)*W + s*(p-1)*U + r*g_s + o.  Both codes work on their own stripe
// instances, so a chunk touches only its own region: no parity is read back,
// and each chunk's region is final once it is coded.
//
// The inverse rebuilds lost data cells straight into the pool pages: surviving
// data cells are read from the pool (the pool is the primary copy of the data),
// parity from the stripe buffers.  Lost parity shards are then re-encoded.
#include "gf8.h"
#include "paged_geom.h"
#include "rdp_plan.h"

namespace kvec {

constexpr int kChunkMaxK = 12;
constexpr int kChunkMaxM = 4;
constexpr int kCBS = 128;  // the decode kernels: two waves per block

// write-mask bits of the encode kernel; RS parity i is bit kWRs + i
constexpr uint32_t kWData = 1u, kWP = 2u, kWQ = 4u, kWRs = 3;

struct ChunkGeom {
    uint64_t nb;              // bytes of every shard buffer
    uint32_t region;          // byte offset of the chunk's region in every shard
    uint32_t recs_per_shard;  // (p-1)*W / record bytes: one data shard's piece
    RdpGeom geo;              // the region's stripes (rows of W bytes, unit U)
    uint32_t nwaves;          // waves over the stripes' rows (1 KiB each)
};

// A thread's place in the chunk's region: wave blockIdx*2 + (tid >> 6) of the
// stripes' rows, 16 bytes per lane.  Row r of the thread's stripe starts at
// shard byte rowbase + r*g (wave-uniform); the thread's bytes are at o within
// the row.  Its data cell (j, r) is record j*recs_per_shard + r*g_rec + lane_rec.
struct ChunkPos {
    uint32_t rowbase, g, o;
    uint32_t lane_rec, g_rec, inner;
    bool ok;
};

__device__ __forceinline__ ChunkPos chunk_pos(const PagedGeom& g, const ChunkGeom& cg, int rows) {
    const uint32_t wave = blockIdx.x * (kCBS / 64) + (threadIdx.x >> 6);
    const RdpWave w = rdp_wave(cg.geo, rows, wave, threadIdx.x & 63);
    ChunkPos c;
    c.ok = wave < cg.nwaves && w.within < w.g;
    c.rowbase = cg.region + uint32_t(w.base);
    c.g = uint32_t(w.g);
    c.o = w.within;
    const uint32_t w0 = fdiv(c.o, g.div_rec);
    c.inner = c.o - w0 * g.rec;
    c.lane_rec = fdiv(uint32_t(w.base), g.div_rec) + w0;
    c.g_rec = fdiv(c.g, g.div_rec);
    return c;
}

__device__ __forceinline__ uint32_t cell_rec(const ChunkGeom& cg, const ChunkPos& c, int j, int r) {
    return uint32_t(j) * cg.recs_per_shard + uint32_t(r) * c.g_rec + c.lane_rec;
}

template <int N>
struct Gf8Tab {
    uint32_t t[N][6];
};

// Copy a coefficient table set from the kernel arguments to LDS.  Read back
// from LDS, the v_perm tables land in VGPRs at their point of use instead of
// holding up to 6*k*m SGPRs for the whole kernel (which overflow the SGPR file
// next to the shard buffer resources and get spilled).
template <int N>
__device__ __forceinline__ void stage_tables(uint32_t (*lds)[6], const Gf8Tab<N>& tab) {
    for (int i = threadIdx.x; i < N * 6; i += blockDim.x) lds[i / 6][i % 6] = tab.t[i / 6][i % 6];
    __syncthreads();
}

// Pool cell (shard j, row r) of the thread's instance; zero for padding records.
__device__ __forceinline__ u32x4 load_cell(const PagedGeom& g, const ChunkGeom& cg, const ChunkPos& c,
                                           int j, int r) {
    return cell_load(g, cell_rec(cg, c, j, r), c.inner);
}

// ------------------------------------------------------------------ encode
// One row per wave.  A block of p-1 waves owns one 1 KiB column piece of a
// stripe; wave r codes row r.  It loads its k cells (page-table entries, then
// the cells) and writes the data cells, P[r] and the RS parity of row r, none
// of which needs another row.  Q mixes rows: cell (r, j) lies on diagonal
// (r + j) % p and P[r] on r - 1, so every wave XORs its cells into the LDS
// accumulators of their diagonals, and after one barrier wave d stores Q[d].
// Compared with one wave walking all rows of its column (two rows in flight,
// 165 VGPRs, 3 waves per SIMD), the waves are p-1 times more numerous and
// short, and at 55 VGPRs and 6 KiB of LDS per block five blocks share a CU:
// the encode of the 16 x 2048-token fp8 chunk went from 103.6 to 98.7 us.
// The same kernel with the Q diagonals exchanged through per-(diagonal, row)
// LDS slots (37 KiB per block, four blocks per CU) took 103.0 us, and with
// two or four columns per wave (fewer, longer waves) 102.7 and 112.7 us.
template <int P, int K, int M, bool DATA>
__global__ __launch_bounds__((P - 1) * 64) void chunk_encode_rows_kernel(
        PagedGeom g, ChunkGeom cg, Ptrs<kChunkMaxK> d, Ptrs<2 + kChunkMaxM> par,
        Gf8Tab<(K * M > 0 ? K * M : 1)> rs, uint32_t wmask) {
    constexpr int ROWS = P - 1;
    constexpr int NT = K * M > 0 ? K * M : 1;
    __shared__ uint32_t tab[NT][6];
    __shared__ uint32_t qacc[ROWS][4][64];  // Q[diagonal], dword-major per lane
    const int r = int(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    const uint32_t lane = threadIdx.x & 63;
    const RdpWave w = rdp_wave(cg.geo, ROWS, blockIdx.x, lane);
    // A short last stripe's rows end before the pieces its unit spans: a piece
    // that starts past the end codes nothing (every wave of the block leaves
    // here).  In the piece that holds the end, lanes past it take offset 0 of
    // the row: they compute lane 0's values and store them to lane 0's
    // addresses (lane 0 is inside the row), and they still reach the barrier.
    const uint32_t piece = uint32_t(__builtin_amdgcn_readfirstlane(w.within));  // lane 0: the piece's start
    if (piece >= w.g) return;
    const uint32_t o = w.within < w.g ? w.within : 0u;
    const uint32_t w0 = fdiv(o, g.div_rec);
    const uint32_t inner = o - w0 * g.rec;
    // cell (j, r) is record j*recs_per_shard + rbase + w0: rbase is the
    // wave's, w0 <= dmax the lane's record within the 1 KiB piece
    const uint32_t rbase = uint32_t(r) * fdiv(uint32_t(w.g), g.div_rec) + fdiv(uint32_t(w.base), g.div_rec);
    const uint32_t dmax = fdiv(piece + kRdpWaveBytes - 16, g.div_rec);
    CellRef ref[K];
#pragma unroll
    for (int j = 0; j < K; ++j) ref[j] = cell_ref_run(g, uint32_t(j) * cg.recs_per_shard + rbase, w0, dmax);
    u32x4 x[K];
#pragma unroll
    for (int j = 0; j < K; ++j) x[j] = cell_load_ref(g, ref[j], inner);
    // while the cells are in flight: clear this row's Q accumulators and stage
    // the RS tables (the barrier inside orders both before any use)
#pragma unroll
    for (int e = 0; e < 4; ++e) qacc[r][e][lane] = 0;
    stage_tables<NT>(tab, rs);
    const uint32_t soff = cg.region + uint32_t(w.base) + uint32_t(r) * uint32_t(w.g) + o;
    const uint64_t nb = cg.nb;
    // Outputs that wmask switches off get a buffer resource of size 0, whose
    // stores the hardware drops.  With no branches around the stores, the
    // compiler cannot sink each output's products into a branch of its own
    // and keep every input's fields live across them.
    auto out = [&](uint8_t* p, uint32_t bit) { return ShardView<true>(p, (wmask & bit) ? nb : 0); };
    if constexpr (DATA) {
#pragma unroll
        for (int j = 0; j < K; ++j) ShardView<true>(d.p[j], nb).store(0, soff, x[j]);
    }
    const u32x4 pr = xor_all<K>(x);
    out(par.p[0], kWP).store(0, soff, pr);
    auto qadd = [&](int dg, const u32x4& v) {
        atomicXor(&qacc[dg][0][lane], v.x);
        atomicXor(&qacc[dg][1][lane], v.y);
        atomicXor(&qacc[dg][2][lane], v.z);
        atomicXor(&qacc[dg][3][lane], v.w);
    };
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const int dg = (r + j) % P;
        if (dg != P - 1) qadd(dg, x[j]);  // diagonal p-1 is not stored
    }
    if (r >= 1) qadd(r - 1, pr);
    if constexpr (M > 0) {
        u32x4 acc[M];
#pragma unroll
        for (int i = 0; i < M; ++i) acc[i] = u32x4{0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < K; ++j) {
            Gf8Fields f[4];
            gf8_fields16(x[j], f);
#pragma unroll
            for (int i = 0; i < M; ++i) acc[i] = gf8_fma16(acc[i], f, tab[i * K + j]);
            // read each input's tables from LDS next to their use, rather
            // than all k*m of them up front into registers
            asm volatile("" ::: "memory");
        }
#pragma unroll
        for (int i = 0; i < M; ++i) out(par.p[2 + i], 1u << (kWRs + i)).store(0, soff, acc[i]);
    }
    __syncthreads();
    out(par.p[1], kWQ).store(0, soff, u32x4{qacc[r][0][lane], qacc[r][1][lane], qacc[r][2][lane], qacc[r][3][lane]});
}

// ------------------------------------------------------------------ RS decode
// Row by row: out_o = XOR_q M[o][q] * in_q.  Input q is data shard src_shard[q]
// read from the pool when in_buf[q] is null, else the parity buffer in_buf[q].
// Output o goes to the pool cells of data shard dst_shard[o] (if >= 0) and to
// out_buf[o] (if not null).
struct RsDecodeIo {
    uint8_t* in_buf[kChunkMaxK];
    int src_shard[kChunkMaxK];
    uint8_t* out_buf[kChunkMaxM];
    int dst_shard[kChunkMaxM];
};

// One row per wave, as in the encode: a block of ROWS waves owns one 1 KiB
// column piece of a stripe and wave r decodes row r (RS mixes no rows).  Each
// wave requests its K inputs' page-table entries, then the cells (parity
// inputs straight from their buffers), stages the coefficient tables while they
// load, and stores its NOUT outputs.  Lanes past a short last stripe's end
// take the row's offset 0, compute lane 0's values and store them to lane 0's
// addresses.  A wave walking its column's rows (two in flight, references in a
// ring of three rows, 128-thread blocks) decoded the 16 x 2048-token fp8
// chunk's three lost data shards in 114.5 us.
template <int ROWS, int K, int NOUT>
__global__ __launch_bounds__(ROWS * 64) void chunk_rs_decode_kernel(PagedGeom g, ChunkGeom cg, RsDecodeIo io,
                                                                    Gf8Tab<K * NOUT> mix) {
    __shared__ uint32_t tab[K * NOUT][6];
    const int r = int(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    const uint32_t lane = threadIdx.x & 63;
    const RdpWave w = rdp_wave(cg.geo, ROWS, blockIdx.x, lane);
    const uint32_t piece = uint32_t(__builtin_amdgcn_readfirstlane(w.within));  // lane 0: the piece's start
    if (piece >= w.g) return;   // the whole block: its piece starts past the short stripe's end
    const uint32_t o = w.within < w.g ? w.within : 0u;
    const uint32_t w0 = fdiv(o, g.div_rec);
    const uint32_t inner = o - w0 * g.rec;
    const uint32_t rbase = uint32_t(r) * fdiv(uint32_t(w.g), g.div_rec) + fdiv(uint32_t(w.base), g.div_rec);
    const uint32_t dmax = fdiv(piece + kRdpWaveBytes - 16, g.div_rec);
    const uint32_t soff = cg.region + uint32_t(w.base) + uint32_t(r) * uint32_t(w.g) + o;
    const uint64_t nb = cg.nb;
    CellRef rin[K], rout[NOUT];
#pragma unroll
    for (int q = 0; q < K; ++q)
        if (!io.in_buf[q]) rin[q] = cell_ref_run(g, uint32_t(io.src_shard[q]) * cg.recs_per_shard + rbase, w0, dmax);
#pragma unroll
    for (int i = 0; i < NOUT; ++i)
        if (io.dst_shard[i] >= 0)
            rout[i] = cell_ref_run(g, uint32_t(io.dst_shard[i]) * cg.recs_per_shard + rbase, w0, dmax);
    u32x4 x[K];
#pragma unroll
    for (int q = 0; q < K; ++q)
        x[q] = io.in_buf[q] ? ShardView<true>(io.in_buf[q], nb).load(0, soff) : cell_load_ref(g, rin[q], inner);
    stage_tables<K * NOUT>(tab, mix);   // while the cells load
    u32x4 acc[NOUT];
#pragma unroll
    for (int i = 0; i < NOUT; ++i) acc[i] = u32x4{0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < K; ++q) {
        Gf8Fields f[4];
        gf8_fields16(x[q], f);
#pragma unroll
        for (int i = 0; i < NOUT; ++i) {
            acc[i] = gf8_fma16(acc[i], f, tab[i * K + q]);
            // the products are formed here, input by input, with each
            // input's tables read from LDS next to their use: left free, the
            // compiler sinks each output's products into its store branch and
            // keeps every input's fields live (138 VGPRs for five inputs and
            // three outputs)
            asm volatile("" : "+v"(acc[i].x), "+v"(acc[i].y), "+v"(acc[i].z), "+v"(acc[i].w)::"memory");
        }
    }
#pragma unroll
    for (int i = 0; i < NOUT; ++i) {
        if (io.dst_shard[i] >= 0) cell_store_ref(g, rout[i], inner, acc[i]);
        if (io.out_buf[i]) ShardView<true>(io.out_buf[i], nb).store(0, soff, acc[i]);
    }
}

// ------------------------------------------------------------------ RDP decode
// The erasure pattern's XOR map (rdp_plan.h) over cells: data cells come from
// (and rebuilt ones go to) the pool, P and Q cells from the parity buffers.
// One output cell at a time, so re-read inputs come from cache.
__device__ __forceinline__ u32x4 rdp_cell_load(const PagedGeom& g, const ChunkGeom& cg, int k,
                                               int rows, const uint8_t* P, const uint8_t* Q, int c,
                                               const ChunkPos& cp) {
    const int s = c / rows, r = c - s * rows;
    if (s < k) return load_cell(g, cg, cp, s, r);
    return ld16((s == k ? P : Q) + uint64_t(cp.rowbase + uint32_t(r) * cp.g) + cp.o);
}

__global__ __launch_bounds__(kCBS) void chunk_rdp_decode_kernel(PagedGeom g, ChunkGeom cg, int k,
                                                                int rows, Ptrs<kChunkMaxK> d,
                                                                uint8_t* P, uint8_t* Q, RdpPlan plan) {
    const ChunkPos cp = chunk_pos(g, cg, rows);
    if (!cp.ok) return;
    for (int oc = 0; oc < plan.nout; ++oc) {
        u32x4 acc = {0, 0, 0, 0};
        for (int wd = 0; wd < kRdpNW; ++wd) {
            uint64_t msk = plan.mask[oc][wd];
            while (msk) {
                const int c = wd * 64 + __builtin_ctzll(msk);
                msk &= msk - 1;
                acc ^= rdp_cell_load(g, cg, k, rows, P, Q, c, cp);
            }
        }
        const int c = plan.out_cell[oc];
        const int s = c / rows, r = c - s * rows;
        const uint64_t rowoff = cp.rowbase + uint32_t(r) * cp.g;
        if (s < k) {
            cell_store(g, cell_rec(cg, cp, s, r), cp.inner, acc);
            if (d.p[s]) st_stream(d.p[s] + rowoff, cp.o, acc);
        } else {
            st_stream((s == k ? P : Q) + rowoff, cp.o, acc);
        }
    }
}

// RS parities the RDP decode re-encodes in the same pass: n of them, to
// out[0..n), with the encode's Cauchy rows of those parities as the tables.
struct RsReenc {
    uint8_t* out[kChunkMaxM];
    int n;
};

// The same map solved at compile time (p = 7, k = 5, the chunked shape), one
// row per wave: a block of p - 1 waves owns one 1 KiB column piece.  Wave r
// loads the cells of row r that the map needs (page-table entries first; P and
// Q from their buffers) and publishes them in LDS; after one barrier it
// rebuilds the lost cells of row r from LDS (straight-line XORs of the map)
// and stores them.  With RS parities lost as well, it then holds all k data
// cells of its row (the surviving ones loaded, the rebuilt ones computed) and
// re-encodes those parities of row r, so the data shards are read once.
// Lanes past a short last stripe's end take offset 0 of the row, as in the
// encode.  A wave walking its whole column (every needed cell in registers,
// 146-178 VGPRs, 2-3 waves per SIMD) followed by a separate RS re-encode
// took 77 + 78 us for two lost data shards and the three RS parities of the
// 16 x 2048-token fp8 chunk.
template <int P, int K, int E0, int E1>
__global__ __launch_bounds__((P - 1) * 64) void chunk_rdp_decode_rows(PagedGeom g, ChunkGeom cg,
                                                                      Ptrs<kChunkMaxK> d, uint8_t* Pp,
                                                                      uint8_t* Qp, RsReenc rs,
                                                                      Gf8Tab<K * kChunkMaxM> rtab) {
    constexpr int ROWS = P - 1, NC = (K + 2) * ROWS;
    constexpr RdpPlan plan = make_rdp_plan(P, K, E0, E1);
    static_assert(plan.ok, "RDP erasure pattern not decodable");
    static_assert(NC <= 64, "the map's cells in one mask word");
    constexpr uint64_t need = plan.need[0];
    constexpr int NS = __builtin_popcountll(need);
    __shared__ u32x4 cells[NS][64];   // the needed cells in cell order, lane-major
    __shared__ uint32_t tab[K * kChunkMaxM][6];
    const int r = int(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    const uint32_t lane = threadIdx.x & 63;
    const RdpWave w = rdp_wave(cg.geo, ROWS, blockIdx.x, lane);
    const uint32_t piece = uint32_t(__builtin_amdgcn_readfirstlane(w.within));  // lane 0: the piece's start
    if (piece >= w.g) return;   // the whole block: its piece starts past the short stripe's end
    const uint32_t o = w.within < w.g ? w.within : 0u;
    const uint32_t w0 = fdiv(o, g.div_rec);
    const uint32_t inner = o - w0 * g.rec;
    const uint32_t rbase = uint32_t(r) * fdiv(uint32_t(w.g), g.div_rec) + fdiv(uint32_t(w.base), g.div_rec);
    const uint32_t dmax = fdiv(piece + kRdpWaveBytes - 16, g.div_rec);
    const uint32_t soff = cg.region + uint32_t(w.base) + uint32_t(r) * uint32_t(w.g) + o;
    const uint64_t nb = cg.nb;
    const ShardView<true> sp(Pp, nb), sq(Qp, nb);
    auto needed = [&](int c) { return ((need >> c) & 1) != 0; };
    auto lost = [](int sh) { return sh == E0 || sh == E1; };
    const bool reenc = rs.n > 0;
    // this row's cells: the needed ones, and every surviving data cell when
    // RS parities are re-encoded.  Every load is issued; one not wanted reads
    // the zero cell (data) or nothing (P, Q through an empty resource).  Loads
    // under per-row conditions left the compiler merging register copies of
    // the cells at every join (400 moves, 149 VGPRs for one lost shard).
    CellRef ref[K];
#pragma unroll
    for (int sh = 0; sh < K; ++sh) {
        if (lost(sh)) continue;
        ref[sh] = cell_ref_run(g, uint32_t(sh) * cg.recs_per_shard + rbase, w0, dmax);
        if (!(reenc || needed(sh * ROWS + r))) ref[sh].base = kNoCell;
    }
    u32x4 x[K + 2];
#pragma unroll
    for (int sh = 0; sh < K; ++sh)
        if (!lost(sh)) x[sh] = cell_load_ref(g, ref[sh], inner);
    if (!lost(K)) x[K] = ShardView<true>(Pp, needed(K * ROWS + r) ? nb : 0).load(0, soff);
    if (!lost(K + 1)) x[K + 1] = ShardView<true>(Qp, needed((K + 1) * ROWS + r) ? nb : 0).load(0, soff);
    if (reenc)   // uniform; the barrier inside also orders the tables before their use
        stage_tables<K * kChunkMaxM>(tab, rtab);
    // publish the row's needed cells (slot = needed cells before c)
#pragma unroll
    for (int sh = 0; sh < K + 2; ++sh) {
        if (lost(sh)) continue;
        const int c = sh * ROWS + r;
        if (needed(c)) cells[__builtin_popcountll(need & ((uint64_t(1) << c) - 1))][lane] = x[sh];
    }
    __syncthreads();
    // the lost cells of row r
#pragma unroll
    for (int i = 0; i < plan.nout; ++i) {
        const int oc = plan.out_cell[i], osh = oc / ROWS;
        if (oc % ROWS != r) continue;
        // each output's LDS reads stay inside its branch: hoisted, the reads
        // of all the map's outputs are held at once
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        u32x4 acc = {0, 0, 0, 0};
        int terms = 0;   // a compile-time count after unrolling
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (!((plan.mask[i][0] >> c) & 1)) continue;
            acc ^= cells[__builtin_popcountll(need & ((uint64_t(1) << c) - 1))][lane];
            // four LDS reads in flight at a time: unfenced, all of an output's
            // reads are issued first (90 VGPRs for a pair of lost shards)
            if (++terms % 4 == 0) asm volatile("" : "+v"(acc.x), "+v"(acc.y), "+v"(acc.z), "+v"(acc.w)::"memory");
        }
        if (osh < K) {
            const CellRef oref = cell_ref_run(g, uint32_t(osh) * cg.recs_per_shard + rbase, w0, dmax);
            cell_store_ref(g, oref, inner, acc);
            if (d.p[osh]) st_stream(d.p[osh], soff, acc);
        } else {
            (osh == K ? sp : sq).store(0, soff, acc);
        }
        x[osh] = acc;
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    }
    if (!reenc) return;
    // the lost RS parities of row r from its k data cells
    u32x4 racc[kChunkMaxM];
#pragma unroll
    for (int j = 0; j < kChunkMaxM; ++j) racc[j] = u32x4{0, 0, 0, 0};
#pragma unroll
    for (int sh = 0; sh < K; ++sh) {
        Gf8Fields f[4];
        gf8_fields16(x[sh], f);
#pragma unroll
        for (int j = 0; j < kChunkMaxM; ++j) {
            if (j >= rs.n) break;
            racc[j] = gf8_fma16(racc[j], f, tab[j * K + sh]);
            // formed here, input by input (see chunk_rs_decode_kernel)
            asm volatile("" : "+v"(racc[j].x), "+v"(racc[j].y), "+v"(racc[j].z), "+v"(racc[j].w)::"memory");
        }
    }
#pragma unroll
    for (int j = 0; j < kChunkMaxM; ++j)
        if (j < rs.n) ShardView<true>(rs.out[j], nb).store(0, soff, racc[j]);
}

// ------------------------------------------------------------------ dispatch
// Launch the encode instantiation <P, K, M> with a table sized for it.
template <int P, int K, int M>
static void launch_encode(hipStream_t st, const PagedGeom& g, const ChunkGeom& cg,
                          const Ptrs<kChunkMaxK>& d, const Ptrs<2 + kChunkMaxM>& par,
                          const uint32_t (*tab)[6], uint32_t wmask) {
    Gf8Tab<(K * M > 0 ? K * M : 1)> t{};
    for (int i = 0; i < K * M; ++i)
        for (int e = 0; e < 6; ++e) t.t[i][e] = tab[i][e];
    // one block of p-1 waves per 1 KiB column piece
    const dim3 rgrid(cg.nwaves), rblock((P - 1) * 64);
    if (wmask & kWData)
        hipLaunchKernelGGL((chunk_encode_rows_kernel<P, K, M, true>), rgrid, rblock, 0, st, g, cg, d, par,
                           t, wmask);
    else
        hipLaunchKernelGGL((chunk_encode_rows_kernel<P, K, M, false>), rgrid, rblock, 0, st, g, cg, d, par,
                           t, wmask);
}

typedef void (*EncLauncher)(hipStream_t, const PagedGeom&, const ChunkGeom&,
                            const Ptrs<kChunkMaxK>&, const Ptrs<2 + kChunkMaxM>&,
                            const uint32_t (*)[6], uint32_t);

template <int P, int K, int M = 0>
EncLauncher pick_encode_m(int m) {
    if constexpr (M > 3) {
        return nullptr;
    } else {
        if (m == M) return &launch_encode<P, K, M>;
        return pick_encode_m<P, K, M + 1>(m);
    }
}

template <int P, int K = 2>
EncLauncher pick_encode_k(int k, int m) {
    if constexpr (K > P - 1) {
        return nullptr;
    } else {
        if (k == K) return pick_encode_m<P, K>(m);
        return pick_encode_k<P, K + 1>(k, m);
    }
}

// Built: p in {3, 5, 7}, 2 <= k <= p-1, 0 <= m <= 3.
static EncLauncher encode_launcher(int p, int k, int m) {
    switch (p) {
        case 3: return pick_encode_k<3>(k, m);
        case 5: return pick_encode_k<5>(k, m);
        case 7: return pick_encode_k<7>(k, m);
        default: return nullptr;
    }
}

template <int ROWS, int K, int NOUT>
static void launch_rs_decode(hipStream_t st, const PagedGeom& g, const ChunkGeom& cg, const RsDecodeIo& io,
                             const uint32_t (*tab)[6]) {
    Gf8Tab<K * NOUT> t{};
    for (int i = 0; i < K * NOUT; ++i)
        for (int e = 0; e < 6; ++e) t.t[i][e] = tab[i][e];
    // one block of ROWS waves per 1 KiB column piece
    hipLaunchKernelGGL((chunk_rs_decode_kernel<ROWS, K, NOUT>), dim3(cg.nwaves), dim3(ROWS * 64), 0, st, g, cg, io,
                       t);
}

typedef void (*RsDecLauncher)(hipStream_t, const PagedGeom&, const ChunkGeom&, const RsDecodeIo&,
                              const uint32_t (*)[6]);

template <int ROWS, int K, int N = 1>
RsDecLauncher pick_rs_dec_n(int n) {
    if constexpr (N > 3) {
        return nullptr;
    } else {
        if (n == N) return &launch_rs_decode<ROWS, K, N>;
        return pick_rs_dec_n<ROWS, K, N + 1>(n);
    }
}

template <int ROWS, int K = 2>
RsDecLauncher pick_rs_dec_k(int k, int n) {
    if constexpr (K > ROWS) {
        return nullptr;
    } else {
        if (k == K) return pick_rs_dec_n<ROWS, K>(n);
        return pick_rs_dec_k<ROWS, K + 1>(k, n);
    }
}

// Built: p in {3, 5, 7} (rows 2, 4, 6), 2 <= k <= p-1, 1..3 outputs.
static RsDecLauncher rs_dec_launcher(int p, int k, int n) {
    switch (p) {
        case 3: return pick_rs_dec_k<2>(k, n);
        case 5: return pick_rs_dec_k<4>(k, n);
        case 7: return pick_rs_dec_k<6>(k, n);
        default: return nullptr;
    }
}

template <int K>
using RdpRowsFn = void (*)(PagedGeom, ChunkGeom, Ptrs<kChunkMaxK>, uint8_t*, uint8_t*, RsReenc,
                           Gf8Tab<K * kChunkMaxM>);

template <int P, int K, int E0, int E1 = E0 + 1>
RdpRowsFn<K> pick_rdp_rows_pair(int e1) {
    if constexpr (E1 > K + 1) {
        return nullptr;
    } else {
        if (e1 == E1) return &chunk_rdp_decode_rows<P, K, E0, E1>;
        return pick_rdp_rows_pair<P, K, E0, E1 + 1>(e1);
    }
}

// Patterns with at least one data shard (the only ones that reach the RDP path).
template <int P, int K, int E0 = 0>
RdpRowsFn<K> pick_rdp_rows(int e0, int e1) {
    if constexpr (E0 >= K) {
        return nullptr;
    } else {
        if (e0 == E0) {
            if (e1 < 0) return &chunk_rdp_decode_rows<P, K, E0, -1>;
            return pick_rdp_rows_pair<P, K, E0>(e1);
        }
        return pick_rdp_rows<P, K, E0 + 1>(e0, e1);
    }
}

struct ChunkArgs {
    PagedGeom g;
    ChunkGeom cg;
    Ptrs<kChunkMaxK> d;
    Ptrs<2 + kChunkMaxM> par;
    bool have_data;
    int k, p, m;
};

static int check_chunk(const kvec_paged_kv* kv, const kvec_chunk_stripe* st, ChunkArgs* a,
                       bool writes_pool, const char* fn) {
    int rc = make_geom(kv, &a->g, fn);
    if (rc) return rc;
    if (!st) return set_error(KVEC_EINVAL, "%s: null stripe", fn);
    const int k = st->k, p = st->p, m = st->m;
    if (!is_prime(p) || p < 3) return set_error(KVEC_EINVAL, "%s: p=%d is not an odd prime", fn, p);
    if (p > kRdpMaxP) return set_error(KVEC_EUNSUPPORTED, "%s: p=%d > %d", fn, p, kRdpMaxP);
    if (k < 1 || k > p - 1 || k > kChunkMaxK)
        return set_error(KVEC_EINVAL, "%s: k=%d not in [1, p-1]", fn, k);
    if (m < 0 || m > kChunkMaxM) return set_error(KVEC_EINVAL, "%s: m=%d not in [0, %d]", fn, m, kChunkMaxM);
    const uint64_t R = uint64_t(st->row_bytes), W = uint64_t(st->width), off = uint64_t(st->region_off);
    const uint64_t U = uint64_t(st->unit_bytes);
    if (st->row_bytes <= 0 || st->width <= 0 || st->region_off < 0 || st->unit_bytes < 0 || R % 16 ||
        off % 16)
        return set_error(KVEC_EINVAL, "%s: row_bytes/region_off must be multiples of 16, width > 0", fn);
    if (W % a->g.rec)
        return set_error(KVEC_EINVAL, "%s: width=%llu must be a multiple of the record size %u", fn,
                         (unsigned long long)W, a->g.rec);
    if (U % kRdpWaveBytes || U % a->g.rec)
        return set_error(KVEC_EINVAL, "%s: unit_bytes=%llu must be 0 or a multiple of 1024 and of the "
                         "record size %u", fn, (unsigned long long)U, a->g.rec);
    if (off + uint64_t(p - 1) * W > uint64_t(p - 1) * R)
        return set_error(KVEC_EINVAL, "%s: region_off + (p-1)*width > (p-1)*row_bytes", fn);
    if (!fits_buffer(uint64_t(p - 1) * R))
        return set_error(KVEC_EUNSUPPORTED, "%s: (p-1)*row_bytes must be < 4 GiB", fn);
    const uint64_t cells = uint64_t(k) * uint64_t(p - 1);
    if (cells * W < a->g.recs_total * a->g.rec)
        return set_error(KVEC_EINVAL, "%s: k*(p-1)*width=%llu < chunk stream bytes %llu", fn,
                         (unsigned long long)(cells * W),
                         (unsigned long long)(a->g.recs_total * a->g.rec));
    if (cells * (W / a->g.rec) >= (uint64_t(1) << 32) || a->g.recs_total * a->g.rec >= (uint64_t(1) << 32))
        return set_error(KVEC_EUNSUPPORTED, "%s: chunk too large for 32-bit record indices", fn);
    if (!st->P || !st->Q || !aligned16(st->P) || !aligned16(st->Q))
        return set_error(KVEC_EINVAL, "%s: P/Q null or not 16-byte aligned", fn);
    a->par = Ptrs<2 + kChunkMaxM>{};
    a->par.p[0] = (uint8_t*)st->P;
    a->par.p[1] = (uint8_t*)st->Q;
    if (m > 0 && !st->rs) return set_error(KVEC_EINVAL, "%s: null RS parity array", fn);
    for (int i = 0; i < m; ++i) {
        if (!st->rs[i] || !aligned16(st->rs[i]))
            return set_error(KVEC_EINVAL, "%s: rs[%d] null or not 16-byte aligned", fn, i);
        a->par.p[2 + i] = (uint8_t*)st->rs[i];
    }
    a->d = Ptrs<kChunkMaxK>{};
    a->have_data = st->data != nullptr;
    if (a->have_data)
        for (int j = 0; j < k; ++j) {
            if (!st->data[j] || !aligned16(st->data[j]))
                return set_error(KVEC_EINVAL, "%s: data[%d] null or not 16-byte aligned", fn, j);
            a->d.p[j] = (uint8_t*)st->data[j];
        }
    a->cg.nb = uint64_t(p - 1) * R;
    {
        // every shard of the stripe set may be written (and the pool, by a
        // decode); nothing written may share a byte with anything else
        Span w[kChunkMaxK + 3 + kChunkMaxM];
        Span r[2] = {pool_span(kv), table_span(kv)};
        int nw = 0, nr = 2;
        if (writes_pool) {
            w[nw++] = r[0];
            r[0] = r[1];
            nr = 1;
        }
        w[nw++] = Span{st->P, a->cg.nb, "P", -1};
        w[nw++] = Span{st->Q, a->cg.nb, "Q", -1};
        for (int i = 0; i < m; ++i) w[nw++] = Span{st->rs[i], a->cg.nb, "rs", i};
        if (a->have_data)
            for (int j = 0; j < k; ++j) w[nw++] = Span{st->data[j], a->cg.nb, "data", j};
        if ((rc = check_no_alias(w, nw, r, nr, fn))) return rc;
    }
    a->cg.region = uint32_t(off);
    a->cg.recs_per_shard = uint32_t(uint64_t(p - 1) * W / a->g.rec);
    a->cg.geo = make_rdp_geom(W, U);
    a->cg.nwaves = uint32_t(rdp_waves(a->cg.geo));
    a->k = k;
    a->p = p;
    a->m = m;
    return KVEC_OK;
}

static dim3 chunk_grid(const ChunkGeom& cg) { return dim3(blocks_for(cg.nwaves, kCBS / 64)); }

static int run_encode(const ChunkArgs& a, uint32_t wmask, hipStream_t st, const char* fn) {
    EncLauncher L = encode_launcher(a.p, a.k, a.m);
    if (!L) return set_error(KVEC_EUNSUPPORTED, "%s: p=%d k=%d m=%d not built", fn, a.p, a.k, a.m);
    uint8_t C[kRs8MaxM * kRs8MaxK];
    cauchy(a.k, a.m, C);
    uint32_t tab[kChunkMaxK * kChunkMaxM][6];
    for (int i = 0; i < a.k * a.m; ++i) perm_tables(C[i], tab[i]);
    L(st, a.g, a.cg, a.d, a.par, tab, wmask);
    return check_launch(fn);
}

}  // namespace kvec

using namespace kvec;

extern "C" int64_t kvec_chunk_width(int64_t chunk_stream_bytes, int k, int p, int64_t record_bytes) {
    if (chunk_stream_bytes < 0 || k < 1 || p < 3 || record_bytes < 16 || record_bytes % 16) return -1;
    const int64_t cells = int64_t(k) * (p - 1);
    const int64_t per = (chunk_stream_bytes + cells - 1) / cells;
    return (per + record_bytes - 1) / record_bytes * record_bytes;
}

extern "C" int kvec_chunk_encode_paged(const kvec_paged_kv* kv, const kvec_chunk_stripe* st,
                                       void* stream) {
    ChunkArgs a;
    int rc = check_chunk(kv, st, &a, false, "kvec_chunk_encode_paged");
    if (rc) return rc;
    uint32_t wmask = kWP | kWQ | (a.have_data ? kWData : 0u);
    for (int i = 0; i < a.m; ++i) wmask |= 1u << (kWRs + i);
    return run_encode(a, wmask, as_stream(stream), "kvec_chunk_encode_paged");
}

extern "C" int kvec_chunk_decode_paged(const kvec_paged_kv* kv, void* pool,
                                       const kvec_chunk_stripe* st, const int32_t* erased,
                                       int n_erased, void* stream) {
    static const char* fn = "kvec_chunk_decode_paged";
    ChunkArgs a;
    int rc = check_chunk(kv, st, &a, true, fn);
    if (rc) return rc;
    if (!pool || pool != kv->pool) return set_error(KVEC_EINVAL, "%s: pool must be kv->pool", fn);
    if (n_erased < 0 || (n_erased > 0 && !erased)) return set_error(KVEC_EINVAL, "%s: bad erasure list", fn);
    const int k = a.k, m = a.m, rows = a.p - 1, nsh = k + 2 + m;
    bool er[kChunkMaxK + 2 + kChunkMaxM] = {};
    for (int i = 0; i < n_erased; ++i) {
        if (erased[i] < 0 || erased[i] >= nsh)
            return set_error(KVEC_EINVAL, "%s: erased index %d not in [0, %d)", fn, erased[i], nsh);
        er[erased[i]] = true;
    }
    int nd = 0, nrs = 0;
    for (int s = 0; s < k; ++s) nd += er[s];
    for (int i = 0; i < m; ++i) nrs += er[k + 2 + i];
    const bool eP = er[k], eQ = er[k + 1];
    hipStream_t hs = as_stream(stream);
    const dim3 grid = chunk_grid(a.cg);
    uint32_t reenc = (eP ? kWP : 0u) | (eQ ? kWQ : 0u);
    if (nd > 0 && nd <= m - nrs) {
        // RS: data shards and RS parity, data first (index order k..k+m-1 for parity)
        bool er_rs[kChunkMaxK + kChunkMaxM] = {};
        for (int s = 0; s < k; ++s) er_rs[s] = er[s];
        for (int i = 0; i < m; ++i) er_rs[k + i] = er[k + 2 + i];
        int surv[kRs8MaxK], outs[kRs8MaxM], no = 0;
        uint8_t M[kRs8MaxM * kRs8MaxK];
        if (!rs8_decode_rows(k, m, er_rs, surv, outs, &no, M))
            return set_error(KVEC_EDECODE, "%s: RS survivor block singular", fn);
        RsDecodeIo io{};
        for (int q = 0; q < k; ++q) {
            io.src_shard[q] = surv[q] < k ? surv[q] : -1;
            io.in_buf[q] = surv[q] < k ? nullptr : a.par.p[2 + (surv[q] - k)];
        }
        for (int o = 0; o < no; ++o) {
            const int s = outs[o];
            io.dst_shard[o] = s < k ? s : -1;
            io.out_buf[o] = s < k ? (a.have_data ? a.d.p[s] : nullptr) : a.par.p[2 + (s - k)];
        }
        uint32_t tab[kChunkMaxK * kChunkMaxM][6];
        for (int i = 0; i < no * k; ++i) perm_tables(M[i], tab[i]);
        RsDecLauncher L = rs_dec_launcher(a.p, k, no);
        if (!L) return set_error(KVEC_EUNSUPPORTED, "%s: p=%d k=%d with %d outputs not built", fn, a.p, k, no);
        L(hs, a.g, a.cg, io, tab);
        rc = check_launch(fn);
        if (rc) return rc;
    } else if (nd > 0 && nd + int(eP) + int(eQ) <= 2) {
        // RDP: the data and P/Q erasures of the pattern, then RS parity re-encoded
        int e[2] = {-1, -1}, ne = 0;
        for (int s = 0; s < k + 2; ++s)
            if (er[s]) e[ne++] = s;
        RdpPlan plan = make_rdp_plan(a.p, k, e[0], e[1]);
        if (!plan.ok) return set_error(KVEC_EDECODE, "%s: RDP pattern (%d, %d) not decodable", fn, e[0], e[1]);
        Ptrs<kChunkMaxK> dd = a.have_data ? a.d : Ptrs<kChunkMaxK>{};
        reenc = 0;
        for (int i = 0; i < m; ++i)
            if (er[k + 2 + i]) reenc |= 1u << (kWRs + i);
        RdpRowsFn<5> fx = (a.p == 7 && k == 5) ? pick_rdp_rows<7, 5>(e[0], e[1]) : nullptr;
        if (fx) {
            // the lost RS parities re-encoded in the same pass
            RsReenc re{};
            Gf8Tab<5 * kChunkMaxM> rt{};
            uint8_t C[kRs8MaxM * kRs8MaxK];
            cauchy(k, m, C);
            for (int i = 0; i < m; ++i) {
                if (!er[k + 2 + i]) continue;
                for (int j = 0; j < k; ++j) perm_tables(C[i * k + j], rt.t[re.n * k + j]);
                re.out[re.n++] = a.par.p[2 + i];
            }
            hipLaunchKernelGGL(fx, dim3(a.cg.nwaves), dim3((a.p - 1) * 64), 0, hs, a.g, a.cg, dd, a.par.p[0],
                               a.par.p[1], re, rt);
            reenc = 0;
        } else {
            hipLaunchKernelGGL(chunk_rdp_decode_kernel, grid, dim3(kCBS), 0, hs, a.g, a.cg, k, rows, dd,
                               a.par.p[0], a.par.p[1], plan);
        }
        rc = check_launch(fn);
        if (rc) return rc;
    } else if (nd > 0) {
        return set_error(KVEC_EDECODE, "%s: %d data erasures with %d of %d RS parities lost and P/Q "
                         "lost (%d, %d) cannot be decoded", fn, nd, nrs, m, int(eP), int(eQ));
    } else {
        for (int i = 0; i < m; ++i)
            if (er[k + 2 + i]) reenc |= 1u << (kWRs + i);
    }
    if (reenc) return run_encode(a, reenc, hs, fn);
    return KVEC_OK;
}
