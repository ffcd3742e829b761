// gs_rs16.hip -- the reference's Reed-Solomon code over GF(2^16), bit-exact
// (benchmark/rs/kernel.cu:16-222), on its packed [(k+m), S] u16 tensors.
//
// Multiplication by a constant c is GF(2)-linear in the symbol x.  Each block
// asks the caller's log/exp tables (exactly the reference's gf_mul) only for
// the sixteen basis products c * 2^b, and builds from them, by linearity, four
// byte-to-byte maps per coefficient:
//     x * c = (lo(x) -> lo, hi(x) -> lo) in the low byte, (lo -> hi, hi -> hi) in the high byte.
// Each byte map is applied with the 3/3/2-bit field split of the GF(2^8)
// kernels: three v_perm_b32 byte-permutes of 8-entry tables, four bytes at a
// time.  The streaming loop therefore holds words byte-transposed: one
// register carries the low bytes of four words and one the high bytes, so a
// coefficient costs 12 v_perm_b32 per four words and no memory lookup.
//
// The encode's coefficients are powers of alpha^(p+1); when the caller's tables
// have alpha = 2 (checked per block), the encode instead folds the inputs by
// Horner's rule with packed-word doublings (below), about half the VALU work.
//
// Reconstruction folds the reference's two steps (right-hand side b, then
// x = V^-1 b) into one coefficient per (output, input) pair: exact in the
// field, so the bytes are those of the two-step computation.  The inverse is
// computed per block with the reference's Gauss-Jordan (pivot order and
// zero-pivot skip included), from indices read on the device.
#include "gf8.h"
#include "tile_engine.h"

namespace kvec {

constexpr int kGfOrder = 65535;
constexpr int kRsMaxM = 16;           // reference limit (benchmark/rs/kernel.cu:118)
constexpr int kRsMaxTables = 48;      // coefficients held in LDS
constexpr int kRs16Tab = 24;          // dwords per coefficient: 4 byte maps x 6
constexpr int kRsGroup = 2;           // outputs accumulated per pass over the inputs
constexpr int kRsGrid = 1024;         // persistent blocks (4 per CU): tables are built once per block

__device__ __forceinline__ uint16_t gf16_mul_tab(uint16_t a, uint16_t b, const uint16_t* ex,
                                                 const uint16_t* lg) {
    if (a == 0 || b == 0) return 0;
    int s = int(lg[a]) + int(lg[b]);
    if (s >= kGfOrder) s -= kGfOrder;
    return ex[s];
}

__device__ __forceinline__ uint16_t gf16_div_tab(uint16_t a, uint16_t b, const uint16_t* ex,
                                                 const uint16_t* lg) {
    if (a == 0 || b == 0) return 0;
    int d = int(lg[a]) - int(lg[b]);
    if (d < 0) d += kGfOrder;
    return ex[d];
}

struct RsJob {
    const uint16_t* in_rows[kRsMaxTables];  // k input rows (u16, logical column 0)
    uint16_t* out_rows[kRsMaxM];            // output rows
    int nin, nout;
    int64_t S;                              // words per row
    FlatCopy copy;                          // data rows -> shard rows (encode), or none
};

// Byte maps of coefficient t, ptab[t][24]: dwords 0-5 lo->lo, 6-11 hi->lo,
// 12-17 lo->hi, 18-23 hi->hi; within a map, the two dwords of field f (bits
// 3f.. of the source byte) hold the images of the field values 0-3 and 4-7.
// All threads call it.
__device__ __forceinline__ void rs_build_perm_tables(uint32_t (*ptab)[kRs16Tab], uint16_t (*basis)[16],
                                     const uint16_t* coef, int ncoef, const uint16_t* ex,
                                     const uint16_t* lg) {
    for (int e = threadIdx.x; e < ncoef * 16; e += kTB)
        basis[e >> 4][e & 15] = gf16_mul_tab(uint16_t(1u << (e & 15)), coef[e >> 4], ex, lg);
    __syncthreads();
    for (int e = threadIdx.x; e < ncoef * kRs16Tab; e += kTB) {
        const int t = e / kRs16Tab, d = e % kRs16Tab;
        const int map = d / 6, f = (d % 6) >> 1, half = d & 1;
        const int src = map & 1, dst = map >> 1;   // 0 = low byte, 1 = high byte
        uint32_t dw = 0;
        for (int q = 0; q < 4; ++q) {
            const int v = half * 4 + q;
            if (f == 2 && v >= 4) continue;
            const uint32_t x = uint32_t(v) << (3 * f);   // source byte value
            uint32_t y = 0;
            for (int b = 0; b < 8; ++b)
                if (x & (1u << b)) y ^= basis[t][b + 8 * src];
            dw |= ((y >> (8 * dst)) & 0xFFu) << (8 * q);
        }
        ptab[t][d] = dw;
    }
}

// Four words' low bytes into one register and their high bytes into another:
// b[0], b[1] for words 0-3 of the window, b[2], b[3] for words 4-7.
__device__ __forceinline__ void split_bytes(u32x4 x, uint32_t b[4]) {
    b[0] = __builtin_amdgcn_perm(x.y, x.x, 0x06040200u);
    b[1] = __builtin_amdgcn_perm(x.y, x.x, 0x07050301u);
    b[2] = __builtin_amdgcn_perm(x.w, x.z, 0x06040200u);
    b[3] = __builtin_amdgcn_perm(x.w, x.z, 0x07050301u);
}

__device__ __forceinline__ u32x4 join_bytes(const uint32_t a[4]) {
    return u32x4{__builtin_amdgcn_perm(a[1], a[0], 0x05010400u),
                 __builtin_amdgcn_perm(a[1], a[0], 0x07030602u),
                 __builtin_amdgcn_perm(a[3], a[2], 0x05010400u),
                 __builtin_amdgcn_perm(a[3], a[2], 0x07030602u)};
}

// acc ^ map_a(bytes of fa) ^ map_b(bytes of fb): six v_perm_b32, three 3-input XORs.
__device__ __forceinline__ uint32_t gf16_fma2(uint32_t acc, const Gf8Fields& fa, const uint32_t* ta,
                                              const Gf8Fields& fb, const uint32_t* tb) {
    const uint32_t p0 = __builtin_amdgcn_perm(ta[1], ta[0], fa.f0);
    const uint32_t p1 = __builtin_amdgcn_perm(ta[3], ta[2], fa.f1);
    const uint32_t p2 = __builtin_amdgcn_perm(ta[5], ta[4], fa.f2);
    const uint32_t p3 = __builtin_amdgcn_perm(tb[1], tb[0], fb.f0);
    const uint32_t p4 = __builtin_amdgcn_perm(tb[3], tb[2], fb.f1);
    const uint32_t p5 = __builtin_amdgcn_perm(tb[5], tb[4], fb.f2);
    return xor3(xor3(xor3(acc, p0, p1), p2, p3), p4, p5);
}

// Words w0 .. w0+7 of a row, zero past its end S.
__device__ __forceinline__ u32x4 rs_window(const uint16_t* row, int64_t w0, int64_t S) {
    if (w0 + 8 <= S) return load_window16(reinterpret_cast<const uint8_t*>(row + w0));
    const gptr<const uint16_t> r = as_global(row) + (w0 < S ? w0 : 0);
    const int nq = w0 < S ? int(S - w0) : 0;   // < 8 here
    uint32_t v[4] = {0, 0, 0, 0};
    for (int q = 0; q < nq; ++q) v[q >> 1] |= uint32_t(r[q]) << (16 * (q & 1));
    return u32x4{v[0], v[1], v[2], v[3]};
}

// Fold input i's NW windows x[] into outputs og .. og+G-1: acc[n][g] holds
// them byte-transposed (split_bytes order).  Each coefficient's tables are
// read from LDS once and applied to all NW windows.
template <int G, int NW>
__device__ __forceinline__ void rs_mix_input(const uint32_t (*ptab)[kRs16Tab], int og, int nin,
                                             int i, const u32x4* x, uint32_t (*acc)[kRsGroup][4]) {
    Gf8Fields f[NW][4];
#pragma unroll
    for (int n = 0; n < NW; ++n) {
        uint32_t by[4];
        split_bytes(x[n], by);
#pragma unroll
        for (int q = 0; q < 4; ++q) f[n][q] = gf8_fields(by[q]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const uint32_t* T = ptab[(og + g) * nin + i];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            acc[n][g][0] = gf16_fma2(acc[n][g][0], f[n][0], T + 0, f[n][1], T + 6);
            acc[n][g][1] = gf16_fma2(acc[n][g][1], f[n][0], T + 12, f[n][1], T + 18);
            acc[n][g][2] = gf16_fma2(acc[n][g][2], f[n][2], T + 0, f[n][3], T + 6);
            acc[n][g][3] = gf16_fma2(acc[n][g][3], f[n][2], T + 12, f[n][3], T + 18);
        }
    }
}

template <int G, int NW>
__device__ __forceinline__ void rs_zero(uint32_t (*acc)[kRsGroup][4]) {
#pragma unroll
    for (int n = 0; n < NW; ++n)
#pragma unroll
        for (int g = 0; g < G; ++g) acc[n][g][0] = acc[n][g][1] = acc[n][g][2] = acc[n][g][3] = 0;
}

// A tile wholly inside the rows, software pipelined over the inputs: input
// i+1's aligned chunks are in flight while input i is folded in.
// With `copy`, the loaded chunks of every input also go to the copy's
// destination (the data rows of an encode are the inputs, in order).
template <int G, int NW>
__device__ __forceinline__ void rs_mix_full(const RsJob& j, const uint32_t (*ptab)[kRs16Tab],
                                            int og, uint64_t t0b, bool copy,
                                            uint32_t (*acc)[kRsGroup][4]) {
    rs_zero<G, NW>(acc);
    const int nin = j.nin;
    u32x4 lo[NW], hi[NW];
    RowWin rw = row_win(reinterpret_cast<const uint8_t*>(j.in_rows[0]) + t0b);
#pragma unroll
    for (int n = 0; n < NW; ++n) win_chunks(rw, 16 * (threadIdx.x + n * kTB), lo[n], hi[n]);
    for (int i = 0; i < nin; ++i) {
        u32x4 x[NW];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            x[n] = win_join(rw, lo[n], hi[n]);
            if (copy) copy_owned<false>(j.copy, rw, 16 * (threadIdx.x + n * kTB), lo[n], hi[n]);
        }
        if (i + 1 < nin) {
            rw = row_win(reinterpret_cast<const uint8_t*>(j.in_rows[i + 1]) + t0b);
#pragma unroll
            for (int n = 0; n < NW; ++n) win_chunks(rw, 16 * (threadIdx.x + n * kTB), lo[n], hi[n]);
        }
        rs_mix_input<G, NW>(ptab, og, nin, i, x, acc);
    }
}

// The last, partial tile.  Whole windows are read, and copied, as in a full
// tile (aligned chunks, each lane storing the chunk that starts inside its
// window); the one window that reaches past the row's end is read word by
// word and copies its own words.
template <int G, int NW>
__device__ __forceinline__ void rs_mix_tail(const RsJob& j, const uint32_t (*ptab)[kRs16Tab],
                                            int og, uint64_t t0b, const int64_t* w0, bool copy,
                                            uint32_t (*acc)[kRsGroup][4]) {
    rs_zero<G, NW>(acc);
    for (int i = 0; i < j.nin; ++i) {
        const RowWin rw = row_win(reinterpret_cast<const uint8_t*>(j.in_rows[i]) + t0b);
        u32x4 x[NW];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            const uint32_t off = 16 * (threadIdx.x + n * kTB);
            if (w0[n] + 8 <= j.S) {
                u32x4 lo, hi;
                win_chunks(rw, off, lo, hi);
                x[n] = win_join(rw, lo, hi);
                if (copy) copy_owned<false>(j.copy, rw, off, lo, hi);
            } else {
                x[n] = rs_window(j.in_rows[i], w0[n], j.S);
                if (copy && w0[n] < j.S) {
                    const uint64_t o = uint64_t(reinterpret_cast<const uint8_t*>(j.in_rows[i] + w0[n]) -
                                                j.copy.src);
                    copy_bytes(j.copy, o, o + 2 * uint64_t(j.S - w0[n]));
                }
            }
        }
        rs_mix_input<G, NW>(ptab, og, j.nin, i, x, acc);
    }
}

// ------------------------------------------------------------ Horner encode
// The encode's coefficients are powers, c(p, i) = g_p^i with g_p = alpha^(p+1),
// so parity p is also D_0 ^ g_p (D_1 ^ g_p (D_2 ^ ...)): inputs taken from the
// last to the first, the accumulator multiplied by g_p before each one.  With
// alpha = 2 that product is p + 1 doublings, each a shift of the two packed
// words and, for a word whose top bit was set, an XOR of the field
// polynomial's low 16 bits: three or four VALU ops per dword instead of the
// byte maps' twelve v_perm_b32 and six XORs per coefficient.  The kernel takes
// this path only after checking, from the caller's tables, that every
// coefficient's map equals its chain of doublings on all sixteen basis
// symbols (both are GF(2)-linear, so they then agree on every symbol).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));

// Scalar doubling, for the check: x * 2 with reduction word `red`.
__host__ __device__ __forceinline__ uint16_t gf16_dbl(uint16_t x, uint16_t red) {
    return uint16_t((x << 1) ^ ((x & 0x8000u) ? red : 0u));
}

// Two packed words times 2; red2 holds the reduction word in both halves.
__device__ __forceinline__ uint32_t gf16_dbl2(uint32_t x, uint32_t red2) {
    const uint32_t sh = __builtin_bit_cast(uint32_t, u16x2(__builtin_bit_cast(u16x2, x) << 1));
    const uint32_t top = __builtin_bit_cast(uint32_t, i16x2(__builtin_bit_cast(i16x2, x) >> 15));
    return __builtin_amdgcn_bitop3_b32(sh, top, red2, 0x78);   // sh ^ (top & red2)
}

// (x * 2) ^ y
__device__ __forceinline__ uint32_t gf16_dbl2_xor(uint32_t x, uint32_t red2, uint32_t y) {
    const uint32_t sh = __builtin_bit_cast(uint32_t, u16x2(__builtin_bit_cast(u16x2, x) << 1));
    const uint32_t top = __builtin_bit_cast(uint32_t, i16x2(__builtin_bit_cast(i16x2, x) >> 15));
    return xor3(sh, top & red2, y);
}

// acc[n][g] = acc[n][g] * alpha^(g+1) ^ x[n]; acc in natural word order.
template <int G, int NW>
__device__ __forceinline__ void rs_horner_step(uint32_t red2, const u32x4* x, uint32_t (*acc)[kRsGroup][4]) {
#pragma unroll
    for (int n = 0; n < NW; ++n) {
        const uint32_t xv[4] = {x[n].x, x[n].y, x[n].z, x[n].w};
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t a = acc[n][g][q];
#pragma unroll
                for (int d = 0; d < g; ++d) a = gf16_dbl2(a, red2);
                acc[n][g][q] = gf16_dbl2_xor(a, red2, xv[q]);
            }
    }
}

template <int G, int NW>
__device__ __forceinline__ void rs_horner_first(const u32x4* x, uint32_t (*acc)[kRsGroup][4]) {
#pragma unroll
    for (int n = 0; n < NW; ++n)
#pragma unroll
        for (int g = 0; g < G; ++g) {
            acc[n][g][0] = x[n].x;
            acc[n][g][1] = x[n].y;
            acc[n][g][2] = x[n].z;
            acc[n][g][3] = x[n].w;
        }
}

// rs_mix_full with Horner's order: the last input first, the input before in
// flight while one is folded in.  (Two inputs in flight measured the same.)
template <int G, int NW>
__device__ __forceinline__ void rs_horner_full(const RsJob& j, uint32_t red2, uint64_t t0b, bool copy,
                                               uint32_t (*acc)[kRsGroup][4]) {
    const int nin = j.nin;
    u32x4 lo[NW], hi[NW];
    RowWin rw = row_win(reinterpret_cast<const uint8_t*>(j.in_rows[nin - 1]) + t0b);
#pragma unroll
    for (int n = 0; n < NW; ++n) win_chunks(rw, 16 * (threadIdx.x + n * kTB), lo[n], hi[n]);
    for (int i = nin - 1; i >= 0; --i) {
        u32x4 x[NW];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            x[n] = win_join(rw, lo[n], hi[n]);
            if (copy) copy_owned<false>(j.copy, rw, 16 * (threadIdx.x + n * kTB), lo[n], hi[n]);
        }
        if (i > 0) {
            rw = row_win(reinterpret_cast<const uint8_t*>(j.in_rows[i - 1]) + t0b);
#pragma unroll
            for (int n = 0; n < NW; ++n) win_chunks(rw, 16 * (threadIdx.x + n * kTB), lo[n], hi[n]);
        }
        if (i == nin - 1) rs_horner_first<G, NW>(x, acc);
        else rs_horner_step<G, NW>(red2, x, acc);
    }
}

// rs_mix_tail with Horner's order.
template <int G, int NW>
__device__ __forceinline__ void rs_horner_tail(const RsJob& j, uint32_t red2, uint64_t t0b, const int64_t* w0,
                                               bool copy, uint32_t (*acc)[kRsGroup][4]) {
    for (int i = j.nin - 1; i >= 0; --i) {
        const RowWin rw = row_win(reinterpret_cast<const uint8_t*>(j.in_rows[i]) + t0b);
        u32x4 x[NW];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            const uint32_t off = 16 * (threadIdx.x + n * kTB);
            if (w0[n] + 8 <= j.S) {
                u32x4 lo, hi;
                win_chunks(rw, off, lo, hi);
                x[n] = win_join(rw, lo, hi);
                if (copy) copy_owned<false>(j.copy, rw, off, lo, hi);
            } else {
                x[n] = rs_window(j.in_rows[i], w0[n], j.S);
                if (copy && w0[n] < j.S) {
                    const uint64_t o = uint64_t(reinterpret_cast<const uint8_t*>(j.in_rows[i] + w0[n]) -
                                                j.copy.src);
                    copy_bytes(j.copy, o, o + 2 * uint64_t(j.S - w0[n]));
                }
            }
        }
        if (i == j.nin - 1) rs_horner_first<G, NW>(x, acc);
        else rs_horner_step<G, NW>(red2, x, acc);
    }
}

constexpr int kRsNW = 2;                              // windows per thread
// Non-temporal stores of the encode's parity rows and the reconstruct's
// rebuilt rows, as measured on the 512 MiB stream: plain for the encode (whose
// data-row copy writes alongside; nt 1 % slower), nt for the reconstruct (2 %
// faster).
constexpr bool kRsEncNT = false, kRsRecNT = true;
constexpr uint32_t kRsTile = kTileBytes * kRsNW;      // logical bytes per row per tile
constexpr uint32_t kRsStage = kRsTile + 16;           // LDS staging row

// Stream every tile of the job through the tables already in LDS; `tile`
// holds kRsGroup staging rows of kRsStage bytes.  Window n of thread t covers
// logical bytes 16 (t + n kTB) .. +15 of the tile, so each window's loads are
// contiguous across the block.  HORNER selects the Horner encode (all
// outputs in one group, accumulators in natural word order; red2 holds the
// reduction word in both halves).  The two are separate loops: sharing one
// loop made the encode kernel spill registers.
template <bool HORNER, bool NT>
__device__ __forceinline__ void rs_run_tiles(const RsJob& j, const uint32_t (*ptab)[kRs16Tab],
                                             uint8_t* tile, uint32_t red2) {
    const uint64_t Sb = uint64_t(j.S) * 2;
    const uint64_t ntiles = (Sb + kRsTile - 1) / kRsTile;
    for (uint64_t tt = blockIdx.x; tt < ntiles; tt += gridDim.x) {
        const uint64_t t0b = tt * kRsTile;
        const uint32_t nbytes = uint32_t(Sb - t0b < uint64_t(kRsTile) ? Sb - t0b : kRsTile);
        int64_t w0[kRsNW];
#pragma unroll
        for (int n = 0; n < kRsNW; ++n) w0[n] = int64_t(t0b / 2) + 8 * (threadIdx.x + n * kTB);
        if (j.copy.dst && tt == 0 && threadIdx.x == 0)
            for (int i = 0; i < j.nin; ++i)
                copy_row_head(j.copy,
                              uint64_t(reinterpret_cast<const uint8_t*>(j.in_rows[i]) - j.copy.src), Sb);
        for (int og = 0; og < j.nout; og += kRsGroup) {
            const bool copy = j.copy.dst != nullptr && og == 0;
            const int G = j.nout - og < kRsGroup ? j.nout - og : kRsGroup;
            uint32_t acc[kRsNW][kRsGroup][4];
            static_assert(kRsGroup == 2, "one instantiation per group size");
            if (HORNER && nbytes == kRsTile) {
                if (G == 1) rs_horner_full<1, kRsNW>(j, red2, t0b, copy, acc);
                else rs_horner_full<2, kRsNW>(j, red2, t0b, copy, acc);
            } else if (HORNER && w0[0] < j.S) {
                if (G == 1) rs_horner_tail<1, kRsNW>(j, red2, t0b, w0, copy, acc);
                else rs_horner_tail<2, kRsNW>(j, red2, t0b, w0, copy, acc);
            } else if (HORNER) {
                for (int n = 0; n < kRsNW; ++n)
                    for (int g = 0; g < kRsGroup; ++g)
                        acc[n][g][0] = acc[n][g][1] = acc[n][g][2] = acc[n][g][3] = 0;
            } else if (nbytes == kRsTile) {
                if (G == 1) rs_mix_full<1, kRsNW>(j, ptab, og, t0b, copy, acc);
                else rs_mix_full<2, kRsNW>(j, ptab, og, t0b, copy, acc);
            } else if (w0[0] < j.S) {
                if (G == 1) rs_mix_tail<1, kRsNW>(j, ptab, og, t0b, w0, copy, acc);
                else rs_mix_tail<2, kRsNW>(j, ptab, og, t0b, w0, copy, acc);
            } else {
                for (int n = 0; n < kRsNW; ++n)
                    for (int g = 0; g < kRsGroup; ++g)
                        acc[n][g][0] = acc[n][g][1] = acc[n][g][2] = acc[n][g][3] = 0;
            }
            for (int g = 0; g < G; ++g)
                for (int n = 0; n < kRsNW; ++n)
                    *reinterpret_cast<u32x4*>(tile + g * kRsStage + 16 * (threadIdx.x + n * kTB)) =
                        HORNER ? u32x4{acc[n][g][0], acc[n][g][1], acc[n][g][2], acc[n][g][3]}
                               : join_bytes(acc[n][g]);
            __syncthreads();
            for (int g = 0; g < G; ++g)
                tile_store<NT>(reinterpret_cast<uint8_t*>(j.out_rows[og + g]) + t0b, tile + g * kRsStage,
                           nbytes);
            __syncthreads();
        }
    }
}

// benchmark/rs/kernel.cu:67-102 parity: Par_p = XOR_i D_i * alpha^((p+1) i mod 65535).
__global__ __launch_bounds__(kTB) __attribute__((amdgpu_waves_per_eu(4))) void rs16_encode_kernel(RsJob job, const uint16_t* ex,
                                                          const uint16_t* lg) {
    __shared__ __attribute__((aligned(16))) uint32_t ptab[kRsMaxTables][kRs16Tab];
    __shared__ uint16_t basis[kRsMaxTables][16];
    __shared__ uint16_t coef[kRsMaxTables];
    __shared__ __attribute__((aligned(16))) uint8_t tile[kRsGroup * kRsStage];
    __shared__ RsJob j;
    if (threadIdx.x == 0) j = job;
    __syncthreads();
    for (int t = threadIdx.x; t < j.nout * j.nin; t += kTB) {
        const int p = t / j.nin, i = t % j.nin;
        coef[t] = ex[((p + 1) * i) % kGfOrder];
    }
    __syncthreads();
    rs_build_perm_tables(ptab, basis, coef, j.nout * j.nin, ex, lg);
    // Horner's order when every basis product c(p, i) * 2^b the tables give
    // equals 2^b doubled (p + 1) i times, the reduction word being 0x8000 * 2
    // from the tables.
    __shared__ int s_horner;
    __shared__ uint16_t s_red;
    if (threadIdx.x == 0) {
        s_red = gf16_mul_tab(0x8000, 2, ex, lg);
        s_horner = j.nout <= kRsGroup;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < j.nout * j.nin * 16; e += kTB) {
        const int t = e >> 4, b = e & 15;
        const int p = t / j.nin, i = t % j.nin;
        uint16_t v = uint16_t(1u << b);
        for (int d = 0; d < (p + 1) * i; ++d) v = gf16_dbl(v, s_red);
        if (v != basis[t][b]) s_horner = 0;
    }
    __syncthreads();
    if (s_horner) rs_run_tiles<true, kRsEncNT>(j, ptab, tile, uint32_t(s_red) * 0x10001u);
    else rs_run_tiles<false, kRsEncNT>(j, ptab, tile, 0u);
}

// benchmark/rs/kernel.cu:105-222 with the right-hand side folded into the
// coefficients.  Inputs: the k - m surviving data rows, then the m parity rows
// of parity_used; outputs: the m missing data rows.
__global__ __launch_bounds__(kTB) __attribute__((amdgpu_waves_per_eu(4))) void rs16_reconstruct_kernel(uint16_t* sh, int64_t S, int k,
                                                               int mpar, int m,
                                                               const int32_t* missing,
                                                               const int32_t* pused,
                                                               const uint16_t* ex,
                                                               const uint16_t* lg) {
    __shared__ __attribute__((aligned(16))) uint32_t ptab[kRsMaxTables][kRs16Tab];
    __shared__ uint16_t basis[kRsMaxTables][16];
    __shared__ uint16_t coef[kRsMaxTables];
    __shared__ uint16_t inv[kRsMaxM * kRsMaxM];
    __shared__ int s_miss[kRsMaxM], s_pu[kRsMaxM];
    __shared__ int s_ok;
    __shared__ __attribute__((aligned(16))) uint8_t tile[kRsGroup * kRsStage];
    __shared__ RsJob j;
    if (threadIdx.x < m) {
        s_miss[threadIdx.x] = missing[threadIdx.x];
        s_pu[threadIdx.x] = pused[threadIdx.x];
    }
    __syncthreads();
    // Indices come from device memory: a row outside the tensor would be an
    // out-of-bounds write, and repeated indices would overflow the LDS tables,
    // so either makes the call write nothing.
    if (threadIdx.x == 0) {
        int ok = 1;
        for (int q = 0; q < m; ++q) {
            ok &= (s_miss[q] >= 0 && s_miss[q] < k && s_pu[q] >= 0 && s_pu[q] < mpar);
            for (int q2 = 0; q2 < q; ++q2) ok &= (s_miss[q2] != s_miss[q]);
        }
        s_ok = ok;
    }
    __syncthreads();
    if (!s_ok) return;
    if (threadIdx.x == 0) {
        uint16_t V[kRsMaxM * kRsMaxM];
        for (int r = 0; r < m; ++r)
            for (int c = 0; c < m; ++c) V[r * m + c] = ex[((s_pu[r] + 1) * s_miss[c]) % kGfOrder];
        for (int r = 0; r < m; ++r)
            for (int c = 0; c < m; ++c) inv[r * m + c] = (r == c) ? 1 : 0;
        for (int i = 0; i < m; ++i) {
            int pr = i;
            while (pr < m && V[pr * m + i] == 0) ++pr;
            if (pr == m) continue;
            if (pr != i)
                for (int c = 0; c < m; ++c) {
                    uint16_t t = V[i * m + c];
                    V[i * m + c] = V[pr * m + c];
                    V[pr * m + c] = t;
                    t = inv[i * m + c];
                    inv[i * m + c] = inv[pr * m + c];
                    inv[pr * m + c] = t;
                }
            const uint16_t piv = V[i * m + i];
            if (piv == 0) continue;
            const uint16_t ip = gf16_div_tab(1, piv, ex, lg);
            for (int c = 0; c < m; ++c) {
                V[i * m + c] = gf16_mul_tab(V[i * m + c], ip, ex, lg);
                inv[i * m + c] = gf16_mul_tab(inv[i * m + c], ip, ex, lg);
            }
            for (int r = 0; r < m; ++r) {
                if (r == i) continue;
                const uint16_t f = V[r * m + i];
                if (!f) continue;
                for (int c = 0; c < m; ++c) {
                    V[r * m + c] ^= gf16_mul_tab(f, V[i * m + c], ex, lg);
                    inv[r * m + c] ^= gf16_mul_tab(f, inv[i * m + c], ex, lg);
                }
            }
        }
    }
    __syncthreads();
    // inputs: surviving data rows in index order, then the used parity rows
    if (threadIdx.x == 0) {
        j.S = S;
        j.nout = m;
        j.copy = FlatCopy{nullptr, nullptr, 0};
        int n = 0;
        for (int i = 0; i < k; ++i) {
            bool miss = false;
            for (int q = 0; q < m; ++q) miss |= (s_miss[q] == i);
            if (!miss && n < kRsMaxTables) j.in_rows[n++] = sh + uint64_t(i) * S;
        }
        for (int r = 0; r < m && n < kRsMaxTables; ++r) j.in_rows[n++] = sh + uint64_t(k + s_pu[r]) * S;
        j.nin = n;
        for (int c = 0; c < m; ++c) j.out_rows[c] = sh + uint64_t(s_miss[c]) * S;
    }
    __syncthreads();
    const int nin = j.nin, ndata = nin - m;
    // coefficient of input `in` for output c
    for (int t = threadIdx.x; t < m * nin; t += kTB) {
        const int c = t / nin, in = t % nin;
        uint16_t v = 0;
        if (in < ndata) {
            int i = 0, seen = -1;
            for (; i < k; ++i) {
                bool miss = false;
                for (int q = 0; q < m; ++q) miss |= (s_miss[q] == i);
                if (!miss && ++seen == in) break;
            }
            for (int r = 0; r < m; ++r)
                v ^= gf16_mul_tab(inv[c * m + r], ex[((s_pu[r] + 1) * i) % kGfOrder], ex, lg);
        } else {
            v = inv[c * m + (in - ndata)];
        }
        coef[t] = v;
    }
    __syncthreads();
    rs_build_perm_tables(ptab, basis, coef, m * nin, ex, lg);
    __syncthreads();
    rs_run_tiles<false, kRsRecNT>(j, ptab, tile, 0u);
}

static int rs_grid(int64_t S) {
    const int64_t tiles = (S * 2 + kRsTile - 1) / kRsTile;
    return int(tiles < kRsGrid ? tiles : kRsGrid);
}

}  // namespace kvec

using namespace kvec;

// pack_fp16_pair_to_u16, benchmark/rs/kernel.cu:225-243: out = K words || V words.
extern "C" int kvec_rs16_pack(const void* k, const void* v, void* out, int64_t N_k, int64_t N_v,
                              void* stream) {
    if (N_k < 0 || N_v < 0) return set_error(KVEC_EINVAL, "kvec_rs16_pack: negative size");
    if ((N_k && (!k || !out)) || (N_v && (!v || !out)))
        return set_error(KVEC_EINVAL, "kvec_rs16_pack: null pointer");
    hipStream_t st = as_stream(stream);
    int rc = copy_d2d(out, k, uint64_t(N_k) * 2, st, "kvec_rs16_pack");
    if (rc) return rc;
    return copy_d2d((uint16_t*)out + N_k, v, uint64_t(N_v) * 2, st, "kvec_rs16_pack");
}

// u16_to_fp16_split, benchmark/rs/kernel.cu:245-263: inverse of the pack.
extern "C" int kvec_rs16_split(const void* in, void* k_out, void* v_out, int64_t N_k, int64_t N_v,
                               void* stream) {
    if (N_k < 0 || N_v < 0) return set_error(KVEC_EINVAL, "kvec_rs16_split: negative size");
    if ((N_k && (!in || !k_out)) || (N_v && (!in || !v_out)))
        return set_error(KVEC_EINVAL, "kvec_rs16_split: null pointer");
    hipStream_t st = as_stream(stream);
    int rc = copy_d2d(k_out, in, uint64_t(N_k) * 2, st, "kvec_rs16_split");
    if (rc) return rc;
    return copy_d2d(v_out, (const uint16_t*)in + N_k, uint64_t(N_v) * 2, st, "kvec_rs16_split");
}

// encode_rs_u16, benchmark/rs/kernel.cu:265-285: copy the data rows, then the
// parity rows.  gf_exp / gf_log are the device tables of init_gf_tables().
extern "C" int kvec_rs16_encode(const void* data_padded, void* shards, int data_shards,
                                int parity_shards, int shard_size, const uint16_t* gf_exp,
                                const uint16_t* gf_log, void* stream) {
    if (!data_padded || !shards || !gf_exp || !gf_log)
        return set_error(KVEC_EINVAL, "kvec_rs16_encode: null pointer");
    if (data_shards < 1 || parity_shards < 0 || shard_size < 0)
        return set_error(KVEC_EINVAL, "kvec_rs16_encode: k=%d m=%d S=%d", data_shards, parity_shards,
                         shard_size);
    if (parity_shards > kRsMaxM || data_shards * parity_shards > kRsMaxTables)
        return set_error(KVEC_EUNSUPPORTED, "kvec_rs16_encode: k*m=%d exceeds %d (m <= %d)",
                         data_shards * parity_shards, kRsMaxTables, kRsMaxM);
    hipStream_t st = as_stream(stream);
    const int64_t S = shard_size;
    if (S == 0) return KVEC_OK;
    const uint64_t data_bytes = uint64_t(data_shards) * S * 2;
    // The data rows are copied by the coding kernel itself when the two
    // buffers are disjoint and equally aligned modulo 16 bytes; otherwise (or
    // with no parity to code) by a separate stream-ordered copy.  The data
    // must not overlap the parity rows the kernel writes, nor the data rows
    // unless it is them (a partial overlap has no stream-ordered meaning).
    if (ranges_overlap(data_padded, data_bytes, (uint16_t*)shards + uint64_t(data_shards) * S,
                       uint64_t(parity_shards) * S * 2))
        return set_error(KVEC_EINVAL, "kvec_rs16_encode: data overlaps the parity rows");
    const bool fuse = parity_shards > 0 && fused_copy_ok(data_padded, shards, data_bytes);
    if (!fuse) {
        int rc = copy_d2d(shards, data_padded, data_bytes, st, "kvec_rs16_encode");
        if (rc) return rc;
    }
    if (parity_shards == 0) return KVEC_OK;
    RsJob j{};
    j.copy = fuse ? FlatCopy{(const uint8_t*)data_padded, (uint8_t*)shards, data_bytes}
                  : FlatCopy{nullptr, nullptr, 0};
    j.S = S;
    j.nin = data_shards;
    j.nout = parity_shards;
    for (int i = 0; i < data_shards; ++i) j.in_rows[i] = (const uint16_t*)data_padded + uint64_t(i) * S;
    for (int p = 0; p < parity_shards; ++p)
        j.out_rows[p] = (uint16_t*)shards + uint64_t(data_shards + p) * S;
    hipLaunchKernelGGL(rs16_encode_kernel, dim3(rs_grid(S)), dim3(kTB), 0, st, j, gf_exp, gf_log);
    return check_launch("kvec_rs16_encode");
}

// reconstruct_rs_u16_inplace, benchmark/rs/kernel.cu:287-312.  missing_data and
// parity_used are device int32 arrays of `m` entries (as the reference reads
// them); only data rows are rebuilt.  Out-of-range or repeated missing indices
// make the kernel write nothing (the reference would write outside the tensor,
// or solve a singular system).
extern "C" int kvec_rs16_reconstruct(void* shards, int shard_size, int data_shards,
                                     int parity_shards, const int32_t* missing_data, int m,
                                     const int32_t* parity_used, const uint16_t* gf_exp,
                                     const uint16_t* gf_log, void* stream) {
    (void)parity_shards;
    if (m == 0) return KVEC_OK;
    if (m < 0 || m > kRsMaxM)
        return set_error(KVEC_EINVAL, "kvec_rs16_reconstruct: m=%d (must be <= %d)", m, kRsMaxM);
    if (!shards || !missing_data || !parity_used || !gf_exp || !gf_log)
        return set_error(KVEC_EINVAL, "kvec_rs16_reconstruct: null pointer");
    if (data_shards < m || parity_shards < m || shard_size < 0)
        return set_error(KVEC_EINVAL, "kvec_rs16_reconstruct: k=%d parity=%d m=%d S=%d", data_shards,
                         parity_shards, m, shard_size);
    if (data_shards * m > kRsMaxTables)
        return set_error(KVEC_EUNSUPPORTED, "kvec_rs16_reconstruct: k*m=%d exceeds %d",
                         data_shards * m, kRsMaxTables);
    if (shard_size == 0) return KVEC_OK;
    hipLaunchKernelGGL(rs16_reconstruct_kernel, dim3(rs_grid(shard_size)), dim3(kTB), 0,
                       as_stream(stream), (uint16_t*)shards, int64_t(shard_size), data_shards,
                       parity_shards, m, missing_data, parity_used, gf_exp, gf_log);
    return check_launch("kvec_rs16_reconstruct");
}

// GF(2^16) tables of benchmark/rs/main.py:39-54 (poly 0x1100B), host memory:
// gf_exp has 2*65535 entries, gf_log 65536.
extern "C" int kvec_gf16_tables(uint16_t* gf_exp, uint16_t* gf_log) {
    if (!gf_exp || !gf_log) return set_error(KVEC_EINVAL, "kvec_gf16_tables: null pointer");
    for (int i = 0; i < 65536; ++i) gf_log[i] = 0;
    uint32_t x = 1;
    for (int i = 0; i < kGfOrder; ++i) {
        gf_exp[i] = uint16_t(x);
        gf_log[x] = uint16_t(i);
        x <<= 1;
        if (x & 0x10000u) x ^= 0x1100Bu;
    }
    for (int i = 0; i < kGfOrder; ++i) gf_exp[kGfOrder + i] = gf_exp[i];
    return KVEC_OK;
}
