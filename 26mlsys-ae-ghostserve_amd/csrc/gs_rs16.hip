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
#include "piece_walk.h"

namespace kvec {

constexpr int kGfOrder = 65535;
constexpr int kRsMaxM = 16;           // reference limit (benchmark/rs/kernel.cu:118)
constexpr int kRsMaxTables = 48;      // coefficients held in LDS
constexpr int kRs16Tab = 24;          // dwords per coefficient: 4 byte maps x 6
constexpr int kRsGroup = 2;           // outputs accumulated per pass over the inputs
// The persistent tile kernels (the encode and the reconstruct for shapes the
// one-shot tile kernels and the piece kernel do not take) run blocks of kRsBS
// threads, two per CU: the tables are built once per block.  Measured on the 512 MiB stream, RS(6,2) encode: 512
// threads (16 KiB tiles) with 512 blocks 245 against 248 us for 256 threads
// with 1024 blocks, and with the XCD-grouped tile order of rs_run_tiles 239 us.
constexpr int kRsBS = 512;
constexpr int kRsGrid = 512;

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

// Table word i (0 <= i < 131069) by a scalar load of the dword holding it,
// through the constant address space: the tables do not change during a
// launch, and the scalar cache answers a block's read of the generator in a
// fraction of a vector load's round trip, which a block otherwise waits for
// before issuing its data loads.  The dword read starts at an even word of
// the 2-byte-aligned table, so it never leaves the table.
__device__ __forceinline__ uint32_t table_word_s(const uint16_t* tab, uint32_t i) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(tab + i);
    const uintptr_t d = a & ~uintptr_t(3);
    const uint32_t w = *reinterpret_cast<const __attribute__((address_space(4))) uint32_t*>(d);
    return (a & 2) ? (w >> 16) : (w & 0xFFFFu);
}

// The rule by which every GF(2^16) kernel here chooses Horner's rule (each
// multiplication by 2 a shift and an XOR of the reduction word) over the byte
// maps: the tables' generator is 2 (gf_exp[1] == 2), and the reduction word is
// gf_exp[16] = 2^16 in the field.  For any field's exp/log pair with generator
// 2 this is exactly the tables' multiplication, so both ways give the same
// bytes; and since every kernel applies the same test, the kernel that serves a
// call's shape never decides which way its bytes are computed.
__device__ __forceinline__ bool horner_tables(const uint16_t* ex) { return table_word_s(ex, 1) == 2; }
__device__ __forceinline__ uint32_t horner_red2(const uint16_t* ex) { return table_word_s(ex, 16) * 0x10001u; }

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
// The maps are built from basis[t][b] = coefficient t times 2^b, which the
// caller has made visible to the threads that call it: dwords first,
// first + stride, ... of the ncoef * kRs16Tab.
__device__ __forceinline__ void rs_maps_from_basis(uint32_t (*ptab)[kRs16Tab], const uint16_t (*basis)[16],
                                                   int ncoef, int first, int stride) {
    for (int e = first; e < ncoef * kRs16Tab; e += stride) {
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

// Byte maps of the coefficients coef[0 .. ncoef), their basis products read
// from the tables (all threads).  The maps loop is written out here rather
// than calling rs_maps_from_basis: the piece kernel compiled through the call
// ran its two-row reconstruct in 165 instead of 151 us.
__device__ __forceinline__ void rs_build_perm_tables(uint32_t (*ptab)[kRs16Tab], uint16_t (*basis)[16],
                                                     const uint16_t* coef, int ncoef, const uint16_t* ex,
                                                     const uint16_t* lg) {
    for (int e = threadIdx.x; e < ncoef * 16; e += blockDim.x)
        basis[e >> 4][e & 15] = gf16_mul_tab(uint16_t(1u << (e & 15)), coef[e >> 4], ex, lg);
    __syncthreads();
    for (int e = threadIdx.x; e < ncoef * kRs16Tab; e += blockDim.x) {
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
    for (int n = 0; n < NW; ++n) win_chunks(rw, 16 * (threadIdx.x + n * kRsBS), lo[n], hi[n]);
    for (int i = 0; i < nin; ++i) {
        u32x4 x[NW];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            x[n] = win_join(rw, lo[n], hi[n]);
            if (copy) copy_owned<false>(j.copy, rw, 16 * (threadIdx.x + n * kRsBS), lo[n], hi[n]);
        }
        if (i + 1 < nin) {
            rw = row_win(reinterpret_cast<const uint8_t*>(j.in_rows[i + 1]) + t0b);
#pragma unroll
            for (int n = 0; n < NW; ++n) win_chunks(rw, 16 * (threadIdx.x + n * kRsBS), lo[n], hi[n]);
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
            const uint32_t off = 16 * (threadIdx.x + n * kRsBS);
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

// Times 4 in one step: a word v = t * 2^14 + low is v * 4 = (low << 2) ^ T[t]
// with T[t] = t * 2^16 reduced, t the two bits shifted out.  T fits the eight
// bytes one v_perm_b32 indexes: lo = T[0] | T[1] << 16, hi = T[2] | T[3] << 16,
// with T[1] = 2^16 reduced (the reduction word) and T[2] = 2^17 reduced (its
// double, reduced again when its top bit is set).
struct Gf16Quad {
    uint32_t lo, hi;
};
__host__ __device__ __forceinline__ Gf16Quad gf16_quad_table(uint16_t red) {
    const uint16_t r2 = gf16_dbl(red, red);
    return Gf16Quad{uint32_t(red) << 16, uint32_t(r2) | (uint32_t(uint16_t(red ^ r2)) << 16)};
}

// (x * 4) ^ y for two packed words: shift, the two top bits' byte selectors
// (2t, 2t + 1) by one packed multiply-add, the table lookup and a 3-input XOR
// (five VALU ops; two doublings and the XOR take seven).
__device__ __forceinline__ uint32_t gf16_quad2_xor(uint32_t x, Gf16Quad q, uint32_t y) {
    const u16x2 v = __builtin_bit_cast(u16x2, x);
    const uint32_t sh = __builtin_bit_cast(uint32_t, u16x2(v << 2));
    const u16x2 t = v >> 14;
    const uint32_t sel = __builtin_bit_cast(uint32_t, u16x2(t * u16x2{0x0202, 0x0202} + u16x2{0x0100, 0x0100}));
    return xor3(sh, __builtin_amdgcn_perm(q.hi, q.lo, sel), y);
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
    for (int n = 0; n < NW; ++n) win_chunks(rw, 16 * (threadIdx.x + n * kRsBS), lo[n], hi[n]);
    for (int i = nin - 1; i >= 0; --i) {
        u32x4 x[NW];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            x[n] = win_join(rw, lo[n], hi[n]);
            if (copy) copy_owned<false>(j.copy, rw, 16 * (threadIdx.x + n * kRsBS), lo[n], hi[n]);
        }
        if (i > 0) {
            rw = row_win(reinterpret_cast<const uint8_t*>(j.in_rows[i - 1]) + t0b);
#pragma unroll
            for (int n = 0; n < NW; ++n) win_chunks(rw, 16 * (threadIdx.x + n * kRsBS), lo[n], hi[n]);
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
            const uint32_t off = 16 * (threadIdx.x + n * kRsBS);
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
constexpr uint32_t kRsTile = 16 * kRsBS * kRsNW;     // logical bytes per row per tile
constexpr uint32_t kRsStage = kRsTile + 16;           // LDS staging row

// Stream every tile of the job through the tables already in LDS; `tile`
// holds kRsGroup staging rows of kRsStage bytes.  Window n of thread t covers
// logical bytes 16 (t + n kRsBS) .. +15 of the tile, so each window's loads
// are contiguous across the block.  HORNER selects the Horner encode (all
// outputs in one group, accumulators in natural word order; red2 holds the
// reduction word in both halves).  The two are separate loops: sharing one
// loop made the encode kernel spill registers.
//
// Tile order: blocks are dispatched round-robin over the eight XCDs (block b
// on XCD b % 8), and the blocks of one XCD take consecutive tiles, so the
// 128-byte lines that two neighbouring tiles of a misaligned row share are
// mostly written through one XCD's L2.
template <bool HORNER, bool NT>
__device__ __forceinline__ void rs_run_tiles(const RsJob& j, const uint32_t (*ptab)[kRs16Tab],
                                             uint8_t* tile, uint32_t red2) {
    const uint64_t Sb = uint64_t(j.S) * 2;
    const uint64_t ntiles = (Sb + kRsTile - 1) / kRsTile;
    // each row's head bytes up to its first 16-byte-aligned address, which no
    // tile's aligned chunks cover: one lane per byte
    if (j.copy.dst && blockIdx.x == 0)
        for (int e = threadIdx.x; e < 16 * j.nin; e += kRsBS) {
            const uint64_t o = uint64_t(reinterpret_cast<const uint8_t*>(j.in_rows[e >> 4]) - j.copy.src);
            const uint32_t mis = uint32_t(reinterpret_cast<uintptr_t>(j.copy.src + o) & 15);
            const uint32_t b = uint32_t(e & 15);
            if (mis && b < 16 - mis && b < Sb) as_global(j.copy.dst)[o + b] = as_global(j.copy.src)[o + b];
        }
    const uint32_t G = gridDim.x;
    const uint32_t first = G % 8 == 0 ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    for (uint64_t tt = first; tt < ntiles; tt += G) {
        const uint64_t t0b = tt * kRsTile;
        const uint32_t nbytes = uint32_t(Sb - t0b < uint64_t(kRsTile) ? Sb - t0b : kRsTile);
        int64_t w0[kRsNW];
#pragma unroll
        for (int n = 0; n < kRsNW; ++n) w0[n] = int64_t(t0b / 2) + 8 * (threadIdx.x + n * kRsBS);
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
                    *reinterpret_cast<u32x4*>(tile + g * kRsStage + 16 * (threadIdx.x + n * kRsBS)) =
                        HORNER ? u32x4{acc[n][g][0], acc[n][g][1], acc[n][g][2], acc[n][g][3]}
                               : join_bytes(acc[n][g]);
            __syncthreads();
            for (int g = 0; g < G; ++g)
                tile_store<NT, kRsBS>(reinterpret_cast<uint8_t*>(j.out_rows[og + g]) + t0b, tile + g * kRsStage,
                                      nbytes);
            __syncthreads();
        }
    }
}

// benchmark/rs/kernel.cu:67-102 parity: Par_p = XOR_i D_i * alpha^((p+1) i mod 65535).
__global__ __launch_bounds__(kRsBS) __attribute__((amdgpu_waves_per_eu(4))) void rs16_encode_kernel(RsJob job, const uint16_t* ex,
                                                          const uint16_t* lg) {
    __shared__ __attribute__((aligned(16))) uint32_t ptab[kRsMaxTables][kRs16Tab];
    __shared__ uint16_t basis[kRsMaxTables][16];
    __shared__ uint16_t coef[kRsMaxTables];
    __shared__ __attribute__((aligned(16))) uint8_t tile[kRsGroup * kRsStage];
    __shared__ RsJob j;
    if (threadIdx.x == 0) j = job;
    __syncthreads();
    for (int t = threadIdx.x; t < j.nout * j.nin; t += kRsBS) {
        const int p = t / j.nin, i = t % j.nin;
        coef[t] = ex[((p + 1) * i) % kGfOrder];
    }
    __syncthreads();
    rs_build_perm_tables(ptab, basis, coef, j.nout * j.nin, ex, lg);
    __syncthreads();   // the maps, written by every thread, before any use
    // Horner's order by horner_tables (up to kRsGroup parities)
    if (j.nout <= kRsGroup && horner_tables(ex)) rs_run_tiles<true, kRsEncNT>(j, ptab, tile, horner_red2(ex));
    else rs_run_tiles<false, kRsEncNT>(j, ptab, tile, 0u);
}

// The reconstruct's plan, shared by its kernels: which rows are inputs and
// outputs, and one coefficient per (output, input) pair.
//   inputs  the k - m surviving data rows in index order, then the m parity
//           rows of parity_used;
//   outputs the m missing data rows.
// benchmark/rs/kernel.cu:105-222 computes the right-hand side b (parity row
// XOR the known data terms) and then x = V^-1 b; folding the two steps into
// one coefficient per pair is exact in the field, so the bytes are those of
// the two-step computation.
struct RsRecPlan {
    int miss[kRsMaxM], pu[kRsMaxM];
    int in_row[kRsMaxTables];       // input i is row in_row[i] of the shard tensor
    int nin;
    int ok;
    uint16_t inv[kRsMaxM * kRsMaxM];
    uint16_t coef[kRsMaxTables];    // coefficient of input i for output c at [c * nin + i]
    uint16_t basis[kRsMaxTables][16];
};

// First phase (all threads; ends with a barrier): the indices, read from
// device memory, and the input rows.  A row index outside the tensor would be
// an out-of-bounds write, and repeated indices would overflow the LDS tables,
// so either leaves pl.ok = 0 and the call writes nothing.
__device__ __forceinline__ void rs16_rec_rows(RsRecPlan& pl, int k, int mpar, int m, const int32_t* missing,
                                              const int32_t* pused) {
    if (threadIdx.x < m) {
        pl.miss[threadIdx.x] = missing[threadIdx.x];
        pl.pu[threadIdx.x] = pused[threadIdx.x];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int ok = 1;
        for (int q = 0; q < m; ++q) {
            ok &= (pl.miss[q] >= 0 && pl.miss[q] < k && pl.pu[q] >= 0 && pl.pu[q] < mpar);
            for (int q2 = 0; q2 < q; ++q2) ok &= (pl.miss[q2] != pl.miss[q]);
        }
        pl.ok = ok;
        int n = 0;
        for (int i = 0; i < k; ++i) {
            bool miss = false;
            for (int q = 0; q < m; ++q) miss |= (pl.miss[q] == i);
            if (!miss && n < kRsMaxTables) pl.in_row[n++] = i;
        }
        for (int r = 0; r < m && n < kRsMaxTables; ++r) pl.in_row[n++] = k + pl.pu[r];
        pl.nin = n;
    }
    __syncthreads();
}

// Second phase (all threads, pl.ok set; ends with a barrier): the inverse of
// V[r][c] = alpha^((pu_r + 1) miss_c) by the reference's Gauss-Jordan (pivot
// order and zero-pivot skip included), the folded coefficients and their
// v_perm byte maps.
__device__ __forceinline__ void rs16_rec_tables(RsRecPlan& pl, uint32_t (*ptab)[kRs16Tab], int k, int m,
                                                const uint16_t* ex, const uint16_t* lg) {
    if (threadIdx.x == 0) {
        uint16_t V[kRsMaxM * kRsMaxM];
        for (int r = 0; r < m; ++r)
            for (int c = 0; c < m; ++c) V[r * m + c] = ex[((pl.pu[r] + 1) * pl.miss[c]) % kGfOrder];
        for (int r = 0; r < m; ++r)
            for (int c = 0; c < m; ++c) pl.inv[r * m + c] = (r == c) ? 1 : 0;
        for (int i = 0; i < m; ++i) {
            int pr = i;
            while (pr < m && V[pr * m + i] == 0) ++pr;
            if (pr == m) continue;
            if (pr != i)
                for (int c = 0; c < m; ++c) {
                    uint16_t t = V[i * m + c];
                    V[i * m + c] = V[pr * m + c];
                    V[pr * m + c] = t;
                    t = pl.inv[i * m + c];
                    pl.inv[i * m + c] = pl.inv[pr * m + c];
                    pl.inv[pr * m + c] = t;
                }
            const uint16_t piv = V[i * m + i];
            if (piv == 0) continue;
            const uint16_t ip = gf16_div_tab(1, piv, ex, lg);
            for (int c = 0; c < m; ++c) {
                V[i * m + c] = gf16_mul_tab(V[i * m + c], ip, ex, lg);
                pl.inv[i * m + c] = gf16_mul_tab(pl.inv[i * m + c], ip, ex, lg);
            }
            for (int r = 0; r < m; ++r) {
                if (r == i) continue;
                const uint16_t f = V[r * m + i];
                if (!f) continue;
                for (int c = 0; c < m; ++c) {
                    V[r * m + c] ^= gf16_mul_tab(f, V[i * m + c], ex, lg);
                    pl.inv[r * m + c] ^= gf16_mul_tab(f, pl.inv[i * m + c], ex, lg);
                }
            }
        }
    }
    __syncthreads();
    const int nin = pl.nin, ndata = nin - m;
    for (int t = threadIdx.x; t < m * nin; t += blockDim.x) {
        const int c = t / nin, in = t % nin;
        uint16_t v = 0;
        if (in < ndata) {
            const int i = pl.in_row[in];
            for (int r = 0; r < m; ++r)
                v ^= gf16_mul_tab(pl.inv[c * m + r], ex[((pl.pu[r] + 1) * i) % kGfOrder], ex, lg);
        } else {
            v = pl.inv[c * m + (in - ndata)];
        }
        pl.coef[t] = v;
    }
    __syncthreads();
    rs_build_perm_tables(ptab, pl.basis, pl.coef, m * nin, ex, lg);
    __syncthreads();
}

// benchmark/rs/kernel.cu:105-222, tile engine: any k, m and row size.
__global__ __launch_bounds__(kRsBS) __attribute__((amdgpu_waves_per_eu(4))) void rs16_reconstruct_kernel(uint16_t* sh, int64_t S, int k,
                                                               int mpar, int m,
                                                               const int32_t* missing,
                                                               const int32_t* pused,
                                                               const uint16_t* ex,
                                                               const uint16_t* lg) {
    __shared__ __attribute__((aligned(16))) uint32_t ptab[kRsMaxTables][kRs16Tab];
    __shared__ RsRecPlan pl;
    __shared__ __attribute__((aligned(16))) uint8_t tile[kRsGroup * kRsStage];
    __shared__ RsJob j;
    rs16_rec_rows(pl, k, mpar, m, missing, pused);
    if (!pl.ok) return;
    rs16_rec_tables(pl, ptab, k, m, ex, lg);
    if (threadIdx.x == 0) {
        j.S = S;
        j.nout = m;
        j.copy = FlatCopy{nullptr, nullptr, 0};
        j.nin = pl.nin;
        for (int i = 0; i < pl.nin; ++i) j.in_rows[i] = sh + uint64_t(pl.in_row[i]) * S;
        for (int c = 0; c < m; ++c) j.out_rows[c] = sh + uint64_t(pl.miss[c]) * S;
    }
    __syncthreads();
    rs_run_tiles<false, kRsRecNT>(j, ptab, tile, 0u);
}

// ------------------------------------------------------------ piece kernel
// The reconstruct on the piece engine (piece_walk.h): waves walk pieces of
// 64 windows of every row, loaded and stored at the rows' own alignment,
// every input row's window of a piece requested at once and the next piece's
// requested before the current one is coded; no LDS tiles and no block
// barriers.  For up to kRsPieceMaxIn inputs, up to kRsGroup outputs and
// tensors of fewer than 2^31 bytes; rows of at least one tile take the
// one-shot tile reconstruct below instead.  Measured on the 512 MiB stream
// against the persistent tile kernel (same box): the reconstruct of 2 rows 165
// against 168-196 us with the folded byte maps, 149.6 us with the syndromes by
// Horner's rule below; the encode on pieces took 279-304 against 245-255 us
// (with aligned or misaligned data-row stores alike), so the encode stays on
// the tiles.
constexpr int kRsPieceMaxIn = 8;
constexpr uint32_t kRsPieceBlocks = 1024;   // persistent: the tables are built once per block

// Outputs of one piece by the byte maps: out[g] = XOR_i c(g, i) * x_i, the
// coefficient of input i for output g at ptab[g * NIN + i].  One
// coefficient's byte maps (24 dwords) and one input's fields are live at a
// time: the LDS reads stay next to their use (memory clobber) and no product
// moves to another coefficient (scheduling barrier).  Without the fences the
// compiler reads every map of an input at once and spills.
template <int NIN, int M>
__device__ __forceinline__ void rs_piece_mix(const u32x4* x, const uint32_t (*ptab)[kRs16Tab], u32x4* out) {
    uint32_t acc[M][4];
#pragma unroll
    for (int g = 0; g < M; ++g) acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0;
#pragma unroll
    for (int i = 0; i < NIN; ++i) {
        uint32_t by[4];
        split_bytes(x[i], by);
        Gf8Fields f[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) f[q] = gf8_fields(by[q]);
#pragma unroll
        for (int g = 0; g < M; ++g) {
            const uint32_t* T = ptab[g * NIN + i];
            acc[g][0] = gf16_fma2(acc[g][0], f[0], T + 0, f[1], T + 6);
            acc[g][1] = gf16_fma2(acc[g][1], f[0], T + 12, f[1], T + 18);
            acc[g][2] = gf16_fma2(acc[g][2], f[2], T + 0, f[3], T + 6);
            acc[g][3] = gf16_fma2(acc[g][3], f[2], T + 12, f[3], T + 18);
            // the accumulators pass through the asm, so the products are
            // computed here rather than sunk towards the final join
            asm volatile("" : "+v"(acc[g][0]), "+v"(acc[g][1]), "+v"(acc[g][2]), "+v"(acc[g][3]) :: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int g = 0; g < M; ++g) out[g] = join_bytes(acc[g]);
}

// Wave-uniform copy of an LDS int.
__device__ __forceinline__ uint32_t lds_uniform(const int& v) {
    return uint32_t(__builtin_amdgcn_readfirstlane(v));
}

// Multiply four packed word pairs by alpha^n (n doublings; n is wave-uniform).
__device__ __forceinline__ u32x4 gf16_dbl_n(u32x4 v, uint32_t n, uint32_t red2) {
    for (uint32_t t = 0; t < n; ++t)
        v = u32x4{gf16_dbl2(v.x, red2), gf16_dbl2(v.y, red2), gf16_dbl2(v.z, red2), gf16_dbl2(v.w, red2)};
    return v;
}

// The same product by n / 2 steps of gf16_quad2_xor and, for odd n, one doubling.
__device__ __forceinline__ u32x4 gf16_dbl_n(u32x4 v, uint32_t n, uint32_t red2, Gf16Quad q) {
    for (; n >= 2; n -= 2)
        v = u32x4{gf16_quad2_xor(v.x, q, 0u), gf16_quad2_xor(v.y, q, 0u), gf16_quad2_xor(v.z, q, 0u),
                  gf16_quad2_xor(v.w, q, 0u)};
    if (n) v = u32x4{gf16_dbl2(v.x, red2), gf16_dbl2(v.y, red2), gf16_dbl2(v.z, red2), gf16_dbl2(v.w, red2)};
    return v;
}

// Four packed word pairs times alpha^e for alpha = 2 and 1 <= e <= 4 (e
// wave-uniform): one times-4 step when e >= 3, then one doubling (e odd) or
// one more times-4 step; straight-line code under two uniform branches.
__device__ __forceinline__ void gf16_step_pow(uint32_t (&a)[4], int e, uint32_t red2, Gf16Quad q) {
    if (e >= 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = gf16_quad2_xor(a[i], q, 0u);
    }
    if (e & 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = gf16_dbl2(a[i], red2);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = gf16_quad2_xor(a[i], q, 0u);
    }
}

// a = a * alpha^e ^ y, as gf16_step_pow with the XOR in the last step.
__device__ __forceinline__ void gf16_step_pow_xor(uint32_t (&a)[4], int e, const uint32_t (&y)[4], uint32_t red2,
                                                  Gf16Quad q) {
    if (e >= 3) {
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = gf16_quad2_xor(a[i], q, 0u);
    }
    if (e & 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = gf16_dbl2_xor(a[i], red2, y[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = gf16_quad2_xor(a[i], q, y[i]);
    }
}

// The reconstruct by Horner's rule, for tables with alpha = 2.  The inputs
// x[] are the ND = NIN - M surviving data rows (rows row[0] < row[1] < ...)
// and the M parity rows of parity_used.  Each parity syndrome
//     b_r = Par_{pu_r} ^ XOR_j D_{row[j]} * alpha^((pu_r + 1) row[j])
// folds the data rows from the highest down, the accumulator multiplied by
// alpha^((pu_r + 1) (row[j+1] - row[j])) between them (dbl[r][j] doublings;
// dbl[r][ND-1] brings the lowest row to its power); then only
// out_c = XOR_r inv[c][r] b_r takes byte maps (itab, M * M coefficients).
// This is the same field arithmetic as the folded coefficients, so the bytes
// are the reference's.
template <int NIN, int M>
__device__ __forceinline__ void rs_rec_horner(const u32x4* x, const uint32_t (*dbl)[NIN], uint32_t red2,
                                              const uint32_t (*itab)[kRs16Tab], u32x4* out) {
    constexpr int ND = NIN - M;
    u32x4 b[M];
#pragma unroll
    for (int r = 0; r < M; ++r) {
        u32x4 a = ND > 0 ? x[ND > 0 ? ND - 1 : 0] : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int j = ND - 2; j >= 0; --j) a = gf16_dbl_n(a, dbl[r][j], red2) ^ x[j];
        if (ND > 0) a = gf16_dbl_n(a, dbl[r][ND > 0 ? ND - 1 : 0], red2);
        b[r] = a ^ x[ND + r];
        asm volatile("" : "+v"(b[r].x), "+v"(b[r].y), "+v"(b[r].z), "+v"(b[r].w));
    }
    rs_piece_mix<M, M>(b, itab, out);
}

// reconstruct_rs_u16_inplace on the piece engine: NIN = k inputs, M = m
// outputs.  The shard tensor starts b15 bytes past base_al (16-aligned); the
// resource covers res_bytes from base_al.
template <int NIN, int M>
__global__ __launch_bounds__(kPieceBS) __attribute__((amdgpu_waves_per_eu(4))) void rs16_reconstruct_piece_kernel(
        uint8_t* base_al, uint32_t b15, uint32_t res_bytes, uint32_t Sb, int mpar,
        const int32_t* missing, const int32_t* pused, const uint16_t* ex, const uint16_t* lg) {
    constexpr int ND = NIN - M;
    // the folded coefficients (M * NIN), then those of the inverse (M * M)
    __shared__ __attribute__((aligned(16))) uint32_t ptab[M * NIN + M * M][kRs16Tab];
    __shared__ RsRecPlan pl;
    rs16_rec_rows(pl, NIN, mpar, M, missing, pused);
    if (!pl.ok) return;
    const __amdgpu_buffer_rsrc_t rs = chunk_rsrc(base_al, res_bytes);
    uint32_t in[NIN], lim[NIN], out[M];
#pragma unroll
    for (int i = 0; i < NIN; ++i) {
        const uint32_t r = lds_uniform(pl.in_row[i]);
        in[i] = b15 + r * Sb;
        lim[i] = r + 1 == uint32_t(NIN + mpar) ? res_bytes - 16 : ~0u;
    }
#pragma unroll
    for (int g = 0; g < M; ++g) out[g] = b15 + lds_uniform(pl.miss[g]) * Sb;
    const PieceWalk wk = wave_walk();
    const uint32_t lane16 = 16 * (threadIdx.x & 63);
    // the first piece's windows are in flight while the tables are built
    u32x4 c[NIN];
    if (wk.first < Sb) {
#pragma unroll
        for (int i = 0; i < NIN; ++i) c[i] = piece_load(rs, in[i], wk.first + lane16, lim[i]);
    }
    rs16_rec_tables(pl, ptab, NIN, M, ex, lg);
    rs_build_perm_tables(ptab + M * NIN, pl.basis, pl.inv, M * M, ex, lg);
    // syndromes by Horner's rule by horner_tables (the barrier after the
    // tables orders them before their use)
    __syncthreads();
    const bool horner = horner_tables(ex);
    const uint32_t red2 = horner_red2(ex);
    uint32_t dbl[M][NIN];
#pragma unroll
    for (int r = 0; r < M; ++r) {
        const uint32_t f = lds_uniform(pl.pu[r]) + 1;
#pragma unroll
        for (int j = 0; j < NIN; ++j)
            dbl[r][j] = j + 1 < ND ? f * (lds_uniform(pl.in_row[j + 1]) - lds_uniform(pl.in_row[j]))
                                   : (j + 1 == ND ? f * lds_uniform(pl.in_row[0]) : 0u);
    }
    for (uint32_t P = wk.first; P < Sb; P += wk.stride) {
        const bool last = P + wk.stride >= Sb;
        u32x4 n[NIN];
        if (!last) {
#pragma unroll
            for (int i = 0; i < NIN; ++i) n[i] = piece_load(rs, in[i], P + wk.stride + lane16, lim[i]);
        }
        // the byte maps are read from LDS at their use in every piece:
        // hoisted out of the loop they would take 24 registers per coefficient
        asm volatile("" ::: "memory");
        u32x4 o[M];
        if (horner) rs_rec_horner<NIN, M>(c, dbl, red2, ptab + M * NIN, o);
        else rs_piece_mix<NIN, M>(c, ptab, o);
#pragma unroll
        for (int g = 0; g < M; ++g) piece_store<kRsRecNT>(rs, out[g], P + lane16, Sb, o[g]);
        if (!last) {
#pragma unroll
            for (int i = 0; i < NIN; ++i) c[i] = n[i];
        }
    }
}

// Piece-kernel instances: [k - 1][m - 1] for k <= kRsPieceMaxIn, m <= kRsGroup.
typedef void (*RsRecPieceFn)(uint8_t*, uint32_t, uint32_t, uint32_t, int, const int32_t*, const int32_t*,
                           const uint16_t*, const uint16_t*);
template <int... I>
struct RsPieceTable {
    static constexpr RsRecPieceFn rec[sizeof...(I)][kRsGroup] = {
        {rs16_reconstruct_piece_kernel<I + 1, 1>, rs16_reconstruct_piece_kernel<I + 1, 2>}...};
};
using RsPiece = RsPieceTable<0, 1, 2, 3, 4, 5, 6, 7>;
static_assert(kRsPieceMaxIn == 8 && kRsGroup == 2, "instance table");

// Resource bytes from the 16-aligned address at or below p to the end of
// [p, p + n), or 0 when that reaches 2^31 (the piece kernel's limit).
static uint32_t piece_res_bytes(const void* p, uint64_t n) {
    const uint64_t r = ((reinterpret_cast<uintptr_t>(p) & 15) + n + 15) & ~uint64_t(15);
    return r < (uint64_t(1) << 31) ? uint32_t(r) : 0u;
}
static uint8_t* align_down16(const void* p) {
    return reinterpret_cast<uint8_t*>(reinterpret_cast<uintptr_t>(p) & ~uintptr_t(15));
}

// ------------------------------------------------------ one-shot tile encode
// encode_rs_u16 on one kTileBytes tile of every row per block, blocks in tile
// order (the shape of the XOR encode), for m <= 2 parities and k <= 8 data
// rows.  Each lane requests its aligned chunk of every data row at once (lane
// 63 also the chunk after it, which a misaligned window reaches into), forms
// its windows by a DPP lane shift, stores its owned chunks into the data rows
// and folds the windows into the parities by Horner's rule; the parities go
// through LDS to tile_store.
//
// The generator is read from the tables per block with scalar loads
// (table_word_s), whose wait counter is not the vector loads': with
// gf_exp[1] == 2 (the tables of
// init_gf_tables, or any field's exp/log pair whose generator is 2) the
// coefficient alpha^((p+1) i) is (p+1) i doublings with the field's reduction
// word gf_exp[16] = 2^16 reduced (one table read; 0x8000 * 2 through the log
// table took two dependent reads and ran 217.5-221.5 against 220.4-229.9 us);
// for other tables each word is multiplied through the tables.  (Like the
// byte maps, this takes the tables to be a field's.)
//
// Data-row copy stores are non-temporal, except the chunks in the two
// 128-byte lines a wave shares with its neighbours, which go through L2
// (copy_chunk_split); the parity rows' stores are non-temporal too.  On the
// 512 MiB stream, RS(6,2), against the persistent tile kernel (plain stores)
// on one box: 218.7-220.9 against 240.5-247.4 us; with plain parity stores
// this kernel took 247-251 us.  Rows of at least one full tile take this path in every
// tile: in a partial last tile the lanes past a row's end fold bytes that are
// never stored, and their copied chunks carry the next row's bytes (the
// values its own tile copies) or lie past the copy range, where they are
// clipped.
template <int ND, int M>
__global__ __launch_bounds__(kTB) void rs16_encode_tiles_kernel(const uint8_t* in, uint32_t Sb, uint32_t in_bytes,
                                                               FlatCopy fc, uint8_t* par,
                                                               const uint16_t* __restrict__ ex,
                                                               const uint16_t* __restrict__ lg) {
    static_assert(ND >= 1 && ND <= 8 && M >= 1 && M <= 2, "instances");
    __shared__ __attribute__((aligned(16))) uint8_t tile[M][kTileBytes + 16];
    const uint32_t t0 = blockIdx.x * uint32_t(kTileBytes);
    const uint32_t nbytes = Sb - t0 < uint32_t(kTileBytes) ? Sb - t0 : uint32_t(kTileBytes);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t b15 = uint32_t(reinterpret_cast<uintptr_t>(in)) & 15;
    const uint8_t* in_al = in - b15;
    const __amdgpu_buffer_rsrc_t rsin = chunk_rsrc(in_al, (b15 + in_bytes + 15) & ~15u);
    auto row_a = [&](int i) { return b15 + uint32_t(i) * Sb + t0; };   // tile start of row i, from in_al
    u32x4 lo[ND], e1[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) {
        const uint32_t A = row_a(i), sh = A & 15, my = A - sh + 16 * threadIdx.x;
        lo[i] = chunk_load(rsin, my);
        e1[i] = chunk_load(rsin, lane == 63 && sh ? my + 16 : kNoLoad);
    }
    __builtin_amdgcn_sched_barrier(0);
    // each row's head bytes before its first 16-byte-aligned address, which no
    // tile's chunks cover: one lane per byte
    if (fc.dst && t0 == 0 && threadIdx.x < 16 * ND) {
        const uint32_t i = threadIdx.x >> 4, b = threadIdx.x & 15;
        const uint64_t o = uint64_t(i) * Sb;
        const uint32_t mis = uint32_t(reinterpret_cast<uintptr_t>(fc.src + o) & 15);
        if (mis && b < 16 - mis && b < Sb) as_global(fc.dst)[o + b] = as_global(fc.src)[o + b];
    }
    const bool horner = horner_tables(ex);
    const uint16_t red = uint16_t(table_word_s(ex, 16));   // g^16 = 2^16 reduced, when g = 2
    const uint32_t red2 = uint32_t(red) * 0x10001u;
    const Gf16Quad quad = gf16_quad_table(red);
    u32x4 acc[M];
    if (horner) {
#pragma unroll
        for (int i = ND - 1; i >= 0; --i) {
            const uint32_t A = row_a(i), sh = A & 15;
            const u32x4 hi = from_next_lane_or(lo[i], e1[i]);
            const u32x4 x = sh ? funnel16(lo[i], hi, sh) : lo[i];
            if (fc.dst) {
                const uint8_t* c = in_al + (A - sh) + 16 * threadIdx.x + (sh ? 16 : 0);
                copy_chunk_split(fc, c, sh ? hi : lo[i]);
            }
            const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int p = 0; p < M; ++p) {
                uint32_t a[4] = {acc[p].x, acc[p].y, acc[p].z, acc[p].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (i == ND - 1) {
                        a[q] = xv[q];
                    } else if (p == 0) {
                        a[q] = gf16_dbl2_xor(a[q], red2, xv[q]);
                    } else {
                        a[q] = gf16_quad2_xor(a[q], quad, xv[q]);   // g_1 = alpha^2 = 4
                    }
                }
                acc[p] = u32x4{a[0], a[1], a[2], a[3]};
            }
        }
    } else {
        // tables with another generator: every word multiplied through them
#pragma unroll
        for (int p = 0; p < M; ++p) acc[p] = u32x4{0, 0, 0, 0};
        for (int i = 0; i < ND; ++i) {
            const uint32_t A = row_a(i), sh = A & 15;
            const u32x4 hi = from_next_lane_or(lo[i], e1[i]);
            const u32x4 x = sh ? funnel16(lo[i], hi, sh) : lo[i];
            if (fc.dst) {
                const uint8_t* c = in_al + (A - sh) + 16 * threadIdx.x + (sh ? 16 : 0);
                copy_chunk_split(fc, c, sh ? hi : lo[i]);
            }
            for (int p = 0; p < M; ++p) {
                const uint16_t cf = ex[((p + 1) * i) % kGfOrder];
                const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
                uint32_t a[4] = {acc[p].x, acc[p].y, acc[p].z, acc[p].w};
                for (int q = 0; q < 4; ++q) {
                    const uint32_t w0 = gf16_mul_tab(uint16_t(xv[q]), cf, ex, lg);
                    const uint32_t w1 = gf16_mul_tab(uint16_t(xv[q] >> 16), cf, ex, lg);
                    a[q] ^= w0 | (w1 << 16);
                }
                acc[p] = u32x4{a[0], a[1], a[2], a[3]};
            }
        }
    }
#pragma unroll
    for (int p = 0; p < M; ++p) *reinterpret_cast<u32x4*>(tile[p] + 16 * threadIdx.x) = acc[p];
    __syncthreads();
#pragma unroll
    for (int p = 0; p < M; ++p) tile_store<true, kTB>(par + uint64_t(p) * Sb + t0, tile[p], nbytes);
}

typedef void (*RsEncTilesFn)(const uint8_t*, uint32_t, uint32_t, FlatCopy, uint8_t*, const uint16_t*,
                             const uint16_t*);
template <int... I>
struct RsEncTilesTable {
    static constexpr RsEncTilesFn fn[sizeof...(I)][2] = {
        {rs16_encode_tiles_kernel<I + 1, 1>, rs16_encode_tiles_kernel<I + 1, 2>}...};
};
using RsEncTiles = RsEncTilesTable<0, 1, 2, 3, 4, 5, 6, 7>;

// ------------------------------------------------- one-shot tile reconstruct
// reconstruct_rs_u16_inplace of m <= 2 lost data rows on one kTileBytes tile
// of every row per block, blocks in tile order, for k <= 8 data rows, tensors
// below 2 GiB and rows of at least one tile.  A block reads the indices,
// requests its tile of every input row (the surviving data rows in order,
// then the parity rows of parity_used) and forms the windows by a DPP lane
// shift; the lost rows go through LDS to tile_store.
//
// The inverse.  V[r][c] = g^((pu_r + 1) miss_c) for the tables' generator g,
// so every entry is a power of g and the reference's Gauss-Jordan steps
// (benchmark/rs/kernel.cu:151-184: pivot V[0][0], never zero; then the
// remainder of V[1][1], skipped when zero) come down to sums of exponents and
// at most one log-table read.  With a, b, c, d the exponents of V[0][0],
// V[0][1], V[1][0], V[1][1] and e = b + c - a:
//     m = 1:           inv = g^-a
//     m = 2, d == e:   inv = [[g^-a, 0], [g^(c-a), 1]]       (singular, step 2 skipped)
//     m = 2, d != e:   p = log(g^d ^ g^e),
//                      inv = [[g^-a ^ g^(b+c-2a-p), g^(b-a-p)], [g^(c-a-p), g^-p]]
// each product taken in the field the tables define, as the reference's
// table products are (the tables are taken to be a field's exp/log pair).
//
// The generator and the inverse's uniform table reads (gf_exp[d], gf_exp[e],
// the log of their sum) are scalar loads: read as vector loads, the
// generator's round trip came before the block's data loads and the other
// two chained two more round trips after the data had arrived (A/B on one
// box, byte-identical: rows 1 and 4 lost 131.2-132.6 against 122.8-125.3 us,
// rows 0 and 5 126.9-128.6 against 118.8-119.4 us; the encode, whose
// generator read already followed its data loads, 218.3 against 213.1 us).
//
// Every wave forms the inverse's byte maps itself, so no wave waits at a
// block barrier for another's table reads: lane t * 16 + j reads entry t
// times 2^j (the entry's basis products) from the tables into the wave's LDS,
// and lanes below 6 m^2 span each 3-bit field's eight images from three of
// them and pack the maps there too.  The syndromes are Horner's rule over the
// surviving rows when g = 2 (the piece kernel's fold); tables of another
// generator fold every input's coefficient into byte maps built by the block
// and read the windows again one input at a time, so that path adds no
// registers (58 VGPRs, 8 waves per SIMD).
//
// Measured on the 512 MiB stream against the piece kernel (one box, A/B,
// byte-identical): rows 1 and 4 lost 132.5-136.6 against 151.3-156.6 us, rows
// 0 and 5 129.2-129.6 against 146.5-148.1 us, row 2 101.9-102.7 against
// 119.6-120.6 us.  Earlier forms: the maps built once per block behind two
// block barriers, 151-157 us for two rows (104 us for one); every wave
// building them with the generic map loop, 172-186 us.
template <int NIN, int M, int BS = kTB>
__global__ __launch_bounds__(BS) void rs16_reconstruct_tiles_kernel(uint8_t* base_al, uint32_t b15,
                                                                    uint32_t res_bytes, uint32_t Sb, int mpar,
                                                                    const int32_t* __restrict__ missing,
                                                                    const int32_t* __restrict__ pused,
                                                                    const uint16_t* __restrict__ ex,
                                                                    const uint16_t* __restrict__ lg) {
    if constexpr (M > NIN) {
        return;   // no such code: the host requires k >= m
    } else {
        constexpr int ND = NIN - M, NW = BS / 64;
        constexpr uint32_t G = kGfOrder;
        constexpr uint32_t TB = 16 * BS;   // logical bytes per row per tile
        __shared__ __attribute__((aligned(16))) uint8_t tile[M][TB + 16];
        __shared__ __attribute__((aligned(16))) uint32_t wtab[NW][M * M][kRs16Tab];
        __shared__ uint16_t wbasis[NW][M * M * 16];
        int miss[M], pu[M];
        bool ok = true;
#pragma unroll
        for (int q = 0; q < M; ++q) {
            miss[q] = missing[q];
            pu[q] = pused[q];
            ok = ok && miss[q] >= 0 && miss[q] < NIN && pu[q] >= 0 && pu[q] < mpar;
        }
        if (M == 2) ok = ok && miss[0] != miss[M - 1];
        if (!ok) return;   // uniform: the whole grid writes nothing
        const bool horner = horner_tables(ex);
        const int m_lo = M == 2 ? min(miss[0], miss[M - 1]) : miss[0];
        const int m_hi = M == 2 ? max(miss[0], miss[M - 1]) : NIN;
        uint32_t rowp = 0;   // the surviving data rows, 4 bits each
#pragma unroll
        for (int j = 0; j < ND; ++j) {
            int r = j + (j >= m_lo ? 1 : 0);
            if (M == 2) r += r >= m_hi ? 1 : 0;
            rowp |= uint32_t(r) << (4 * j);
        }
        auto row = [&](int j) { return int((rowp >> (4 * j)) & 15); };
        auto in_off = [&](int i) {
            return b15 + uint32_t(i < ND ? row(i) : NIN + pu[i < ND ? 0 : i - ND]) * Sb;
        };
        const uint32_t t0 = blockIdx.x * TB;
        const uint32_t nbytes = Sb - t0 < TB ? Sb - t0 : TB;
        const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
        const __amdgpu_buffer_rsrc_t rs = chunk_rsrc(base_al, res_bytes);
        auto add = [](uint32_t x, uint32_t y) { return x + y >= G ? x + y - G : x + y; };
        auto neg = [](uint32_t x) { return x ? G - x : 0u; };
        // the inverse's entries t = c * M + r as up to two powers of g
        uint32_t L1[M * M], L2[M * M];
        bool has1[M * M], has2[M * M];
        auto inverse = [&]() {
            const uint32_t a = uint32_t((pu[0] + 1) * miss[0]) % G;
#pragma unroll
            for (int t = 0; t < M * M; ++t) has1[t] = true, has2[t] = false, L1[t] = L2[t] = 0;
            L1[0] = neg(a);
            if constexpr (M == 2) {
                const uint32_t b = uint32_t((pu[0] + 1) * miss[1]) % G;
                const uint32_t c = uint32_t((pu[1] + 1) * miss[0]) % G;
                const uint32_t d = uint32_t((pu[1] + 1) * miss[1]) % G;
                const uint32_t e = add(add(b, c), neg(a));
                if (d == e) {
                    has1[1] = false;
                    L1[2] = add(c, neg(a));
                } else {
                    // uniform table reads on the scalar cache, while the
                    // data loads are in flight
                    const uint32_t p = table_word_s(lg, table_word_s(ex, d) ^ table_word_s(ex, e)) % G, np = neg(p);
                    L2[0] = add(add(e, neg(a)), np);   // b + c - 2a - p
                    has2[0] = true;
                    L1[1] = add(add(b, neg(a)), np);
                    L1[2] = add(add(c, neg(a)), np);
                    L1[3] = np;
                }
            }
        };
        u32x4 o[M];
        if (horner) {
            u32x4 lo[NIN], e1[NIN];
            uint32_t shp = 0;   // the windows' shifts, 4 bits each
#pragma unroll
            for (int i = 0; i < NIN; ++i) {
                const uint32_t A = in_off(i) + t0, sh = A & 15, my = A - sh + 16 * threadIdx.x;
                lo[i] = chunk_load(rs, my);
                e1[i] = chunk_load(rs, lane == 63 && sh ? my + 16 : kNoLoad);
                shp |= sh << (4 * i);
            }
            __builtin_amdgcn_sched_barrier(0);
            inverse();
            // this lane's basis product (lanes below 16 M^2), in flight with
            // the data; with g = 2, log(2^j) = j
            uint32_t bv = 0;
            {
                const int t = int(lane >> 4);
                const uint32_t j = lane & 15;
                uint32_t l1 = L1[0], l2 = L2[0];
                bool h1 = has1[0], h2 = has2[0];
#pragma unroll
                for (int q = 1; q < M * M; ++q)
                    if (t == q) l1 = L1[q], l2 = L2[q], h1 = has1[q], h2 = has2[q];
                if (t < M * M) {
                    bv = h1 ? ex[add(l1, j)] : 0u;
                    if (h2) bv ^= ex[add(l2, j)];
                }
            }
            const uint16_t red = uint16_t(table_word_s(ex, 16));   // g^16 = 2^16 reduced, as g = 2
            const uint32_t red2 = uint32_t(red) * 0x10001u;
            const Gf16Quad quad = gf16_quad_table(red);
            u32x4 x[NIN];
#pragma unroll
            for (int i = 0; i < NIN; ++i) {
                const uint32_t sh = (shp >> (4 * i)) & 15;
                const u32x4 hi = from_next_lane_or(lo[i], e1[i]);
                x[i] = sh ? funnel16(lo[i], hi, sh) : lo[i];
            }
            u32x4 bsyn[M];
#pragma unroll
            for (int r = 0; r < M; ++r) {
                const uint32_t f = uint32_t(pu[r] + 1);
                u32x4 acc = ND > 0 ? x[ND > 0 ? ND - 1 : 0] : u32x4{0, 0, 0, 0};
#pragma unroll
                for (int j = ND - 2; j >= 0; --j)
                    acc = gf16_dbl_n(acc, f * uint32_t(row(j + 1) - row(j)), red2, quad) ^ x[j];
                if (ND > 0) acc = gf16_dbl_n(acc, f * uint32_t(row(0)), red2, quad);
                bsyn[r] = acc ^ x[ND + r];
            }
            // byte maps: lane g < 6 M^2 takes coefficient g / 6, source byte
            // (g % 6) / 3 and field g % 3; its three basis products are those
            // of the field's bits (none for bit 8 of the 2-bit field)
            auto wave_lds_sync = []() {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            };
            if (lane < M * M * 16) wbasis[wv][lane] = uint16_t(bv);
            wave_lds_sync();
            {
                const int g = int(lane), t = g / 6, src = (g % 6) / 3, f = g % 3;
                const int b0 = t * 16 + 8 * src + 3 * f;
                if (g < 6 * M * M) {
                    const uint32_t B0 = wbasis[wv][b0], B1 = wbasis[wv][b0 + 1], B2 = f < 2 ? wbasis[wv][b0 + 2] : 0u;
                    const uint32_t e[8] = {0u, B0, B1, B0 ^ B1, B2, B0 ^ B2, B1 ^ B2, B0 ^ B1 ^ B2};
#pragma unroll
                    for (int dst = 0; dst < 2; ++dst) {
#pragma unroll
                        for (int half = 0; half < 2; ++half) {
                            uint32_t dw = 0;
#pragma unroll
                            for (int q = 0; q < 4; ++q) dw |= ((e[4 * half + q] >> (8 * dst)) & 0xFFu) << (8 * q);
                            if (f == 2 && half) dw = 0;   // the 2-bit field has four images
                            wtab[wv][t][(2 * dst + src) * 6 + 2 * f + half] = dw;
                        }
                    }
                }
            }
            wave_lds_sync();
            rs_piece_mix<M, M>(bsyn, wtab[wv], o);
        } else {
            // tables of another generator: the byte maps of the folded
            // coefficients, output c's coefficient of input i at
            // fold[c * NIN + i], built by the block; the windows are read again
            // one input at a time so that this path holds no more registers
            // than the one above
            __shared__ uint16_t fold[M * NIN];
            __shared__ uint16_t fbasis[M * NIN][16];
            __shared__ __attribute__((aligned(16))) uint32_t ftab[M * NIN][kRs16Tab];
            inverse();
            if (threadIdx.x < M * NIN) {
                const int c = threadIdx.x / NIN, in = threadIdx.x % NIN;
                auto inv = [&](int r) {
                    uint16_t v = 0;
#pragma unroll
                    for (int t = 0; t < M * M; ++t)
                        if (t == c * M + r) v = (has1[t] ? ex[L1[t]] : 0) ^ (has2[t] ? ex[L2[t]] : 0);
                    return v;
                };
                uint16_t v = 0;
                if (in < ND) {
#pragma unroll
                    for (int r = 0; r < M; ++r)
                        v ^= gf16_mul_tab(inv(r), ex[(uint32_t(pu[r] + 1) * uint32_t(row(in))) % G], ex, lg);
                } else {
                    v = inv(in - ND);
                }
                fold[threadIdx.x] = v;
            }
            __syncthreads();
            rs_build_perm_tables(ftab, fbasis, fold, M * NIN, ex, lg);
            __syncthreads();
            uint32_t acc[M][4];
#pragma unroll
            for (int c = 0; c < M; ++c) acc[c][0] = acc[c][1] = acc[c][2] = acc[c][3] = 0;
#pragma unroll
            for (int i = 0; i < NIN; ++i) {
                const uint32_t A = in_off(i) + t0, sh = A & 15, my = A - sh + 16 * threadIdx.x;
                const u32x4 l = chunk_load(rs, my);
                const u32x4 h = from_next_lane_or(l, chunk_load(rs, lane == 63 && sh ? my + 16 : kNoLoad));
                const u32x4 xi = sh ? funnel16(l, h, sh) : l;
                uint32_t by[4];
                split_bytes(xi, by);
                Gf8Fields fl[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) fl[q] = gf8_fields(by[q]);
#pragma unroll
                for (int c = 0; c < M; ++c) {
                    const uint32_t* T = ftab[c * NIN + i];
                    acc[c][0] = gf16_fma2(acc[c][0], fl[0], T + 0, fl[1], T + 6);
                    acc[c][1] = gf16_fma2(acc[c][1], fl[0], T + 12, fl[1], T + 18);
                    acc[c][2] = gf16_fma2(acc[c][2], fl[2], T + 0, fl[3], T + 6);
                    acc[c][3] = gf16_fma2(acc[c][3], fl[2], T + 12, fl[3], T + 18);
                    asm volatile("" : "+v"(acc[c][0]), "+v"(acc[c][1]), "+v"(acc[c][2]), "+v"(acc[c][3]) :: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int c = 0; c < M; ++c) o[c] = join_bytes(acc[c]);
        }
#pragma unroll
        for (int c = 0; c < M; ++c) *reinterpret_cast<u32x4*>(tile[c] + 16 * threadIdx.x) = o[c];
        __syncthreads();
#pragma unroll
        for (int c = 0; c < M; ++c)
            tile_store<true, BS>(base_al + b15 + uint64_t(miss[c]) * Sb + t0, tile[c], nbytes);
    }
}

constexpr int kRsRecTB = kTB;                         // threads per block
constexpr uint32_t kRsRecTile = 16 * kRsRecTB;        // logical bytes per row per tile
typedef void (*RsRecTilesFn)(uint8_t*, uint32_t, uint32_t, uint32_t, int, const int32_t*, const int32_t*,
                             const uint16_t*, const uint16_t*);
template <int... I>
struct RsRecTilesTable {
    static constexpr RsRecTilesFn fn[sizeof...(I)][2] = {
        {rs16_reconstruct_tiles_kernel<I + 1, 1, kRsRecTB>, rs16_reconstruct_tiles_kernel<I + 1, 2, kRsRecTB>}...};
};
using RsRecTiles = RsRecTilesTable<0, 1, 2, 3, 4, 5, 6, 7>;

static int rs_grid(int64_t S) {
    const int64_t tiles = (S * 2 + kRsTile - 1) / kRsTile;
    return int(tiles < kRsGrid ? tiles : kRsGrid);
}

// ------------------------------------------- any k and m: Horner over byte maps
// The shapes whose k * m coefficient maps do not fit the kernels above
// (k * m > kRsMaxTables).  Parity p of the encode is Horner's rule over the
// data rows from the last to the first,
//     acc = acc * g_p ^ D_i,   g_p = gf_exp[p + 1] = alpha^(p+1),
// which leaves D_i multiplied by g_p^i = alpha^((p+1) i) = gf_exp[((p+1) i) mod
// 65535], the reference's coefficient (benchmark/rs/kernel.cu:88-95): one
// multiplier per output whatever k is, applied through its byte maps.  The
// reconstruct's syndromes
//     b_r = Par_{pu_r} ^ XOR_{j not lost} D_j * alpha^((pu_r+1) j)
// (benchmark/rs/kernel.cu:190-207) are the same rule over all k data rows, a
// lost row adding nothing but its multiplication; the lost rows are then
// x_c = XOR_r inv[c][r] b_r (:209-219), the inverse by the reference's
// Gauss-Jordan with one thread per matrix entry.  Both take the tables to be a
// field's exp/log pair, as the byte maps everywhere in this file do.
//
// Accumulators are byte-transposed (split_bytes order); a product costs the
// four fields of the accumulator and four gf16_fma2.  Rows are read through
// 16-byte windows at any alignment (RowWin), outputs staged in LDS one row at
// a time and written by tile_store, so every row alignment and length is
// taken.  The encode runs one block row per group of G parities
// (blockIdx.y), each block building its G maps once and walking tiles; the
// reconstruct keeps all M lost rows of a tile in registers.
constexpr int kRsHBS = 256;      // threads per block
constexpr int kRsHGrid = 1024;   // blocks per output group (tiles are walked)
constexpr int kRsHMaxG = 8;      // encode parities per block; reconstruct syndromes per pass

// Keeps one coefficient's byte maps live at a time: the accumulators pass
// through the asm (their products are formed here), the memory clobber keeps
// the next maps' LDS reads after it and the scheduling barrier keeps them
// from moving up.  Without it the compiler reads every loop-invariant map
// into registers ahead of the loops and spills.
__device__ __forceinline__ void rs_h_fence(uint32_t acc[4]) {
    asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]) :: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// acc = acc * c ^ y (byte-transposed words; T = c's byte maps).
__device__ __forceinline__ void gf16_mul_split_xor(uint32_t acc[4], const uint32_t* T, const uint32_t y[4]) {
    Gf8Fields f[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) f[q] = gf8_fields(acc[q]);
    acc[0] = gf16_fma2(y[0], f[0], T + 0, f[1], T + 6);
    acc[1] = gf16_fma2(y[1], f[0], T + 12, f[1], T + 18);
    acc[2] = gf16_fma2(y[2], f[2], T + 0, f[3], T + 6);
    acc[3] = gf16_fma2(y[3], f[2], T + 12, f[3], T + 18);
    rs_h_fence(acc);
}

// acc ^= x * c, with x given by its fields.
__device__ __forceinline__ void gf16_fma_split(uint32_t acc[4], const Gf8Fields f[4], const uint32_t* T) {
    acc[0] = gf16_fma2(acc[0], f[0], T + 0, f[1], T + 6);
    acc[1] = gf16_fma2(acc[1], f[0], T + 12, f[1], T + 18);
    acc[2] = gf16_fma2(acc[2], f[2], T + 0, f[3], T + 6);
    acc[3] = gf16_fma2(acc[3], f[2], T + 12, f[3], T + 18);
    rs_h_fence(acc);
}

// Window n of this thread in a tile at logical byte t0b of `row`: 16 bytes
// starting at word w0, zero past the row's end S (words); `full` when the
// tile lies wholly inside the row (the aligned-chunk path, RowWin rules).
template <int NW>
__device__ __forceinline__ void rs_h_windows(const uint16_t* row, uint64_t t0b, int64_t S, bool full,
                                             u32x4* x) {
    if (full) {
        const RowWin rw = row_win(reinterpret_cast<const uint8_t*>(row) + t0b);
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            u32x4 lo, hi;
            win_chunks(rw, 16 * (threadIdx.x + n * kRsHBS), lo, hi);
            x[n] = win_join(rw, lo, hi);
        }
    } else {
#pragma unroll
        for (int n = 0; n < NW; ++n)
            x[n] = rs_window(row, int64_t(t0b / 2) + 8 * (threadIdx.x + n * kRsHBS), S);
    }
}

// Stage one output row's windows (byte-transposed) and write them to dst.
template <int NW>
__device__ __forceinline__ void rs_h_store(uint8_t* stage, const uint32_t (*acc)[4], uint8_t* dst,
                                           uint32_t nbytes) {
#pragma unroll
    for (int n = 0; n < NW; ++n)
        *reinterpret_cast<u32x4*>(stage + 16 * (threadIdx.x + n * kRsHBS)) = join_bytes(acc[n]);
    __syncthreads();
    tile_store<true, kRsHBS>(dst, stage, nbytes);
    __syncthreads();
}

// With gf_exp[1] == 2 (the tables' generator is 2, the rule of the tile
// kernels), parity p's multiplier alpha^(p+1) is p + 1 doublings: up to
// kRsHChainMax of them (times-4 steps and at most one doubling, 5 VALU ops
// per two doublings of a dword) cost less than a byte-map product (about 14
// per dword).
constexpr int kRsHChainMax = 6;

// The tiles of rs16_encode_horner_kernel.  CHAINS (group 0 only): accumulators
// in natural word order, parity g multiplied by its chain of g + 1 doublings
// (a compile-time length, unrolled), parities past nout skipped; else
// byte-transposed, multiplied through the byte maps ptab.
// Fold one input's windows x (natural word order) into the accumulators:
// the first input (i == k - 1) starts them, every later one is
// acc = acc * g ^ x, by doubling chains (CHAINS) or the byte maps.
template <int G, int NW, bool CHAINS>
__device__ __forceinline__ void rs_h_fold(uint32_t (*acc)[G][4], const u32x4* x, bool first, int nout,
                                          const uint32_t (*ptab)[kRs16Tab], uint32_t red2, Gf16Quad quad) {
#pragma unroll
    for (int n = 0; n < NW; ++n) {
        uint32_t y[4];
        if (CHAINS) y[0] = x[n].x, y[1] = x[n].y, y[2] = x[n].z, y[3] = x[n].w;
        else split_bytes(x[n], y);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (CHAINS && g >= nout) continue;
            if (first) {
                acc[n][g][0] = y[0], acc[n][g][1] = y[1], acc[n][g][2] = y[2], acc[n][g][3] = y[3];
            } else if (CHAINS) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint32_t a = acc[n][g][q];
#pragma unroll
                    for (int d = 0; d + 2 <= g + 1; d += 2) a = gf16_quad2_xor(a, quad, 0u);
                    acc[n][g][q] = (g + 1) & 1 ? gf16_dbl2_xor(a, red2, y[q]) : a ^ y[q];
                }
            } else {
                gf16_mul_split_xor(acc[n][g], ptab[g], y);
            }
        }
    }
}

// The parities of one tile from the accumulators: natural word order (chains)
// back to the byte-transposed form rs_h_store writes.
template <int G, int NW, bool CHAINS>
__device__ __forceinline__ void rs_h_store_all(uint16_t* par, int64_t S, int og, int nout, uint64_t t0b,
                                               uint32_t nbytes, uint32_t (*acc)[G][4], uint8_t* stage) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (g >= nout) break;
        uint32_t o[NW][4];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            if (CHAINS) split_bytes(u32x4{acc[n][g][0], acc[n][g][1], acc[n][g][2], acc[n][g][3]}, o[n]);
            else o[n][0] = acc[n][g][0], o[n][1] = acc[n][g][1], o[n][2] = acc[n][g][2], o[n][3] = acc[n][g][3];
        }
        rs_h_store<NW>(stage, o, reinterpret_cast<uint8_t*>(par + uint64_t(og + g) * S) + t0b, nbytes);
    }
}

// A full tile of 16-byte-aligned rows (each window one aligned load):
// inputs from the last to the first, each one's loads issued two inputs ahead
// into a ring of three window sets, the loop unrolled by three so that no set
// is copied (a copy would wait for its loads).  Past row 0 the ring loads row
// 0 again (cache hits), so every load is unconditional: the compiler then
// waits for an input's windows with the next two inputs' loads still in
// flight, on the first pass through the loop as on the others.  Used for
// three and four parities, where an input's doubling chains give the loads
// ahead of it the most time to arrive; with one or two parities it cost a
// wave per SIMD and ran slower ((25, 2): 118.9 against 111.5 us), with five
// and more its registers spilled SGPRs.  It runs as a kernel instance of its
// own (RING) over the full tiles: beside the general tile loop in one kernel
// it spilled SGPRs too.
template <int G, int NW, bool CHAINS>
__device__ __forceinline__ void rs_h_ring(const uint16_t* in, int64_t S, int k, uint64_t t0b, int nout,
                                          const uint32_t (*ptab)[kRs16Tab], uint32_t red2, Gf16Quad quad,
                                          uint32_t (*acc)[G][4]) {
    u32x4 wa[NW], wb[NW], wc[NW];
    auto load = [&](int i, u32x4* w) {
        const uint8_t* r = reinterpret_cast<const uint8_t*>(in + uint64_t(i > 0 ? i : 0) * S) + t0b;
#pragma unroll
        for (int n = 0; n < NW; ++n) w[n] = ld16(r + 16 * (threadIdx.x + n * kRsHBS));
    };
    int i = k - 1;
    load(i, wa);
    load(i - 1, wb);
    load(i - 2, wc);
    rs_h_fold<G, NW, CHAINS>(acc, wa, true, nout, ptab, red2, quad);
    // from here on, the set after the one just folded holds row i, the next row i - 1
    while (i > 0) {
        --i;
        load(i - 2, wa);
        rs_h_fold<G, NW, CHAINS>(acc, wb, false, nout, ptab, red2, quad);
        if (i == 0) break;
        --i;
        load(i - 2, wb);
        rs_h_fold<G, NW, CHAINS>(acc, wc, false, nout, ptab, red2, quad);
        if (i == 0) break;
        --i;
        load(i - 2, wc);
        rs_h_fold<G, NW, CHAINS>(acc, wa, false, nout, ptab, red2, quad);
    }
}

template <int G, int NW, bool CHAINS, bool RING>
__device__ __forceinline__ void rs_h_encode_tiles(const uint16_t* in, uint16_t* par, int64_t S, int k, int og,
                                                  int nout, const uint32_t (*ptab)[kRs16Tab], uint32_t red2,
                                                  Gf16Quad quad, uint8_t* stage, uint64_t t_begin,
                                                  uint64_t t_end) {
    constexpr uint32_t TB = 16 * kRsHBS * NW;
    const uint64_t Sb = uint64_t(S) * 2;
    for (uint64_t tt = t_begin + blockIdx.x; tt < t_end; tt += gridDim.x) {
        const uint64_t t0b = tt * TB;
        const uint32_t nbytes = uint32_t(Sb - t0b < TB ? Sb - t0b : TB);
        uint32_t acc[NW][G][4];
        if constexpr (RING) {
            rs_h_ring<G, NW, CHAINS>(in, S, k, t0b, nout, ptab, red2, quad, acc);
            rs_h_store_all<G, NW, CHAINS>(par, S, og, nout, t0b, nbytes, acc, stage);
            continue;
        }
        const bool full = nbytes == TB;
        u32x4 x[NW], nx[NW];
        rs_h_windows<NW>(in + uint64_t(k - 1) * S, t0b, S, full, x);
        for (int i = k - 1; i >= 0; --i) {
            if (i > 0) rs_h_windows<NW>(in + uint64_t(i - 1) * S, t0b, S, full, nx);
#pragma unroll
            for (int n = 0; n < NW; ++n) {
                uint32_t y[4];
                if (CHAINS) y[0] = x[n].x, y[1] = x[n].y, y[2] = x[n].z, y[3] = x[n].w;
                else split_bytes(x[n], y);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if (CHAINS && g >= nout) continue;
                    if (i == k - 1) {
                        acc[n][g][0] = y[0], acc[n][g][1] = y[1], acc[n][g][2] = y[2], acc[n][g][3] = y[3];
                    } else if (CHAINS) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            uint32_t a = acc[n][g][q];
#pragma unroll
                            for (int d = 0; d + 2 <= g + 1; d += 2) a = gf16_quad2_xor(a, quad, 0u);
                            acc[n][g][q] = (g + 1) & 1 ? gf16_dbl2_xor(a, red2, y[q]) : a ^ y[q];
                        }
                    } else {
                        gf16_mul_split_xor(acc[n][g], ptab[g], y);
                    }
                }
            }
            if (i > 0) {
#pragma unroll
                for (int n = 0; n < NW; ++n) x[n] = nx[n];
            }
        }
        rs_h_store_all<G, NW, CHAINS>(par, S, og, nout, t0b, nbytes, acc, stage);
    }
}

// encode_rs_u16's parity rows og .. og + G - 1 (og = blockIdx.y * G; those at
// or past m are computed and not stored).  in: the k data rows of S words;
// par: parity row 0.
template <int G, int NW, bool RING>
__global__ __launch_bounds__(kRsHBS) void rs16_encode_horner_kernel(const uint16_t* in, uint16_t* par, int64_t S,
                                                                    int k, int m, const uint16_t* ex,
                                                                    const uint16_t* lg, uint64_t t_begin,
                                                                    uint64_t t_end) {
    constexpr uint32_t TB = 16 * kRsHBS * NW;
    __shared__ __attribute__((aligned(16))) uint32_t ptab[G][kRs16Tab];
    __shared__ uint16_t basis[G][16];
    __shared__ uint16_t coef[G];
    __shared__ __attribute__((aligned(16))) uint8_t stage[TB + 16];
    const int og = int(blockIdx.y) * G;
    const int nout = m - og < G ? m - og : G;
    // (the chains with eight parities held spilled SGPRs: m <= 6 only)
    if constexpr (G <= kRsHChainMax) {
        if (og == 0 && nout <= kRsHChainMax && horner_tables(ex)) {
            const uint16_t red = uint16_t(table_word_s(ex, 16));   // 2^16 reduced
            rs_h_encode_tiles<G, NW, true, RING>(in, par, S, k, og, nout, ptab, uint32_t(red) * 0x10001u,
                                                 gf16_quad_table(red), stage, t_begin, t_end);
            return;
        }
    }
    if (threadIdx.x < G) {
        const int p = og + int(threadIdx.x);
        coef[threadIdx.x] = p < m ? ex[uint32_t(p + 1) % kGfOrder] : uint16_t(0);
    }
    __syncthreads();
    rs_build_perm_tables(ptab, basis, coef, G, ex, lg);
    __syncthreads();
    rs_h_encode_tiles<G, NW, false, RING>(in, par, S, k, og, nout, ptab, 0u, Gf16Quad{0, 0}, stage, t_begin, t_end);
}

// The inverse of V[r][c] = gf_exp[((pu_r + 1) miss_c) mod 65535] by
// benchmark/rs/kernel.cu:135-185 (pivot order, zero-pivot skip), one thread
// per entry: within a step the rows r != i change only from row i and their
// own factor V[r][i], read by every thread of row r before any writes it, so
// each entry sees the serial loop's sequence of products.  All threads of the
// block call it; inv (m x m) is left in LDS, followed by a barrier.
__device__ __forceinline__ void rs16_gauss_jordan(int m, const int* miss, const int* pu, uint16_t* V, uint16_t* inv,
                                                  const uint16_t* ex, const uint16_t* lg) {
    const int t = int(threadIdx.x), r = t / m, c = t % m;
    const bool mine = t < m * m;
    if (mine) {
        V[t] = ex[uint32_t((pu[r] + 1) * miss[c]) % kGfOrder];
        inv[t] = r == c ? 1 : 0;
    }
    __syncthreads();
    for (int i = 0; i < m; ++i) {
        int pr = i;
        while (pr < m && V[pr * m + i] == 0) ++pr;
        if (pr == m) continue;   // uniform: every thread read the same V
        if (pr != i && t < m) {
            uint16_t s = V[i * m + t];
            V[i * m + t] = V[pr * m + t];
            V[pr * m + t] = s;
            s = inv[i * m + t];
            inv[i * m + t] = inv[pr * m + t];
            inv[pr * m + t] = s;
        }
        __syncthreads();
        const uint16_t ip = gf16_div_tab(1, V[i * m + i], ex, lg);   // V[i][i] != 0 here
        __syncthreads();
        if (t < m) {
            V[i * m + t] = gf16_mul_tab(V[i * m + t], ip, ex, lg);
            inv[i * m + t] = gf16_mul_tab(inv[i * m + t], ip, ex, lg);
        }
        __syncthreads();
        const uint16_t f = mine && r != i ? V[r * m + i] : uint16_t(0);
        __syncthreads();
        if (f) {
            V[r * m + c] ^= gf16_mul_tab(f, V[i * m + c], ex, lg);
            inv[r * m + c] ^= gf16_mul_tab(f, inv[i * m + c], ex, lg);
        }
        __syncthreads();
    }
}

// Whether the reconstruct of M <= 4 lost rows runs its syndromes as doubling
// chains on rs16_reconstruct_ring_kernel: tables with generator 2
// (horner_tables) and every parity row used below 4, so each syndrome's
// multiplier alpha^(pu + 1) is at most four doublings per row.  s_pu in LDS;
// uniform.
template <int M>
__device__ __forceinline__ bool rs_rec_ring_ok(const int* s_pu, const uint16_t* ex) {
    bool ok = M <= 4 && horner_tables(ex);
#pragma unroll
    for (int r = 0; r < M; ++r) ok = ok && lds_uniform(s_pu[r]) <= 3;
    return ok;
}

// reconstruct_rs_u16_inplace of M lost data rows, any k (inputs: the
// surviving data rows and the parity rows of parity_used).  sh: the shard
// tensor, rows of S words.  Out-of-range or repeated lost rows, or parity rows
// outside the tensor, write nothing.
template <int M>
__device__ __forceinline__ void rs_rec_general(uint16_t* sh, int64_t S, int k, int mpar, const int32_t* missing,
                                               const int32_t* pused, const uint16_t* ex, const uint16_t* lg) {
    constexpr int NW = 1, G = M < kRsHMaxG ? M : kRsHMaxG, NT = M + M * M;
    constexpr uint32_t TB = 16 * kRsHBS * NW;
    static_assert(M * M <= kRsHBS, "one thread per inverse entry");
    // maps: syndrome multipliers g_r = gf_exp[pu_r + 1] at [r], inverse entry
    // inv[c][r] at [M + c * M + r]
    __shared__ __attribute__((aligned(16))) uint32_t ptab[NT][kRs16Tab];
    __shared__ uint16_t basis[NT][16];
    __shared__ uint16_t coef[NT];
    __shared__ uint16_t sV[M * M], sInv[M * M];
    __shared__ int s_miss[M], s_pu[M], s_desc[M], s_ok;
    __shared__ __attribute__((aligned(16))) uint8_t stage[TB + 16];
    if (threadIdx.x < M) {
        s_miss[threadIdx.x] = missing[threadIdx.x];
        s_pu[threadIdx.x] = pused[threadIdx.x];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int ok = 1;
        for (int q = 0; q < M; ++q) {
            ok &= s_miss[q] >= 0 && s_miss[q] < k && s_pu[q] >= 0 && s_pu[q] < mpar;
            for (int q2 = 0; q2 < q; ++q2) ok &= s_miss[q2] != s_miss[q];
        }
        s_ok = ok;
        // the lost rows from the highest down, the order the syndromes meet them
        for (int q = 0; q < M; ++q) {
            int v = s_miss[q], at = q;
            while (at > 0 && s_desc[at - 1] < v) s_desc[at] = s_desc[at - 1], --at;
            s_desc[at] = v;
        }
    }
    __syncthreads();
    if (!s_ok) return;   // uniform: the whole grid writes nothing
    const uint64_t Sb = uint64_t(S) * 2;
    const uint64_t ntiles = (Sb + TB - 1) / TB;
    if (blockIdx.x >= ntiles) return;
    rs16_gauss_jordan(M, s_miss, s_pu, sV, sInv, ex, lg);
    for (int e = threadIdx.x; e < NT; e += kRsHBS)
        coef[e] = e < M ? ex[uint32_t(s_pu[e] + 1) % kGfOrder] : sInv[e - M];
    __syncthreads();
    rs_build_perm_tables(ptab, basis, coef, NT, ex, lg);
    __syncthreads();
    // indices stay in LDS and are read where used (2 M of them held in scalar
    // registers beside the loop's own spilled SGPRs for M >= 8)
    auto desc = [&](int q) { return q < M ? int(lds_uniform(s_desc[q])) : -1; };
    for (uint64_t tt = blockIdx.x; tt < ntiles; tt += gridDim.x) {
        const uint64_t t0b = tt * TB;
        const uint32_t nbytes = uint32_t(Sb - t0b < TB ? Sb - t0b : TB);
        const bool full = nbytes == TB;
        uint32_t out[M][NW][4];
#pragma unroll
        for (int c = 0; c < M; ++c)
#pragma unroll
            for (int n = 0; n < NW; ++n) out[c][n][0] = out[c][n][1] = out[c][n][2] = out[c][n][3] = 0;
#pragma unroll
        for (int og = 0; og < M; og += G) {
            constexpr int GG = G;
            const int ng = M - og < GG ? M - og : GG;
            uint32_t acc[GG][NW][4];
#pragma unroll
            for (int g = 0; g < GG; ++g)
#pragma unroll
                for (int n = 0; n < NW; ++n) acc[g][n][0] = acc[g][n][1] = acc[g][n][2] = acc[g][n][3] = 0;
            u32x4 x[NW], nx[NW];
            // nxt: the highest lost row below the rows passed (nl of them lost)
            int nl = 0, nxt = desc(0);
            bool have = k - 1 != nxt;
            if (!have) nxt = desc(++nl);
            if (have) rs_h_windows<NW>(sh + uint64_t(k - 1) * S, t0b, S, full, x);
            for (int j = k - 1; j >= 0; --j) {
                const bool next = j > 0 && j - 1 != nxt;
                if (j > 0 && !next) nxt = desc(++nl);
                if (next) rs_h_windows<NW>(sh + uint64_t(j - 1) * S, t0b, S, full, nx);
                uint32_t y[NW][4];
#pragma unroll
                for (int n = 0; n < NW; ++n) {
                    if (have) split_bytes(x[n], y[n]);
                    else y[n][0] = y[n][1] = y[n][2] = y[n][3] = 0;
                }
#pragma unroll
                for (int g = 0; g < GG; ++g) {
                    if (g >= ng) break;
#pragma unroll
                    for (int n = 0; n < NW; ++n) gf16_mul_split_xor(acc[g][n], ptab[og + g], y[n]);
                }
                if (next) {
#pragma unroll
                    for (int n = 0; n < NW; ++n) x[n] = nx[n];
                }
                have = next;
            }
            // b_r = acc ^ Par_{pu_r}, then out_c ^= inv[c][r] b_r
#pragma unroll
            for (int g = 0; g < GG; ++g) {
                if (g >= ng) break;
                u32x4 pw[NW];
                rs_h_windows<NW>(sh + uint64_t(k + int(lds_uniform(s_pu[og + g]))) * S, t0b, S, full, pw);
#pragma unroll
                for (int n = 0; n < NW; ++n) {
                    uint32_t y[4];
                    split_bytes(pw[n], y);
                    Gf8Fields f[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) f[q] = gf8_fields(acc[g][n][q] ^ y[q]);
#pragma unroll
                    for (int c = 0; c < M; ++c) gf16_fma_split(out[c][n], f, ptab[M + c * M + og + g]);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < M; ++c)
            rs_h_store<NW>(stage, out[c], reinterpret_cast<uint8_t*>(sh + uint64_t(lds_uniform(s_miss[c])) * S) + t0b,
                           nbytes);
    }
}

template <int M>
__global__ __launch_bounds__(kRsHBS) void rs16_reconstruct_horner_kernel(uint16_t* sh, int64_t S, int k, int mpar,
                                                                         const int32_t* missing,
                                                                         const int32_t* pused,
                                                                         const uint16_t* ex,
                                                                         const uint16_t* lg) {
    rs_rec_general<M>(sh, S, k, mpar, missing, pused, ex, lg);
}

// reconstruct_rs_u16_inplace of M <= 4 lost data rows, any k, on the tiles
// [0, t_end) of 16-byte-aligned rows whose length is a multiple of 16 bytes
// (tiles of NW windows of 16 bytes per thread; the last may be partial), when
// rs_rec_ring_ok holds (else the block codes the general kernel's tiles
// instead, through rs_rec_general: one launch serves either way).  Syndrome r is b_r = Par_{pu_r} ^ XOR over surviving rows j of
// D_j * g_r^j, g_r = alpha^(pu_r + 1), by Horner's rule over the surviving
// rows only (highest first): between consecutive survivors j > j' the
// accumulator is multiplied by g_r^(j - j') -- j - j' steps of gf16_step_pow,
// in natural word order -- and after the lowest survivor by g_r^(j_min).
// Each surviving row's windows are loaded two survivors ahead into a ring of
// three window sets (no register copies; past the last survivor the ring
// loads parity row pu_0's windows, which the tile reads again at its end), so
// a row is waited for with the next two rows' loads in flight.  The lost rows
// come from the syndromes through the inverse's byte maps, out_c = XOR_r
// inv[c][r] * b_r, as in the general kernel, and are stored straight from
// registers (each thread's 16-byte windows, aligned).
template <int M, int NW>
__global__ __launch_bounds__(kRsHBS) void rs16_reconstruct_ring_kernel(uint16_t* sh, int64_t S, int k, int mpar,
                                                                       const int32_t* missing,
                                                                       const int32_t* pused,
                                                                       const uint16_t* ex, const uint16_t* lg,
                                                                       uint64_t t_end) {
    static_assert(M >= 1 && M <= 4, "ring reconstruct: at most four lost rows");
    constexpr uint32_t TB = 16 * kRsHBS * NW;
    __shared__ __attribute__((aligned(16))) uint32_t ptab[M * M][kRs16Tab];   // inv[c][r] at [c * M + r]
    __shared__ uint16_t basis[M * M][16];
    __shared__ uint16_t coef[M * M];
    __shared__ uint16_t sV[M * M], sInv[M * M];
    __shared__ int s_miss[M], s_pu[M], s_desc[M], s_ok;
    if (threadIdx.x < M) {
        s_miss[threadIdx.x] = missing[threadIdx.x];
        s_pu[threadIdx.x] = pused[threadIdx.x];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int ok = 1;
        for (int q = 0; q < M; ++q) {
            ok &= s_miss[q] >= 0 && s_miss[q] < k && s_pu[q] >= 0 && s_pu[q] < mpar;
            for (int q2 = 0; q2 < q; ++q2) ok &= s_miss[q2] != s_miss[q];
        }
        s_ok = ok;
        for (int q = 0; q < M; ++q) {
            int v = s_miss[q], at = q;
            while (at > 0 && s_desc[at - 1] < v) s_desc[at] = s_desc[at - 1], --at;
            s_desc[at] = v;
        }
    }
    __syncthreads();
    if (!s_ok) return;   // uniform: the whole grid writes nothing
    if (!rs_rec_ring_ok<M>(s_pu, ex)) {   // uniform: every tile through the byte maps
        rs_rec_general<M>(sh, S, k, mpar, missing, pused, ex, lg);
        return;
    }
    rs16_gauss_jordan(M, s_miss, s_pu, sV, sInv, ex, lg);
    for (int e = threadIdx.x; e < M * M; e += kRsHBS) coef[e] = sInv[e];
    __syncthreads();
    rs_build_perm_tables(ptab, basis, coef, M * M, ex, lg);
    __syncthreads();
    const uint16_t red = uint16_t(table_word_s(ex, 16));
    const uint32_t red2 = uint32_t(red) * 0x10001u;
    const Gf16Quad quad = gf16_quad_table(red);
    auto desc = [&](int q) { return q < M ? int(lds_uniform(s_desc[q])) : -1; };
    auto pu = [&](int r) { return int(lds_uniform(s_pu[r])); };
    const int dummy = k + pu(0);
    const uint64_t Sb = uint64_t(S) * 2;
    for (uint64_t tt = blockIdx.x; tt < t_end; tt += gridDim.x) {
        const uint64_t t0b = tt * TB;
        // window n at byte lo[n] of the tile; windows past the row's end (the
        // last tile may be partial) read the tile's first window and store nothing
        uint32_t lo[NW];
        bool in[NW];
#pragma unroll
        for (int n = 0; n < NW; ++n) {
            const uint32_t o = 16 * (threadIdx.x + n * kRsHBS);
            in[n] = t0b + o < Sb;
            lo[n] = in[n] ? o : 0u;
        }
        auto load = [&](int row, u32x4 (&w)[NW]) {
            const uint8_t* rp =
                    reinterpret_cast<const uint8_t*>(sh + uint64_t(row >= 0 ? row : dummy) * uint64_t(S)) + t0b;
#pragma unroll
            for (int n = 0; n < NW; ++n) w[n] = ld16(rp + lo[n]);
        };
        // the next surviving row below j (-1 when none): nl counts the lost
        // rows passed, all of them above the rows still to come
        int nl = 0;
        auto next = [&](int j) {
            if (j <= 0) return -1;
            int r = j - 1;
            while (nl < M && desc(nl) == r) {
                --r;
                ++nl;
            }
            return r;
        };
        uint32_t acc[M][NW][4];
        // acc = acc * g^gap ^ w (acc = w for gap 0): gap - 1 plain steps, then
        // one step with the XOR
        auto fold = [&](const u32x4 (&w)[NW], int gap) {
#pragma unroll
            for (int n = 0; n < NW; ++n) {
                const uint32_t y[4] = {w[n].x, w[n].y, w[n].z, w[n].w};
#pragma unroll
                for (int r = 0; r < M; ++r) {
                    if (gap == 0) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc[r][n][q] = y[q];
                    } else {
                        const int e = pu(r) + 1;
                        for (int t = 1; t < gap; ++t) gf16_step_pow(acc[r][n], e, red2, quad);
                        gf16_step_pow_xor(acc[r][n], e, y, red2, quad);
                    }
                }
            }
        };
        u32x4 wa[NW], wb[NW], wc[NW];
        int ra = next(k);
        load(ra, wa);
        int rb = next(ra);
        load(rb, wb);
        int rc = next(rb);
        load(rc, wc);
        if (ra >= 0) {
            fold(wa, 0);
        } else {   // every data row lost: the syndromes are the parity rows
#pragma unroll
            for (int r = 0; r < M; ++r)
#pragma unroll
                for (int n = 0; n < NW; ++n) acc[r][n][0] = acc[r][n][1] = acc[r][n][2] = acc[r][n][3] = 0;
        }
        int prev = ra;
        for (;;) {
            if (rb < 0) break;
            ra = next(rc);
            load(ra, wa);
            fold(wb, prev - rb);
            prev = rb;
            if (rc < 0) break;
            rb = next(ra);
            load(rb, wb);
            fold(wc, prev - rc);
            prev = rc;
            if (ra < 0) break;
            rc = next(rb);
            load(rc, wc);
            fold(wa, prev - ra);
            prev = ra;
        }
        // the lowest survivor's power, the parity rows, then the inverse
        u32x4 pw[M][NW];
#pragma unroll
        for (int r = 0; r < M; ++r) load(k + pu(r), pw[r]);
        uint32_t out[M][NW][4];
#pragma unroll
        for (int c = 0; c < M; ++c)
#pragma unroll
            for (int n = 0; n < NW; ++n) out[c][n][0] = out[c][n][1] = out[c][n][2] = out[c][n][3] = 0;
#pragma unroll
        for (int r = 0; r < M; ++r) {
#pragma unroll
            for (int n = 0; n < NW; ++n) {
                for (int t = 0; t < prev; ++t) gf16_step_pow(acc[r][n], pu(r) + 1, red2, quad);
                uint32_t b[4];
                split_bytes(u32x4{acc[r][n][0] ^ pw[r][n].x, acc[r][n][1] ^ pw[r][n].y, acc[r][n][2] ^ pw[r][n].z,
                                  acc[r][n][3] ^ pw[r][n].w},
                            b);
                Gf8Fields f[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) f[q] = gf8_fields(b[q]);
#pragma unroll
                for (int c = 0; c < M; ++c) gf16_fma_split(out[c][n], f, ptab[c * M + r]);
            }
        }
#pragma unroll
        for (int c = 0; c < M; ++c) {
            uint8_t* dst = reinterpret_cast<uint8_t*>(sh + uint64_t(lds_uniform(s_miss[c])) * uint64_t(S)) + t0b;
#pragma unroll
            for (int n = 0; n < NW; ++n)
                if (in[n]) st16(dst + lo[n], join_bytes(out[c][n]));
        }
    }
}

typedef void (*RsRecHornerFn)(uint16_t*, int64_t, int, int, const int32_t*, const int32_t*, const uint16_t*,
                              const uint16_t*);
template <int... I>
struct RsRecHornerTable {
    static constexpr RsRecHornerFn fn[sizeof...(I)] = {rs16_reconstruct_horner_kernel<I + 1>...};
};
using RsRecHorner = RsRecHornerTable<0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15>;
static_assert(kRsMaxM == 16, "instance table");

static unsigned rs_h_grid(int64_t S, uint32_t tile) {
    const uint64_t tiles = (uint64_t(S) * 2 + tile - 1) / tile;
    return unsigned(tiles < uint64_t(kRsHGrid) ? tiles : uint64_t(kRsHGrid));
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
    // every k and m whose exponents (p + 1) i the reference's int arithmetic
    // holds (benchmark/rs/kernel.cu:93), with at most 65535 groups of parities
    if (int64_t(data_shards - 1) * parity_shards >= (int64_t(1) << 31) ||
        int64_t(parity_shards) > int64_t(65535) * kRsHMaxG)
        return set_error(KVEC_EUNSUPPORTED, "kvec_rs16_encode: k=%d m=%d out of range", data_shards,
                         parity_shards);
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
    // k * m maps beyond the LDS tables: Horner over byte maps, data rows copied apart
    const bool general = int64_t(data_shards) * parity_shards > kRsMaxTables;
    const bool fuse = !general && parity_shards > 0 && fused_copy_ok(data_padded, shards, data_bytes);
    if (!fuse) {
        int rc = copy_d2d(shards, data_padded, data_bytes, st, "kvec_rs16_encode");
        if (rc) return rc;
    }
    if (parity_shards == 0) return KVEC_OK;
    if (general) {
        const uint16_t* in = (const uint16_t*)data_padded;
        uint16_t* par = (uint16_t*)shards + uint64_t(data_shards) * S;
        constexpr uint32_t TB = 16 * kRsHBS * 2;
        const uint64_t Sb = uint64_t(S) * 2, ntiles = (Sb + TB - 1) / TB;
        // three or four parities over 16-byte-aligned rows: the full tiles on
        // the ring kernel, a partial last tile on the other
        const bool aligned = (reinterpret_cast<uintptr_t>(in) & 15) == 0 && Sb % 16 == 0;
        const uint64_t nring = (parity_shards == 3 || parity_shards == 4) && aligned ? Sb / TB : 0;
        auto range = [&](auto kern, int G, uint64_t t0, uint64_t t1) {
            if (t1 <= t0) return;
            const uint64_t n = t1 - t0;
            const unsigned groups = unsigned((parity_shards + G - 1) / G);
            hipLaunchKernelGGL(kern, dim3(unsigned(n < uint64_t(kRsHGrid) ? n : uint64_t(kRsHGrid)), groups),
                               dim3(kRsHBS), 0, st, in, par, S, data_shards, parity_shards, gf_exp, gf_log, t0, t1);
        };
        auto launch = [&](auto kern, int G) { range(kern, G, nring, ntiles); };
        // one group of exactly m parities up to kRsHMaxG, else groups of kRsHMaxG
        switch (parity_shards) {
            case 1: launch(rs16_encode_horner_kernel<1, 2, false>, 1); break;
            case 2: launch(rs16_encode_horner_kernel<2, 2, false>, 2); break;
            case 3:
                range(rs16_encode_horner_kernel<3, 2, true>, 3, 0, nring);
                launch(rs16_encode_horner_kernel<3, 2, false>, 3);
                break;
            case 4:
                range(rs16_encode_horner_kernel<4, 2, true>, 4, 0, nring);
                launch(rs16_encode_horner_kernel<4, 2, false>, 4);
                break;
            case 5: launch(rs16_encode_horner_kernel<5, 2, false>, 5); break;
            case 6: launch(rs16_encode_horner_kernel<6, 2, false>, 6); break;
            case 7: launch(rs16_encode_horner_kernel<7, 2, false>, 7); break;
            default: launch(rs16_encode_horner_kernel<kRsHMaxG, 2, false>, kRsHMaxG); break;
        }
        return check_launch("kvec_rs16_encode");
    }
    RsJob j{};
    j.copy = fuse ? FlatCopy{(const uint8_t*)data_padded, (uint8_t*)shards, data_bytes}
                  : FlatCopy{nullptr, nullptr, 0};
    j.S = S;
    j.nin = data_shards;
    j.nout = parity_shards;
    for (int i = 0; i < data_shards; ++i) j.in_rows[i] = (const uint16_t*)data_padded + uint64_t(i) * S;
    for (int p = 0; p < parity_shards; ++p)
        j.out_rows[p] = (uint16_t*)shards + uint64_t(data_shards + p) * S;
    const uint64_t Sb = uint64_t(S) * 2;
    if (data_shards <= 8 && parity_shards <= 2 && Sb >= uint64_t(kTileBytes) &&
        data_bytes < (uint64_t(1) << 31)) {
        hipLaunchKernelGGL(RsEncTiles::fn[data_shards - 1][parity_shards - 1],
                           dim3(uint32_t((Sb + kTileBytes - 1) / kTileBytes)), dim3(kTB), 0, st,
                           (const uint8_t*)data_padded, uint32_t(Sb), uint32_t(data_bytes), j.copy,
                           (uint8_t*)shards + uint64_t(data_shards) * Sb, gf_exp, gf_log);
        return check_launch("kvec_rs16_encode");
    }
    hipLaunchKernelGGL(rs16_encode_kernel, dim3(rs_grid(S)), dim3(kRsBS), 0, st, j, gf_exp, gf_log);
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
    if (m == 0) return KVEC_OK;
    if (m < 0 || m > kRsMaxM)
        return set_error(KVEC_EINVAL, "kvec_rs16_reconstruct: m=%d (must be <= %d)", m, kRsMaxM);
    if (!shards || !missing_data || !parity_used || !gf_exp || !gf_log)
        return set_error(KVEC_EINVAL, "kvec_rs16_reconstruct: null pointer");
    if (data_shards < m || parity_shards < m || shard_size < 0)
        return set_error(KVEC_EINVAL, "kvec_rs16_reconstruct: k=%d parity=%d m=%d S=%d", data_shards,
                         parity_shards, m, shard_size);
    if (shard_size == 0) return KVEC_OK;
    if (int64_t(data_shards) * m > kRsMaxTables) {
        // k * m maps beyond the LDS tables: syndromes by Horner's rule.  Up to
        // four lost rows over 16-byte-aligned rows: the ring kernel, whose
        // blocks take the byte-map tiles instead when the tables or parity rows
        // do not allow doubling chains; otherwise the byte-map kernel.
        // Windows per thread of the ring tiles by M (measured on the 512 MiB
        // stream: one for two lost rows, 121-123 against 123-127 us; two for
        // the others, four lost rows 217 against 225 us).
        constexpr uint32_t TB = 16 * kRsHBS;
        const uint32_t ring_nw = m == 2 ? 1 : 2;
        const uint64_t Sb = uint64_t(shard_size) * 2;
        const bool aligned = (reinterpret_cast<uintptr_t>(shards) & 15) == 0 && Sb % 16 == 0;
        hipStream_t st = as_stream(stream);
        if (m > 4 || !aligned) {
            hipLaunchKernelGGL(RsRecHorner::fn[m - 1], dim3(rs_h_grid(shard_size, TB)), dim3(kRsHBS), 0, st,
                               (uint16_t*)shards, int64_t(shard_size), data_shards, parity_shards, missing_data,
                               parity_used, gf_exp, gf_log);
            return check_launch("kvec_rs16_reconstruct");
        }
        // the ring's tiles, a partial last one included; its grid also serves
        // the byte-map tiles (walked by grid stride)
        const uint64_t nring = (Sb + TB * ring_nw - 1) / (TB * ring_nw);
        const uint64_t nmap = (Sb + TB - 1) / TB;
        const uint64_t nblk = nring > nmap ? nring : nmap;
        const dim3 grid(unsigned(nblk < uint64_t(kRsHGrid) ? nblk : uint64_t(kRsHGrid)));
        auto ring = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(kRsHBS), 0, st, (uint16_t*)shards, int64_t(shard_size), data_shards,
                               parity_shards, missing_data, parity_used, gf_exp, gf_log, nring);
        };
        switch (m) {
            case 1: ring(rs16_reconstruct_ring_kernel<1, 2>); break;
            case 2: ring(rs16_reconstruct_ring_kernel<2, 1>); break;
            case 3: ring(rs16_reconstruct_ring_kernel<3, 2>); break;
            default: ring(rs16_reconstruct_ring_kernel<4, 2>); break;
        }
        return check_launch("kvec_rs16_reconstruct");
    }
    const uint64_t Sb = uint64_t(shard_size) * 2;
    const uint32_t res = piece_res_bytes(shards, uint64_t(data_shards + parity_shards) * Sb);
    if (data_shards <= kRsPieceMaxIn && m <= kRsGroup && res && Sb >= kRsRecTile) {
        hipLaunchKernelGGL(RsRecTiles::fn[data_shards - 1][m - 1], dim3(uint32_t((Sb + kRsRecTile - 1) / kRsRecTile)),
                           dim3(kRsRecTB), 0, as_stream(stream), align_down16(shards),
                           uint32_t(reinterpret_cast<uintptr_t>(shards) & 15), res, uint32_t(Sb), parity_shards,
                           missing_data, parity_used, gf_exp, gf_log);
        return check_launch("kvec_rs16_reconstruct");
    }
    if (data_shards <= kRsPieceMaxIn && m <= kRsGroup && res) {
        hipLaunchKernelGGL(RsPiece::rec[data_shards - 1][m - 1], dim3(piece_grid(Sb, kRsPieceBlocks)), dim3(kPieceBS), 0,
                           as_stream(stream), align_down16(shards), uint32_t(reinterpret_cast<uintptr_t>(shards) & 15),
                           res, uint32_t(Sb), parity_shards, missing_data, parity_used, gf_exp, gf_log);
        return check_launch("kvec_rs16_reconstruct");
    }
    hipLaunchKernelGGL(rs16_reconstruct_kernel, dim3(rs_grid(shard_size)), dim3(kRsBS), 0,
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
