// tile_engine.h -- column tiles over the reference's packed row layout.
//
// The reference keeps all shards of a stripe in one [(rows), S] tensor, so row
// r starts at byte r*S*es: rows are misaligned whenever S*es % 16 != 0.  A
// block here owns a tile of kTileBytes logical bytes (the same columns of
// every row).  Each thread computes 16 logical bytes of every output row from
// 16-byte windows of the input rows: a window at any byte address is two
// aligned 16-byte loads joined with v_alignbyte (the second load is skipped
// when the window is aligned).  Outputs are staged in LDS and written back at
// the output row's own alignment: whole aligned 16-byte stores inside the
// tile, byte stores for the partial chunks at its two ends.
#pragma once

#include "kvec_internal.h"

namespace kvec {

// Threads per tile block.  Measured on the 512 MiB stream against 256-thread
// (4 KiB) tiles, same box, byte-identical: backup 238 against 242 us, P/Q 118
// against 119, the two-row recovery 201 against 207, the XOR encode 203
// against 206, reconstruct_xor 118 against 122.  A tile boundary of a
// misaligned row splits a 128-byte line between two blocks; wider tiles have
// half as many.  (The XOR encode from K and V keeps 256-thread tiles: 201
// against 195 us with 512.)
constexpr int kTB = 512;
constexpr int kTileBytes = kTB * 16;    // logical bytes per row per tile

// Bytes sh .. sh+15 of the 32-byte value (a = bytes 0..15, b = 16..31).
__device__ __forceinline__ u32x4 funnel16(u32x4 a, u32x4 b, uint32_t sh) {
    const uint32_t r = sh & 3;
    uint32_t s0, s1, s2, s3, s4;
    switch (sh >> 2) {
        case 0: s0 = a.x; s1 = a.y; s2 = a.z; s3 = a.w; s4 = b.x; break;
        case 1: s0 = a.y; s1 = a.z; s2 = a.w; s3 = b.x; s4 = b.y; break;
        case 2: s0 = a.z; s1 = a.w; s2 = b.x; s3 = b.y; s4 = b.z; break;
        default: s0 = a.w; s1 = b.x; s2 = b.y; s3 = b.z; s4 = b.w; break;
    }
    return u32x4{__builtin_amdgcn_alignbyte(s1, s0, r), __builtin_amdgcn_alignbyte(s2, s1, r),
                 __builtin_amdgcn_alignbyte(s3, s2, r), __builtin_amdgcn_alignbyte(s4, s3, r)};
}

// Wave-wide lane shifts (DPP wave_shl:1 / wave_shr:1, one VALU op per dword):
// from_next_lane gives lane i the value of lane i+1 (lane 63 gets 0),
// from_prev_lane gives lane i the value of lane i-1 (lane 0 gets 0).
__device__ __forceinline__ u32x4 from_next_lane(u32x4 v) {
    return u32x4{uint32_t(__builtin_amdgcn_update_dpp(0, int(v.x), 0x130, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(0, int(v.y), 0x130, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(0, int(v.z), 0x130, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(0, int(v.w), 0x130, 0xF, 0xF, false))};
}
__device__ __forceinline__ u32x4 from_prev_lane(u32x4 v) {
    return u32x4{uint32_t(__builtin_amdgcn_update_dpp(0, int(v.x), 0x138, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(0, int(v.y), 0x138, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(0, int(v.z), 0x138, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(0, int(v.w), 0x138, 0xF, 0xF, false))};
}

// The same shifts with the lane whose source is outside the wave (63 for
// from_next_lane_or, 0 for from_prev_lane_or) taking `edge` instead of 0: DPP
// leaves the destination's old value in a lane with no source lane, and the
// old value is `edge`.  One instruction per dword and no per-lane select.
__device__ __forceinline__ u32x4 from_next_lane_or(u32x4 v, u32x4 edge) {
    return u32x4{uint32_t(__builtin_amdgcn_update_dpp(int(edge.x), int(v.x), 0x130, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(int(edge.y), int(v.y), 0x130, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(int(edge.z), int(v.z), 0x130, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(int(edge.w), int(v.w), 0x130, 0xF, 0xF, false))};
}
__device__ __forceinline__ u32x4 from_prev_lane_or(u32x4 v, u32x4 edge) {
    return u32x4{uint32_t(__builtin_amdgcn_update_dpp(int(edge.x), int(v.x), 0x138, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(int(edge.y), int(v.y), 0x138, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(int(edge.z), int(v.z), 0x138, 0xF, 0xF, false)),
                 uint32_t(__builtin_amdgcn_update_dpp(int(edge.w), int(v.w), 0x138, 0xF, 0xF, false))};
}

// Lane j's value of v, in every lane (ds_bpermute; j in [0, 64)).
__device__ __forceinline__ u32x4 lane_value(u32x4 v, int j) {
    const int a = 4 * j;
    return u32x4{uint32_t(__builtin_amdgcn_ds_bpermute(a, int(v.x))),
                 uint32_t(__builtin_amdgcn_ds_bpermute(a, int(v.y))),
                 uint32_t(__builtin_amdgcn_ds_bpermute(a, int(v.z))),
                 uint32_t(__builtin_amdgcn_ds_bpermute(a, int(v.w)))};
}

// 16-byte loads through a buffer resource of fewer than 2^31 bytes.  A
// voffset at or past 2^31 is then out of range: the load returns 0 without
// touching memory, which lets only some lanes (a wave's edge lanes) fetch a
// chunk with no branch around the load.
constexpr uint32_t kNoLoad = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t chunk_rsrc(const void* p, uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)n, (int)kBufWord3);
}

__device__ __forceinline__ u32x4 chunk_load(__amdgpu_buffer_rsrc_t rs, uint32_t voff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, kAuxLoadNT));
}

// A pointer that every lane holds the same value of, moved to scalar
// registers: offsets and shifts derived from it are then wave-uniform, so a
// switch on them is a scalar branch rather than per-lane selects.
template <class T>
__device__ __forceinline__ T* wave_uniform(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(v))));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(v >> 32))));
    return reinterpret_cast<T*>((uint64_t(hi) << 32) | lo);
}

// 16 bytes at any address.  The caller guarantees the 16 bytes belong to the
// tensor; the aligned chunks read around them then hold at least one of its
// bytes each and cannot cross into an unmapped page.
__device__ __forceinline__ u32x4 load_window16(const uint8_t* p) {
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p) & 15);
    const uint8_t* al = p - sh;
    const u32x4 lo = ld16(al);
    if (sh == 0) return lo;
    return funnel16(lo, ld16(al + 16), sh);
}

// A row seen from one tile: the 16-byte-aligned address at or below the
// tile's first byte `p` and the misalignment, both wave-uniform.
struct RowWin {
    const uint8_t* al;
    uint32_t sh;
};

__device__ __forceinline__ RowWin row_win(const uint8_t* p) {
    p = wave_uniform(p);
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p) & 15);
    return RowWin{p - sh, sh};
}

// The aligned chunks under the 16 bytes at tile offset `off` (a multiple of
// 16) of a tile that lies wholly inside its row: lo, and hi when the row is
// misaligned (hi then holds at least one byte of the row).  Both loads are
// always issued (hi re-reads lo's chunk, a cache hit, when the row is
// aligned and hi is unused): a branch around the second load would make the
// compiler wait for the first at the join, serializing the rows' loads.
__device__ __forceinline__ void win_chunks(const RowWin& r, uint32_t off, u32x4& lo, u32x4& hi) {
    lo = ld16(r.al + off);
    hi = ld16(r.al + off + (r.sh ? 16 : 0));
}

__device__ __forceinline__ u32x4 win_join(const RowWin& r, u32x4 lo, u32x4 hi) {
    return r.sh ? funnel16(lo, hi, r.sh) : lo;
}

__device__ __forceinline__ uint8_t byte_of(u32x4 v, int i) {
    const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return uint8_t(w >> (8 * (i & 3)));
}

__device__ __forceinline__ u32x4 set_byte(u32x4 v, int i, uint8_t b) {
    const uint32_t sh = 8 * (i & 3), m = ~(0xFFu << sh), x = uint32_t(b) << sh;
    if (i < 4) v.x = (v.x & m) | x;
    else if (i < 8) v.y = (v.y & m) | x;
    else if (i < 12) v.z = (v.z & m) | x;
    else v.w = (v.w & m) | x;
    return v;
}

// ------------------------------------------------------------- fused copy
// A flat device-to-device copy of [src, src+len) to dst carried by a coding
// kernel's own tile loads, so the copied bytes are read from HBM once (the
// reference's encode kernels copy the data rows into the shard tensor while
// coding them: benchmark/xor/kernel.cu:17-41, benchmark/rs/kernel.cu:67-102).
// dst - src is a multiple of 16, so an aligned source chunk is an aligned
// destination chunk.  Ownership, for rows laid end to end in the range:
//   - in a tile wholly inside its row, each lane stores the aligned chunk
//     starting inside its window (hi when the row is misaligned, else lo);
//     over the tile these are disjoint and continue where the previous tile's
//     stopped;
//   - the first tile stores each row's head bytes up to its first aligned
//     address, and the row's partial last tile stores its bytes one by one.
// Chunks that reach into the next row store bytes that row also stores,
// with the same values; nothing past src+len is written.
struct FlatCopy {
    const uint8_t* src;
    uint8_t* dst;   // null: no copy
    uint64_t len;
};

// Host side: whether a copy of `len` bytes from src to dst can ride on the
// coding kernel (disjoint ranges, equal alignment modulo 16).
inline bool fused_copy_ok(const void* src, const void* dst, uint64_t len) {
    const uintptr_t s = reinterpret_cast<uintptr_t>(src), d = reinterpret_cast<uintptr_t>(dst);
    return ((s ^ d) & 15) == 0 && (d >= s + len || s >= d + len);
}

// Store the source chunk at `c` (16-byte aligned, value v) at its place in dst.
// NT: non-temporal stores, faster for the XOR encode's copy (measured on
// MI355X), slower for the RS GF(2^16) encode's.
template <bool NT = true>
__device__ __forceinline__ void copy_chunk(const FlatCopy& fc, const uint8_t* c, u32x4 v) {
    const uint64_t o = uint64_t(c - fc.src);
    if (o + 16 <= fc.len) {
        if (NT) st_stream(fc.dst, o, v);
        else st16(fc.dst + o, v);
        return;
    }
    const gptr<uint8_t> d = as_global(fc.dst);
    for (int i = 0; i < 16 && o + i < fc.len; ++i) d[o + i] = byte_of(v, i);
}

// copy_chunk for a wave whose lanes store consecutive chunks: non-temporal,
// except the chunks of the two 128-byte lines the wave shares with its
// neighbours when its 1 KiB does not start on a line, which go through L2,
// where the two parts of such a line merge (written non-temporally, the two
// parts reach HBM separately).
__device__ __forceinline__ void copy_chunk_split(const FlatCopy& fc, const uint8_t* c, u32x4 v) {
    const uint64_t o = uint64_t(c - fc.src);
    if (o + 16 <= fc.len) {
        const uint32_t lane = threadIdx.x & 63;
        const uint32_t pre = uint32_t((reinterpret_cast<uintptr_t>(fc.dst) + o - 16 * uint64_t(lane)) >> 4) & 7;
        if (pre != 0 && (lane < 8 - pre || lane >= 64 - pre)) st16(fc.dst + o, v);
        else st_stream(fc.dst, o, v);
        return;
    }
    const gptr<uint8_t> d = as_global(fc.dst);
    for (int i = 0; i < 16 && o + i < fc.len; ++i) d[o + i] = byte_of(v, i);
}

template <bool NT = true>
__device__ __forceinline__ void copy_owned(const FlatCopy& fc, const RowWin& r, uint32_t off,
                                           u32x4 lo, u32x4 hi) {
    if (r.sh) copy_chunk<NT>(fc, r.al + off + 16, hi);
    else copy_chunk<NT>(fc, r.al + off, lo);
}

// Bytes [a, b) of the range, one by one.
__device__ __forceinline__ void copy_bytes(const FlatCopy& fc, uint64_t a, uint64_t b) {
    const gptr<const uint8_t> s = as_global(fc.src);
    const gptr<uint8_t> d = as_global(fc.dst);
    for (uint64_t i = a; i < b; ++i) d[i] = s[i];
}

// Head bytes of the row starting at range offset `o`: up to its first
// 16-byte-aligned address (at most 15, no further than `row_len`).
__device__ __forceinline__ void copy_row_head(const FlatCopy& fc, uint64_t o, uint64_t row_len) {
    const uint32_t mis = uint32_t(reinterpret_cast<uintptr_t>(fc.src + o) & 15);
    const uint64_t n = mis ? 16 - mis : 0;
    copy_bytes(fc, o, o + (n < row_len ? n : row_len));
}

// Write logical bytes [0, nbytes) of the LDS tile `t` (16-byte aligned, with 16
// bytes of slack after nbytes) to dst, any alignment.  All BS threads of the
// block call it.  NT: the aligned 16-byte stores are non-temporal.  Which is
// faster depends on the kernel's other traffic (measured per kernel on
// MI355X): the P/Q rows of the star-diagonal code write 12 % faster with it,
// the XOR parity row next to the fused data-row copy 7 % slower.
template <bool NT = false, int BS = kTB>
__device__ __forceinline__ void tile_store(uint8_t* dst, const uint8_t* t, uint32_t nbytes) {
    dst = wave_uniform(dst);
    nbytes = uint32_t(__builtin_amdgcn_readfirstlane(int(nbytes)));
    const uintptr_t D0 = reinterpret_cast<uintptr_t>(dst);
    const uintptr_t E = D0 + nbytes;
    const uintptr_t A0 = (D0 + 15) & ~uintptr_t(15);
    const uintptr_t A1 = E & ~uintptr_t(15);
    if (A0 < A1) {
        const uint32_t delta = uint32_t(A0 - D0);
        const uint32_t dsh = delta & 15, dal = delta - dsh;   // uniform
        const uint32_t nch = uint32_t((A1 - A0) >> 4);
        // head [D0, A0) and tail [A1, E), at most 15 bytes each, stored before
        // the chunks (measured on the 512 MiB stream against after them: the
        // two-row recovery 196.5 against 200.8 us, reconstruct_xor 115.5
        // against 118.3, P/Q 116.0 against 117.5)
        const uint32_t nh = uint32_t(A0 - D0), nt = uint32_t(E - A1);
        const uint32_t i = threadIdx.x;
        const gptr<uint8_t> g = as_global(dst);
        if (i < nh) g[i] = t[i];
        else if (i >= 16 && i - 16 < nt) g[(A1 - D0) + (i - 16)] = t[(A1 - D0) + (i - 16)];
        // Thread slot j stores chunk j - pre, pre being the position of chunk
        // 0 in its 128-byte line, so that every wave's store instruction
        // covers whole lines: with chunk j per thread, each 1 KiB a wave
        // stored began and ended inside a line that the neighbouring wave's
        // store completed (measured on the 512 MiB stream, rows misaligned by
        // 86 bytes mod 128: the two-row recovery 191.5 against 196.5 us, the
        // fused backup 234.9 against 237.3).
        const uint32_t pre = uint32_t(A0 >> 4) & 7;
        for (uint32_t j = threadIdx.x; j < nch + pre; j += BS) {
            if (j < pre) continue;
            const uint32_t k = j - pre;
            const uint32_t al = dal + 16 * k;
            u32x4 v = *reinterpret_cast<const u32x4*>(t + al);
            if (dsh) v = funnel16(v, *reinterpret_cast<const u32x4*>(t + al + 16), dsh);
            if (NT) st_stream(reinterpret_cast<uint8_t*>(A0 + 16 * uintptr_t(k)), 0, v);
            else st16(reinterpret_cast<uint8_t*>(A0 + 16 * uintptr_t(k)), v);
        }
    } else {
        const gptr<uint8_t> g = as_global(dst);
        for (uint32_t i = threadIdx.x; i < nbytes; i += BS) g[i] = t[i];
    }
}

}  // namespace kvec
