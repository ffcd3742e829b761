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

constexpr int kTB = 256;                // threads per tile block
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

// Write logical bytes [0, nbytes) of the LDS tile `t` (16-byte aligned, with 16
// bytes of slack after nbytes) to dst, any alignment.  All threads call it.
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
        for (uint32_t k = threadIdx.x; k < nch; k += kTB) {
            const uint32_t al = dal + 16 * k;
            u32x4 v = *reinterpret_cast<const u32x4*>(t + al);
            if (dsh) v = funnel16(v, *reinterpret_cast<const u32x4*>(t + al + 16), dsh);
            st16(reinterpret_cast<uint8_t*>(A0 + 16 * uintptr_t(k)), v);
        }
        // head [D0, A0) and tail [A1, E): at most 15 bytes each
        const uint32_t nh = uint32_t(A0 - D0), nt = uint32_t(E - A1);
        const uint32_t i = threadIdx.x;
        const gptr<uint8_t> g = as_global(dst);
        if (i < nh) g[i] = t[i];
        else if (i >= 16 && i - 16 < nt) g[(A1 - D0) + (i - 16)] = t[(A1 - D0) + (i - 16)];
    } else {
        const gptr<uint8_t> g = as_global(dst);
        for (uint32_t i = threadIdx.x; i < nbytes; i += kTB) g[i] = t[i];
    }
}

}  // namespace kvec
