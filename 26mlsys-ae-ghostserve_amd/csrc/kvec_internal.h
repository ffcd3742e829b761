// kvec_internal.h -- shared device and host helpers of libkvec (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kvec.h"

namespace kvec {

// 16-byte vector: one global_load_dwordx4 / global_store_dwordx4.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxShards = 64;

// Host array of device pointers, passed to kernels by value (kernarg).
template <int N>
struct Ptrs {
    uint8_t* p[N];
};

// ------------------------------------------------------------- memory ops
// Streaming loads/stores: every byte of the coded stripes is touched once per
// launch, so they bypass cache residency (nt bit on gfx950).
__device__ __forceinline__ u32x4 ld_stream(const uint8_t* base, uint64_t off) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + off));
}
__device__ __forceinline__ void st_stream(uint8_t* base, uint64_t off, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(base + off));
}
// Global-memory views of a generic pointer.  Row pointers that a kernel reads
// out of LDS or a table have no provable address space, and generic (flat)
// accesses count against both the memory and the LDS wait counters, so a wait
// for an LDS read would also wait for every load in flight.
template <class T>
using gptr = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> as_global(T* p) {
    return (gptr<T>)p;
}

// Ordinary (cached) 16-byte load, for data that neighbouring lanes re-read.
__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
    return *as_global(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(uint8_t* p, u32x4 v) {
    *as_global(reinterpret_cast<u32x4*>(p)) = v;
}

// Three-input XOR in one VALU op (v_bitop3_b32 with truth table 0x96); the
// compiler does not form it from a ^ b ^ c by itself.
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}
__device__ __forceinline__ u32x4 xor3(u32x4 a, u32x4 b, u32x4 c) {
    return u32x4{xor3(a.x, b.x, c.x), xor3(a.y, b.y, c.y), xor3(a.z, b.z, c.z), xor3(a.w, b.w, c.w)};
}

// XOR accumulator that folds its inputs two at a time with the 3-input XOR.
// Whether an input is held is known at compile time once the loops that feed
// it are unrolled, so `held` costs nothing.
struct Xor3Acc {
    u32x4 a, pend;
    bool held;
    __device__ __forceinline__ explicit Xor3Acc(u32x4 init = u32x4{0, 0, 0, 0})
        : a(init), pend{0, 0, 0, 0}, held(false) {}
    __device__ __forceinline__ void add(u32x4 x) {
        if (held) a = xor3(a, pend, x);
        else pend = x;
        held = !held;
    }
    __device__ __forceinline__ u32x4 get() const { return held ? a ^ pend : a; }
};

// Xor3Acc for one dword.
struct Xor3Acc1 {
    uint32_t a, pend;
    bool held;
    __device__ __forceinline__ Xor3Acc1() : a(0), pend(0), held(false) {}
    __device__ __forceinline__ void add(uint32_t x) {
        if (held) a = xor3(a, pend, x);
        else pend = x;
        held = !held;
    }
    __device__ __forceinline__ uint32_t get() const { return held ? a ^ pend : a; }
};

// The same interface with 2-input XORs and one register per accumulator, for
// kernels whose accumulators alone would otherwise crowd the register file
// (RDP over p >= 11 keeps 2(p-1) of them).
struct XorAcc {
    u32x4 a;
    __device__ __forceinline__ explicit XorAcc(u32x4 init = u32x4{0, 0, 0, 0}) : a(init) {}
    __device__ __forceinline__ void add(u32x4 x) { a ^= x; }
    __device__ __forceinline__ u32x4 get() const { return a; }
};

// Accumulator for an RDP kernel over prime p: 3-input XORs while the 2(p-1)
// accumulators' held inputs fit beside the cells in flight.
template <int P>
using RdpAcc = typename std::conditional<(P <= 7), Xor3Acc, XorAcc>::type;

// XOR of N cells with 3-input XORs.
template <int N>
__device__ __forceinline__ u32x4 xor_all(const u32x4* v) {
    u32x4 a = v[0];
    int i = 1;
#pragma unroll
    for (; i + 1 < N; i += 2) a = xor3(a, v[i], v[i + 1]);
    if (i < N) a ^= v[i];
    return a;
}

// ------------------------------------------------------------- shard views
// One shard buffer seen by a kernel.  Shards below 4 GiB use a buffer
// resource: a load's row offset rides in an SGPR (soffset), the lane offset in
// one VGPR, and there is no 64-bit address arithmetic per access.  Larger
// shards use 64-bit global addressing.  Loads and stores are non-temporal:
// every byte is read or written once per launch.
constexpr int kAuxLoadNT = 2;        // nt
constexpr int kAuxStoreNT = 2;       // nt
constexpr uint32_t kBufWord3 = 0x00020000;

template <bool BUF>
struct ShardView;

template <>
struct ShardView<true> {
    __amdgpu_buffer_rsrc_t rs;
    __device__ __forceinline__ ShardView(const uint8_t* p, uint64_t nbytes)
        : rs(__builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)(uint32_t)nbytes,
                                               (int)kBufWord3)) {}
    __device__ __forceinline__ u32x4 load(uint64_t row_off, uint32_t lane_off) const {
        return __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane_off, (uint32_t)row_off, kAuxLoadNT));
    }
    // Stores fold the row offset into the lane offset and pass an immediate
    // soffset of 0.  The compiler enforces the wait states between a store of
    // more than 64 bits and a VALU write of its data registers only for
    // stores without an SGPR soffset; with the row offset in an SGPR it let
    // such writes follow a store back to back (found by scanning the
    // generated code), which the code here never allows.
    __device__ __forceinline__ void store(uint64_t row_off, uint32_t lane_off, u32x4 v) const {
        __builtin_amdgcn_raw_buffer_store_b128(v, rs, lane_off + (uint32_t)row_off, 0, kAuxStoreNT);
    }
};

template <>
struct ShardView<false> {
    uint8_t* p;
    __device__ __forceinline__ ShardView(const uint8_t* q, uint64_t) : p((uint8_t*)q) {}
    __device__ __forceinline__ u32x4 load(uint64_t row_off, uint32_t lane_off) const {
        return ld_stream(p + row_off, lane_off);
    }
    __device__ __forceinline__ void store(uint64_t row_off, uint32_t lane_off, u32x4 v) const {
        st_stream(p + row_off, lane_off, v);
    }
};

// A buffer resource addresses at most 2^32 - 1 bytes.
inline bool fits_buffer(uint64_t nbytes) { return nbytes < (uint64_t(1) << 32); }

// ------------------------------------------------------------- fast u32 div
// Division of a 32-bit unsigned value by a run-time invariant divisor
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up variant with the 33-bit multiplier
// split into mulhi + add).  Exact for every n, d < 2^32, d >= 1.
struct FastDiv {
    uint32_t d, m, s1, s2;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t l = 0;
    while (l < 32 && (uint64_t(1) << l) < d) ++l;  // l = ceil(log2 d)
    f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
    f.s1 = l < 1 ? l : 1;
    f.s2 = l > 1 ? l - 1 : 0;
    return f;
}

__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
#ifdef __HIP_DEVICE_COMPILE__
    uint32_t q = __umulhi(n, f.m);
#else
    uint32_t q = uint32_t((uint64_t(n) * f.m) >> 32);
#endif
    return (((n - q) >> f.s1) + q) >> f.s2;
}

// ------------------------------------------------------------- RDP stripes
// Stripe geometry of a spec RDP shard set.  Every shard is (p-1)*R bytes, cut
// into stripes of (p-1)*U bytes (the last one shorter when U does not divide
// R).  Stripe s has rows of g_s = min(U, R - s*U) bytes, row r at byte
// s*(p-1)*U + r*g_s of the shard, and byte offset o < g_s of its rows is one
// RDP instance.  U = 0 (or U >= R) is a single stripe: p-1 row planes of R
// bytes.  Kernels run one wave per 1 KiB of a stripe's row (16 bytes per
// lane), so every wave-uniform quantity below is a scalar.
constexpr uint32_t kRdpWaveBytes = 1024;

struct RdpGeom {
    uint64_t U;        // row bytes of a full stripe
    uint64_t g_last;   // row bytes of the last stripe
    uint32_t ns;       // stripes
    FastDiv bps;       // waves (1 KiB row pieces) per stripe
};

// rows-per-stripe (p-1) is a kernel template parameter; R, U in bytes.
inline RdpGeom make_rdp_geom(uint64_t R, uint64_t U) {
    RdpGeom g{};
    if (U == 0 || U >= R) U = R;
    g.U = U;
    g.ns = U ? uint32_t((R + U - 1) / U) : 0;
    g.g_last = U ? R - uint64_t(g.ns - 1) * U : 0;
    g.bps = make_fastdiv(uint32_t((U + kRdpWaveBytes - 1) / kRdpWaveBytes));
    return g;
}
inline uint64_t rdp_waves(const RdpGeom& g) { return uint64_t(g.ns) * g.bps.d; }

// The calling wave's stripe: its shard-relative base, its row length, and the
// lane's byte offset within the rows (>= g when the lane is past the row end).
struct RdpWave {
    uint64_t base;
    uint64_t g;
    uint32_t within;
};
__device__ __forceinline__ RdpWave rdp_wave(const RdpGeom& G, int rows, uint32_t wave, uint32_t lane) {
    const uint32_t s = fdiv(wave, G.bps);
    const uint32_t cb = wave - s * G.bps.d;
    RdpWave w;
    w.base = uint64_t(s) * uint64_t(rows) * G.U;
    w.g = s + 1 == G.ns ? G.g_last : G.U;
    w.within = cb * kRdpWaveBytes + lane * 16;
    return w;
}

// ------------------------------------------------------------- host status
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Whether [a, a+na) and [b, b+nb) share a byte.
inline bool ranges_overlap(const void* a, uint64_t na, const void* b, uint64_t nb) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return na && nb && x < y + nb && y < x + na;
}

// One buffer of a launch, for check_no_alias (idx < 0: no index in messages).
struct Span {
    const void* p;
    uint64_t n;
    const char* name;
    int idx;
};

// Host check before a launch that no buffer it writes (w) shares a byte with
// another written buffer or with a buffer it only reads (r; those may alias
// each other).  The kernels read their inputs while other blocks of the same
// launch write their outputs, so with such an overlap the bytes a block reads
// would depend on block timing.  KVEC_EINVAL names the first pair found.
int check_no_alias(const Span* w, int nw, const Span* r, int nr, const char* fn);

// Stream-ordered device copies and zero fills done by kernels (copy.hip), so
// that no entry point records a memcpy or memset node under graph capture.
// copy_d2d: n bytes, any alignments; dst == src is a no-op; other overlaps
// are refused (KVEC_EINVAL).
int copy_d2d(void* dst, const void* src, uint64_t n, hipStream_t st, const char* what);
int zero_d(void* dst, uint64_t n, hipStream_t st, const char* what);

inline bool is_prime(int p) {
    if (p < 2) return false;
    for (int q = 2; q * q <= p; ++q)
        if (p % q == 0) return false;
    return true;
}

inline unsigned blocks_for(int64_t work, int threads) {
    return unsigned((work + threads - 1) / threads);
}

}  // namespace kvec
