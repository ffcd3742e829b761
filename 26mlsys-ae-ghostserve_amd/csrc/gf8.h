// gf8.h -- GF(2^8) with polynomial 0x11D: host tables, the systematic Cauchy
// parity block C[i][j] = 1 / ((k+i) ^ j), matrix inversion, and the
// v_perm_b32 constant multiply shared by the RS kernels.
//
// Multiplication by a constant c is GF(2)-linear in x, so with x split into
// bit fields x = f0 + f1*2^3 + f2*2^6 (3, 3 and 2 bits):
//     x*c = T0[f0] ^ T1[f1] ^ T2[f2],   T0[v] = v*c, T1[v] = (v<<3)*c, T2[v] = (v<<6)*c.
// Each table has at most 8 one-byte entries, i.e. two dwords, which is exactly
// what one v_perm_b32 indexes: a byte-permute of the 8-byte table by the field
// values of four data bytes at once.
#pragma once

#include "kvec_internal.h"

namespace kvec {

// ------------------------------------------------------------ GF(2^8) host side
struct Gf8 {
    uint8_t exp[512], log[256];
    constexpr Gf8() : exp(), log() {
        unsigned x = 1;
        for (int i = 0; i < 255; ++i) {
            exp[i] = uint8_t(x);
            log[x] = uint8_t(i);
            x <<= 1;
            if (x & 0x100) x ^= 0x11D;
        }
        for (int i = 255; i < 512; ++i) exp[i] = exp[i - 255];
    }
    constexpr uint8_t mul(uint8_t a, uint8_t b) const {
        return (a && b) ? exp[log[a] + log[b]] : 0;
    }
    constexpr uint8_t inv(uint8_t a) const { return a ? exp[255 - log[a]] : 0; }
};
static constexpr Gf8 kGf8{};

constexpr int kRs8MaxK = 32;
constexpr int kRs8MaxM = 8;
constexpr int kRs8MaxCoef = 64;   // k * m (keeps the kernel arguments under 2 KiB)
constexpr int kRs8BS = 128;

// v_perm tables of one coefficient: {T0 lo, T0 hi, T1 lo, T1 hi, T2 lo, T2 hi}
inline void perm_tables(uint8_t c, uint32_t t[6]) {
    for (int f = 0; f < 3; ++f) {
        uint8_t e[8];
        for (int v = 0; v < 8; ++v) e[v] = (f == 2 && v > 3) ? 0 : kGf8.mul(uint8_t(v << (3 * f)), c);
        t[2 * f] = e[0] | (e[1] << 8) | (e[2] << 16) | (uint32_t(e[3]) << 24);
        t[2 * f + 1] = e[4] | (e[5] << 8) | (e[6] << 16) | (uint32_t(e[7]) << 24);
    }
}

// coefficient (o, j) of an nout x nin mix lives at t[o * nin + j]
struct Gf8Mix {
    uint32_t t[kRs8MaxCoef][6];
};

// ------------------------------------------------------------ device side
__device__ __forceinline__ uint32_t gf8_mul4(uint32_t f0, uint32_t f1, uint32_t f2,
                                             const uint32_t* t) {
    // v_perm_b32 D, S0, S1, sel: selector bytes 0-3 pick S1 bytes, 4-7 S0 bytes
    return __builtin_amdgcn_perm(t[1], t[0], f0) ^ __builtin_amdgcn_perm(t[3], t[2], f1) ^
           __builtin_amdgcn_perm(t[5], t[4], f2);
}

inline void cauchy(int k, int m, uint8_t* C) {
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < k; ++j) C[i * k + j] = kGf8.inv(uint8_t((k + i) ^ j));
}

// Gauss-Jordan inverse of a k x k matrix over GF(2^8); false if singular.
inline bool gf8_invert(int k, const uint8_t* A, uint8_t* X) {
    uint8_t M[kRs8MaxK][2 * kRs8MaxK];
    for (int r = 0; r < k; ++r)
        for (int c = 0; c < 2 * k; ++c) M[r][c] = c < k ? A[r * k + c] : uint8_t(c - k == r);
    for (int c = 0; c < k; ++c) {
        int piv = c;
        while (piv < k && !M[piv][c]) ++piv;
        if (piv == k) return false;
        if (piv != c)
            for (int x = 0; x < 2 * k; ++x) {
                uint8_t t = M[c][x];
                M[c][x] = M[piv][x];
                M[piv][x] = t;
            }
        const uint8_t ip = kGf8.inv(M[c][c]);
        for (int x = 0; x < 2 * k; ++x) M[c][x] = kGf8.mul(M[c][x], ip);
        for (int r = 0; r < k; ++r) {
            if (r == c || !M[r][c]) continue;
            const uint8_t f = M[r][c];
            for (int x = 0; x < 2 * k; ++x) M[r][x] ^= kGf8.mul(f, M[c][x]);
        }
    }
    for (int r = 0; r < k; ++r)
        for (int c = 0; c < k; ++c) X[r * k + c] = M[r][k + c];
    return true;
}

// Decode map of systematic RS(k, m) with Cauchy block C for the erased shards
// er[0 .. k+m) (data 0..k-1, parity k..k+m-1).  The inputs are the first k
// surviving shards in index order (surv[0..k)); the outputs are the erased
// shards in index order (outs[0..*nout)), output o = XOR_q M[o*k + q] * in_q.
// A data shard's row is that of the inverse of the survivors' k x k block of
// [I; C]; a parity shard's row is C[i] times that inverse.  False when fewer
// than k shards survive (or the block is singular, which a Cauchy code never is).
inline bool rs8_decode_rows(int k, int m, const bool* er, int* surv, int* outs, int* nout,
                            uint8_t* M) {
    uint8_t C[kRs8MaxM * kRs8MaxK];
    cauchy(k, m, C);
    int ns = 0;
    for (int s = 0; s < k + m && ns < k; ++s)
        if (!er[s]) surv[ns++] = s;
    if (ns < k) return false;
    uint8_t A[kRs8MaxK * kRs8MaxK], Ai[kRs8MaxK * kRs8MaxK];
    for (int q = 0; q < k; ++q)
        for (int j = 0; j < k; ++j)
            A[q * k + j] = surv[q] < k ? uint8_t(surv[q] == j) : C[(surv[q] - k) * k + j];
    if (!gf8_invert(k, A, Ai)) return false;
    int no = 0;
    for (int s = 0; s < k + m; ++s) {
        if (!er[s]) continue;
        for (int q = 0; q < k; ++q) {
            uint8_t v = 0;
            if (s < k) {
                v = Ai[s * k + q];
            } else {
                for (int j = 0; j < k; ++j) v ^= kGf8.mul(C[(s - k) * k + j], Ai[j * k + q]);
            }
            M[no * k + q] = v;
        }
        outs[no++] = s;
    }
    *nout = no;
    return true;
}

// Fields of four data bytes, shared by every coefficient they are multiplied by.
struct Gf8Fields {
    uint32_t f0, f1, f2;
};

__device__ __forceinline__ Gf8Fields gf8_fields(uint32_t w) {
    return Gf8Fields{w & 0x07070707u, (w >> 3) & 0x07070707u, (w >> 6) & 0x03030303u};
}

__device__ __forceinline__ uint32_t gf8_mul4(const Gf8Fields& f, const uint32_t* t) {
    return gf8_mul4(f.f0, f.f1, f.f2, t);
}

// acc ^ x*c for four bytes: three v_perm_b32 and two 3-input XORs.
__device__ __forceinline__ uint32_t gf8_fma4(uint32_t acc, const Gf8Fields& f, const uint32_t* t) {
    const uint32_t p0 = __builtin_amdgcn_perm(t[1], t[0], f.f0);
    const uint32_t p1 = __builtin_amdgcn_perm(t[3], t[2], f.f1);
    const uint32_t p2 = __builtin_amdgcn_perm(t[5], t[4], f.f2);
    return xor3(xor3(acc, p0, p1), p2, 0u);
}

// acc ^ x*c for a 16-byte cell.
__device__ __forceinline__ u32x4 gf8_fma16(u32x4 acc, const Gf8Fields* f, const uint32_t* t) {
    return u32x4{gf8_fma4(acc.x, f[0], t), gf8_fma4(acc.y, f[1], t), gf8_fma4(acc.z, f[2], t),
                 gf8_fma4(acc.w, f[3], t)};
}

__device__ __forceinline__ void gf8_fields16(u32x4 x, Gf8Fields* f) {
    f[0] = gf8_fields(x.x);
    f[1] = gf8_fields(x.y);
    f[2] = gf8_fields(x.z);
    f[3] = gf8_fields(x.w);
}

}  // namespace kvec
