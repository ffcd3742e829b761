// rdp_plan.h -- decode plans of textbook RDP over a prime p (Corbett et al.,
// FAST 2004), shared by the stripe and paged-pool decoders.
//
// Cells are numbered shard * (p-1) + row; shards 0..k-1 are data, k is the
// row parity P and k+1 the diagonal parity Q (diagonals 0..p-2 over columns
// 0..p-1, the P column being p-1; data columns k..p-2 are implicit zeros).
// An erasure pattern's decode is a fixed GF(2) linear map from the surviving
// cells to the erased ones; make_rdp_plan solves it by Gauss-Jordan over the
// code's row and diagonal equations (constexpr, so kernels can take it as a
// compile-time constant).
#pragma once

#include "kvec_internal.h"

namespace kvec {

constexpr int kRdpMaxP = 13;
constexpr int kRdpMaxRows = kRdpMaxP - 1;
constexpr int kRdpMaxShards = kRdpMaxP + 1;  // k+2 with k <= p-1
constexpr int kRdpMaxOut = 2 * kRdpMaxRows;
constexpr int kRdpNW = (kRdpMaxShards * kRdpMaxRows + 63) / 64;

typedef Ptrs<kRdpMaxShards> RdpPtrs;

// ---------------------------------------------------------------- decode plan
// Cells are numbered shard * (p-1) + row; shards 0..k-1 are data, k is P and
// k+1 is Q.  mask[o] lists the surviving cells whose XOR is output cell o.
struct RdpPlan {
    int ok;
    int nout;
    int out_cell[kRdpMaxOut];
    uint64_t mask[kRdpMaxOut][kRdpNW];
    uint64_t need[kRdpNW];
};

struct RdpEq {
    uint32_t um;            // unknowns (bit = index into the unknown list)
    uint64_t km[kRdpNW];    // known cells
};

constexpr void eq_add(RdpEq& e, int cell, const int* unk_of_cell) {
    if (unk_of_cell[cell] >= 0)
        e.um ^= 1u << unk_of_cell[cell];
    else
        e.km[cell >> 6] ^= uint64_t(1) << (cell & 63);
}

// Equations used (the same ones the peeling decoder of the oracle ends up
// using, so both give the same bytes even for inconsistent input):
//   rows      when a data or P column is erased,
//   diagonals when Q is erased or two non-Q columns are erased.
constexpr RdpPlan make_rdp_plan(int P, int K, int e0, int e1) {
    RdpPlan pl{};
    const int rows = P - 1, nsh = K + 2;
    if (P < 3 || P > kRdpMaxP || K < 1 || K > P - 1) return pl;
    if (e0 < -1 || e0 >= nsh || e1 < -1 || e1 >= nsh) return pl;
    bool er[kRdpMaxShards] = {};
    if (e0 >= 0) er[e0] = true;
    if (e1 >= 0) er[e1] = true;
    int unk_of_cell[kRdpMaxShards * kRdpMaxRows] = {};
    for (int c = 0; c < nsh * rows; ++c) unk_of_cell[c] = -1;
    int nu = 0;
    for (int s = 0; s < nsh; ++s)
        if (er[s])
            for (int r = 0; r < rows; ++r) {
                pl.out_cell[nu] = s * rows + r;
                unk_of_cell[s * rows + r] = nu++;
            }
    pl.nout = nu;
    if (nu == 0) {
        pl.ok = 1;
        return pl;
    }
    const bool q_er = er[K + 1];
    const int n_other = (er[K + 1] ? nu / rows - 1 : nu / rows);
    RdpEq eq[kRdpMaxOut] = {};
    int ne = 0;
    if (n_other >= 1)
        for (int r = 0; r < rows; ++r) {
            RdpEq e{};
            for (int j = 0; j < K; ++j) eq_add(e, j * rows + r, unk_of_cell);
            eq_add(e, K * rows + r, unk_of_cell);
            eq[ne++] = e;
        }
    if (q_er || n_other == 2)
        for (int d = 0; d < rows; ++d) {
            RdpEq e{};
            for (int j = 0; j < K; ++j) {
                const int r = ((d - j) % P + P) % P;
                if (r < rows) eq_add(e, j * rows + r, unk_of_cell);
            }
            const int rp = (d + 1) % P;  // P cell (rp, column p-1) lies on diagonal d
            if (rp < rows) eq_add(e, K * rows + rp, unk_of_cell);
            eq_add(e, (K + 1) * rows + d, unk_of_cell);
            eq[ne++] = e;
        }
    if (ne != nu) return pl;
    // Gauss-Jordan over GF(2) on the unknown part.
    for (int i = 0; i < nu; ++i) {
        int piv = -1;
        for (int e = i; e < ne; ++e)
            if ((eq[e].um >> i) & 1u) {
                piv = e;
                break;
            }
        if (piv < 0) return pl;
        if (piv != i) {
            RdpEq t = eq[i];
            eq[i] = eq[piv];
            eq[piv] = t;
        }
        for (int e = 0; e < ne; ++e)
            if (e != i && ((eq[e].um >> i) & 1u)) {
                eq[e].um ^= eq[i].um;
                for (int w = 0; w < kRdpNW; ++w) eq[e].km[w] ^= eq[i].km[w];
            }
    }
    for (int o = 0; o < nu; ++o)
        for (int w = 0; w < kRdpNW; ++w) {
            pl.mask[o][w] = eq[o].km[w];
            pl.need[w] |= eq[o].km[w];
        }
    pl.ok = 1;
    return pl;
}

// ---------------------------------------------------------------- XOR schedule
// The outputs of one pattern share most of their inputs (a decode chain
// rebuilds each cell from a neighbour's equation), so an output is cheapest as
// an earlier output XOR the cells where the two masks differ.  The order and
// bases form a minimum spanning tree (Prim) over the outputs plus a zero root,
// with edge weight = XORs needed: popcount(mask) - 1 from the root,
// popcount(mask_a ^ mask_b) between outputs.  For the p = 7 data pairs this
// takes the expanded map's ~200 cell terms per lane down to about a third.
struct RdpSched {
    int order[kRdpMaxOut];              // outputs in computation order
    int base[kRdpMaxOut];               // per output: the earlier output it extends, or -1
    uint64_t dmask[kRdpMaxOut][kRdpNW]; // per output: cells XORed onto its base
};

constexpr int mask_pop(const uint64_t* m) {
    int n = 0;
    for (int w = 0; w < kRdpNW; ++w) n += __builtin_popcountll(m[w]);
    return n;
}

constexpr int mask_dist(const uint64_t* a, const uint64_t* b) {
    int n = 0;
    for (int w = 0; w < kRdpNW; ++w) n += __builtin_popcountll(a[w] ^ b[w]);
    return n;
}

constexpr RdpSched make_rdp_sched(const RdpPlan& pl) {
    RdpSched s{};
    bool done[kRdpMaxOut] = {};
    int cost[kRdpMaxOut] = {}, par[kRdpMaxOut] = {};
    for (int o = 0; o < pl.nout; ++o) {
        cost[o] = mask_pop(pl.mask[o]) - 1;
        par[o] = -1;
    }
    for (int step = 0; step < pl.nout; ++step) {
        int o = -1;
        for (int i = 0; i < pl.nout; ++i)
            if (!done[i] && (o < 0 || cost[i] < cost[o])) o = i;
        done[o] = true;
        s.order[step] = o;
        s.base[o] = par[o];
        for (int w = 0; w < kRdpNW; ++w)
            s.dmask[o][w] = par[o] < 0 ? pl.mask[o][w] : pl.mask[o][w] ^ pl.mask[par[o]][w];
        for (int i = 0; i < pl.nout; ++i)
            if (!done[i]) {
                const int c = mask_dist(pl.mask[i], pl.mask[o]);
                if (c < cost[i]) {
                    cost[i] = c;
                    par[i] = o;
                }
            }
    }
    return s;
}

}  // namespace kvec
