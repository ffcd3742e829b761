/*
 * kvec_oracle.c -- CPU restatement of the GhostServe KV-cache erasure-coding
 * path.  TEST INFRASTRUCTURE ONLY (the reference for comparison, never the product): loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Citations are to the reference repository (project-ghostserve/
 * 26mlsys-AE-GhostServe).  The spec-family functions have no reference
 * counterpart; they restate Corbett et al., "Row-Diagonal Parity for Double
 * Disk Failure Correction" (FAST 2004) and the textbook systematic
 * Reed-Solomon construction with a Cauchy parity block.
 *
 * Pinning (which independent check fixes each function) is listed in the
 * header of tests/test_oracle.py.
 */
#include "kvec_oracle.h"

#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int kvo_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void kvo_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ======================================================================== */
/* Galois fields                                                            */
/* ======================================================================== */

/* benchmark/rs/main.py:39-54 -- LFSR walk of alpha^i with poly 0x1100B. */
void kvo_gf16_tables(uint16_t* gf_exp, uint16_t* gf_log) {
    const uint32_t poly = 0x1100B, size = 1u << 16, order = size - 1;
    memset(gf_log, 0, sizeof(uint16_t) * size);
    uint32_t x = 1;
    for (uint32_t i = 0; i < order; ++i) {
        gf_exp[i] = (uint16_t)x;
        gf_log[x] = (uint16_t)i;
        x <<= 1;
        if (x & size) x ^= poly;
    }
    for (uint32_t i = 0; i < order; ++i) gf_exp[order + i] = gf_exp[i];
}

static uint8_t g8_exp[510], g8_log[256];
static int g8_ready = 0;

void kvo_gf8_tables(uint8_t* gf_exp, uint8_t* gf_log) {
    uint32_t x = 1;
    memset(gf_log, 0, 256);
    for (int i = 0; i < 255; ++i) {
        gf_exp[i] = (uint8_t)x;
        gf_log[x] = (uint8_t)i;
        x <<= 1;
        if (x & 0x100) x ^= 0x11D;
    }
    for (int i = 0; i < 255; ++i) gf_exp[255 + i] = gf_exp[i];
}

static void g8_init(void) {
    if (!g8_ready) {
        kvo_gf8_tables(g8_exp, g8_log);
        g8_ready = 1;
    }
}

uint8_t kvo_gf8_mul(uint8_t a, uint8_t b) {
    g8_init();
    if (!a || !b) return 0;
    return g8_exp[g8_log[a] + g8_log[b]];
}

uint8_t kvo_gf8_inv(uint8_t a) {
    g8_init();
    if (!a) return 0;
    return g8_exp[255 - g8_log[a]];
}

int kvo_rs8_cauchy(int k, int m, uint8_t* C) {
    if (k <= 0 || m < 0 || k + m > 256) return -1;
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < k; ++j) C[i * k + j] = kvo_gf8_inv((uint8_t)((k + i) ^ j));
    return 0;
}

/* ======================================================================== */
/* gs family: XOR                                                           */
/* ======================================================================== */

/* benchmark/xor/kernel.cu:17-41 -- copy data rows, then P[j] = XOR_i data[i*S+j]. */
void kvo_xor_encode(const uint8_t* data_padded, uint8_t* shards, int data_shards,
                    int64_t S) {
    const int64_t total = (int64_t)data_shards * S;
    memcpy(shards, data_padded, (size_t)total);
#pragma omp parallel for schedule(static)
    for (int64_t off = 0; off < S; ++off) {
        uint8_t acc = 0;
        for (int k = 0; k < data_shards; ++k) acc ^= data_padded[(int64_t)k * S + off];
        shards[total + off] = acc;
    }
}

/* benchmark/xor/kernel.cu:47-88 -- single missing shard (data via P, or P). */
void kvo_xor_reconstruct(const uint8_t* enc, uint8_t* rec, uint8_t* rec_missing,
                         int64_t S, int nd, const int32_t* missing_indices,
                         int missing_count) {
    if (missing_count != 1) return;
    const int missing = missing_indices[0];
    if (missing >= 0 && missing < nd) {
#pragma omp parallel for schedule(static)
        for (int64_t off = 0; off < S; ++off) {
            uint8_t acc = enc[(int64_t)nd * S + off];
            for (int k = 0; k < nd; ++k)
                if (k != missing) acc ^= enc[(int64_t)k * S + off];
            rec[(int64_t)missing * S + off] = acc;
            rec_missing[off] = acc;
        }
        return;
    }
    if (missing == nd) {
#pragma omp parallel for schedule(static)
        for (int64_t off = 0; off < S; ++off) {
            uint8_t acc = 0;
            for (int k = 0; k < nd; ++k) acc ^= enc[(int64_t)k * S + off];
            rec[(int64_t)nd * S + off] = acc;
            rec_missing[off] = acc;
        }
    }
}

/* benchmark/xor/kernel.cu:93-119 -- fp16 words to little-endian byte pairs. */
void kvo_pack_kv(const uint16_t* k, const uint16_t* v, uint8_t* out, int n, int seq_len) {
    const int64_t total = (int64_t)seq_len * n;
    for (int64_t i = 0; i < total; ++i) {
        out[2 * i + 0] = (uint8_t)(k[i] & 0xFF);
        out[2 * i + 1] = (uint8_t)(k[i] >> 8);
        out[2 * total + 2 * i + 0] = (uint8_t)(v[i] & 0xFF);
        out[2 * total + 2 * i + 1] = (uint8_t)(v[i] >> 8);
    }
}

/* benchmark/xor/kernel.cu:122-146 -- inverse of kvo_pack_kv. */
void kvo_unpack_kv(const uint8_t* in, uint16_t* out, int n, int seq_len) {
    const int64_t total = (int64_t)seq_len * n;
    for (int64_t i = 0; i < total; ++i) {
        out[i] = (uint16_t)(in[2 * i] | (in[2 * i + 1] << 8));
        out[total + i] = (uint16_t)(in[2 * total + 2 * i] | (in[2 * total + 2 * i + 1] << 8));
    }
}

/* ======================================================================== */
/* gs family: RDP star-diagonal code                                        */
/* ======================================================================== */

/* benchmark/rdp/kernel.cu:19-25 */
static inline int64_t modS(int64_t x, int64_t S) {
    if (S <= 0) return 0;
    int64_t r = x % S;
    if (r < 0) r += S;
    return r;
}

/* benchmark/rdp/kernel.cu:32-72 -- shards.flat[pos] = (K_TN || V_TN)[pos] for
 * every pos whose row pos/S is a data row.  Words past 2*T*n are untouched. */
void kvo_gs_pack(const uint16_t* K, const uint16_t* V, uint16_t* shards, int nd, int S,
                 int T, int n) {
    if (T <= 0 || n <= 0 || nd <= 0 || S <= 0) return;
    for (int t = 0; t < T; ++t) {
        const int64_t baseK = (int64_t)t * n, baseV = (int64_t)T * n + (int64_t)t * n;
        for (int i = 0; i < n; ++i) {
            int64_t pk = baseK + i, pv = baseV + i;
            if (pk / S < nd) shards[pk] = K[(int64_t)t * n + i];
            if (pv / S < nd) shards[pv] = V[(int64_t)t * n + i];
        }
    }
}

/* benchmark/rdp/kernel.cu:76-107 (identical math in bench_ghostserve_rdp.py:121-150):
 * P[c] = XOR_r D_r[c];  Q[d] = XOR_r D_r[(d-r) mod S] except the row's star
 * column (star_base + r) % S.  That is C's truncating remainder: when
 * star_base + r is negative it is negative too and no column is skipped. */
void kvo_gs_parity(uint16_t* sh, int nd, int S, int star_base) {
    if (nd <= 0 || S <= 0) return;
    uint16_t* P = sh + (int64_t)nd * S;
    uint16_t* Q = sh + (int64_t)(nd + 1) * S;
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < S; ++c) {
        uint16_t acc = 0;
        for (int r = 0; r < nd; ++r) acc ^= sh[(int64_t)r * S + c];
        P[c] = acc;
    }
#pragma omp parallel for schedule(static)
    for (int64_t d = 0; d < S; ++d) {
        uint16_t acc = 0;
        for (int r = 0; r < nd; ++r) {
            int64_t c = modS(d - r, S);
            int star_r = (star_base + r) % S;
            if (c == star_r) continue;
            acc ^= sh[(int64_t)r * S + c];
        }
        Q[d] = acc;
    }
}

/* benchmark/rdp/kernel.cu:286-301 -- row t := P ^ XOR_{r != t} rows. */
static void gs_rebuild_from_P(uint16_t* sh, int nd, int S, int t) {
    const uint16_t* P = sh + (int64_t)nd * S;
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < S; ++c) {
        uint16_t acc = P[c];
        for (int r = 0; r < nd; ++r)
            if (r != t) acc ^= sh[(int64_t)r * S + c];
        sh[(int64_t)t * S + c] = acc;
    }
}

/* benchmark/rdp/kernel.cu:397-507 (recovery half of fused_recovery_full_kv).
 * Indices outside [0, nd) are dropped (:402-404).  With two distinct data rows
 * a < b the launcher runs the ring-walk kernels (:411-470), whose writes all
 * land in row a, and then rebuild_row_from_P(a) (:473-480), which rewrites
 * every column of row a, then rebuild_row_from_P(b) (:482-490).  Only the last
 * two writes are observable, so they are what is restated here. */
void kvo_gs_recover(uint16_t* sh, int nd, int S, int star_base, int a, int b) {
    /* star_base is read by the ring-walk kernels, whose output is dead, and by
     * fill_a_star_from_P (:268-282), which writes row a at column
     * (star_base + a) % S: for a non-negative remainder a cell that the
     * rebuild of row a rewrites, for a negative one (star_base + a < 0 and
     * not a multiple of S) an address outside row a, which the library
     * refuses and which is not restated here. */
    (void)star_base;
    a = (a >= 0 && a < nd) ? a : -1;
    b = (b >= 0 && b < nd) ? b : -1;
    if (a >= 0 && b >= 0 && a != b) {
        if (b < a) { int t = a; a = b; b = t; }
        gs_rebuild_from_P(sh, nd, S, a);
        gs_rebuild_from_P(sh, nd, S, b);
    } else if (a >= 0 && b < 0) {
        gs_rebuild_from_P(sh, nd, S, a); /* rdp_reconstruct_single_kernel :111-128 */
    } else if (b >= 0 && a < 0) {
        gs_rebuild_from_P(sh, nd, S, b);
    }
}

/* benchmark/rdp/kernel.cu:305-345 -- out[pos] = flat[pos] for pos < 2*T*n whose
 * row is a data row, else 0. */
void kvo_gs_load_full(const uint16_t* sh, uint16_t* out, int nd, int S, int T, int n) {
    if (T <= 0 || n <= 0 || nd <= 0 || S <= 0) return;
    const int64_t total = 2 * (int64_t)T * n;
    for (int64_t pos = 0; pos < total; ++pos) out[pos] = (pos / S < nd) ? sh[pos] : 0;
}

/* bench_ghostserve_rdp.py:105-118, :152-175 -- rows[row] = K || V words. */
int kvo_gs_pack_row(const uint16_t* k, const uint16_t* v, uint16_t* rows, int64_t words,
                    int row, int S) {
    if (S < 2 * words) return -1;
    uint16_t* rp = rows + (int64_t)row * S;
    memcpy(rp, k, (size_t)words * 2);
    memcpy(rp + words, v, (size_t)words * 2);
    return 0;
}

/* ======================================================================== */
/* gs family: RS over GF(2^16)                                              */
/* ======================================================================== */

static inline uint16_t g16_mul(uint16_t a, uint16_t b, const uint16_t* ex,
                               const uint16_t* lg) {
    /* benchmark/rs/kernel.cu:16-23 */
    if (a == 0 || b == 0) return 0;
    int s = (int)lg[a] + (int)lg[b];
    if (s >= 65535) s -= 65535;
    return ex[s];
}

static inline uint16_t g16_div(uint16_t a, uint16_t b, const uint16_t* ex,
                               const uint16_t* lg) {
    /* benchmark/rs/kernel.cu:25-33 */
    if (a == 0) return 0;
    if (b == 0) return 0;
    int d = (int)lg[a] - (int)lg[b];
    if (d < 0) d += 65535;
    return ex[d];
}

/* benchmark/rs/kernel.cu:67-102 -- copy data; Par_p[j] = XOR_i D_i[j]*alpha^((p+1)i). */
void kvo_rs16_encode(const uint16_t* data, uint16_t* shards, int k, int m, int64_t S,
                     const uint16_t* ex, const uint16_t* lg) {
    memcpy(shards, data, (size_t)((int64_t)k * S) * 2);
#pragma omp parallel for schedule(static)
    for (int64_t pos = 0; pos < S; ++pos) {
        for (int p = 0; p < m; ++p) {
            uint16_t acc = 0;
            const int base = p + 1;
            for (int i = 0; i < k; ++i) {
                uint16_t x = data[(int64_t)i * S + pos];
                if (x) acc ^= g16_mul(x, ex[(base * i) % 65535], ex, lg);
            }
            shards[((int64_t)k + p) * S + pos] = acc;
        }
    }
}

/* benchmark/rs/kernel.cu:135-185 -- Gauss-Jordan inverse of
 * V[r][c] = alpha^((pused_r+1) * missing_c), with the reference's pivot order
 * and its skip-on-zero-pivot behaviour. */
static void rs16_invert(int m, const int32_t* miss, const int32_t* pused, const uint16_t* ex,
                        const uint16_t* lg, uint16_t* inv) {
    uint16_t V[16 * 16];
    for (int r = 0; r < m; ++r)
        for (int c = 0; c < m; ++c) V[r * m + c] = ex[((pused[r] + 1) * miss[c]) % 65535];
    for (int r = 0; r < m; ++r)
        for (int c = 0; c < m; ++c) inv[r * m + c] = (r == c) ? 1 : 0;
    for (int i = 0; i < m; ++i) {
        int pr = i;
        while (pr < m && V[pr * m + i] == 0) ++pr;
        if (pr == m) continue;
        if (pr != i)
            for (int c = 0; c < m; ++c) {
                uint16_t t = V[i * m + c]; V[i * m + c] = V[pr * m + c]; V[pr * m + c] = t;
                t = inv[i * m + c]; inv[i * m + c] = inv[pr * m + c]; inv[pr * m + c] = t;
            }
        uint16_t piv = V[i * m + i];
        if (piv == 0) continue;
        uint16_t ip = g16_div(1, piv, ex, lg);
        for (int c = 0; c < m; ++c) {
            V[i * m + c] = g16_mul(V[i * m + c], ip, ex, lg);
            inv[i * m + c] = g16_mul(inv[i * m + c], ip, ex, lg);
        }
        for (int r = 0; r < m; ++r) {
            if (r == i) continue;
            uint16_t f = V[r * m + i];
            if (!f) continue;
            for (int c = 0; c < m; ++c) {
                V[r * m + c] ^= g16_mul(f, V[i * m + c], ex, lg);
                inv[r * m + c] ^= g16_mul(f, inv[i * m + c], ex, lg);
            }
        }
    }
}

/* benchmark/rs/kernel.cu:105-222 -- rebuild the m missing data shards in place
 * from the parities in parity_used; parity shards are never rewritten. */
int kvo_rs16_reconstruct(uint16_t* sh, int64_t S, int k, int mpar, const int32_t* miss,
                         int m, const int32_t* pused, const uint16_t* ex,
                         const uint16_t* lg) {
    (void)mpar;
    if (m == 0) return 0;
    if (m > 16) return -1;
    uint16_t inv[16 * 16];
    rs16_invert(m, miss, pused, ex, lg, inv);
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < S; ++t) {
        uint16_t b[16];
        for (int r = 0; r < m; ++r) {
            const int pr = pused[r];
            uint16_t acc = sh[((int64_t)k + pr) * S + t];
            const int base = pr + 1;
            for (int i = 0; i < k; ++i) {
                int is_m = 0;
                for (int mi = 0; mi < m; ++mi)
                    if (i == miss[mi]) { is_m = 1; break; }
                if (is_m) continue;
                uint16_t x = sh[(int64_t)i * S + t];
                if (x) acc ^= g16_mul(x, ex[(base * i) % 65535], ex, lg);
            }
            b[r] = acc;
        }
        uint16_t x[16];
        for (int c = 0; c < m; ++c) {
            uint16_t s = 0;
            for (int r = 0; r < m; ++r) s ^= g16_mul(inv[c * m + r], b[r], ex, lg);
            x[c] = s;
        }
        for (int c = 0; c < m; ++c) sh[(int64_t)miss[c] * S + t] = x[c];
    }
    return 0;
}

/* ======================================================================== */
/* spec family: textbook RDP (Corbett et al., FAST 2004)                    */
/* ======================================================================== */

static int is_prime(int p) {
    if (p < 2) return 0;
    for (int q = 2; q * q <= p; ++q)
        if (p % q == 0) return 0;
    return 1;
}

static inline void xor_into(uint8_t* restrict dst, const uint8_t* restrict src, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] ^= src[i];
}

/* Columns 0..p-2 hold data (k..p-2 are all-zero when k < p-1), column p-1 is
 * the row parity P and Q[d] is the XOR of diagonal d = (row + col) mod p over
 * columns 0..p-1, for d = 0..p-2 (diagonal p-1 is not stored).  Each byte
 * offset of a row plane is an independent RDP instance. */
/* Columns [o0, o0 + n) of one stripe whose p-1 rows are R bytes apart. */
static void rdp_encode_cols(const uint8_t* const* data, int k, uint8_t* P, uint8_t* Q, int p,
                            int64_t R, int64_t o0, int64_t n) {
    const int rows = p - 1;
    for (int r = 0; r < rows; ++r) {
        memset(P + r * R + o0, 0, (size_t)n);
        memset(Q + r * R + o0, 0, (size_t)n);
    }
    for (int j = 0; j < k; ++j)
        for (int r = 0; r < rows; ++r) {
            const uint8_t* src = data[j] + r * R + o0;
            xor_into(P + r * R + o0, src, n);
            const int d = (r + j) % p;
            if (d != p - 1) xor_into(Q + d * R + o0, src, n);
        }
    for (int r = 0; r < rows; ++r) {
        const int d = (r + p - 1) % p;
        if (d != p - 1) xor_into(Q + d * R + o0, P + r * R + o0, n);
    }
}

int kvo_rdp_encode(const uint8_t* const* data, int k, uint8_t* P, uint8_t* Q, int p,
                   int64_t R) {
    if (!is_prime(p) || p < 3 || k < 1 || k > p - 1 || R < 0) return -1;
    const int64_t BLK = 1 << 14;
#pragma omp parallel for schedule(static)
    for (int64_t o0 = 0; o0 < R; o0 += BLK)
        rdp_encode_cols(data, k, P, Q, p, R, o0, (R - o0 < BLK) ? R - o0 : BLK);
    return 0;
}

/* Decode by peeling: the p-1 row equations (XOR of columns 0..p-1 is zero)
 * and the p-1 stored diagonal equations (XOR of the diagonal's cells over
 * columns 0..p-1, plus Q[d], is zero) are solved one at a time whenever an
 * equation has a single unknown cell.  For RDP every pattern of at most two
 * erased columns peels completely (this is the row/diagonal chain walk of the
 * paper).  The schedule depends only on the erasure pattern, so it is found
 * once on the cell grid and then run on whole row planes. */
int kvo_rdp_decode(uint8_t* const* cols, int k, int p, int64_t R, int e0, int e1) {
    if (!is_prime(p) || p < 3 || p > 31 || k < 1 || k > p - 1 || R < 0) return -1;
    if (e0 < -1 || e0 > k + 1 || e1 < -1 || e1 > k + 1) return -2;
    const int rows = p - 1;
    /* textbook column index of shard s */
    int tc[2] = {-1, -1};
    int ne = 0;
    int es[2] = {e0, e1};
    for (int q = 0; q < 2; ++q) {
        if (es[q] < 0) continue;
        int c = es[q] < k ? es[q] : (es[q] == k ? p - 1 : p);
        if (ne == 1 && tc[0] == c) continue;
        tc[ne++] = c;
    }
    if (ne == 0) return 0;
    /* known[c][r]; columns 0..p (p is Q) */
    int known[32][32];
    for (int c = 0; c <= p; ++c)
        for (int r = 0; r < rows; ++r) known[c][r] = 1;
    for (int q = 0; q < ne; ++q)
        for (int r = 0; r < rows; ++r) known[tc[q]][r] = 0;
    /* pointer to a cell's row plane, NULL for a virtual zero column */
#define CELL(c, r)                                                              \
    ((c) < k ? cols[(c)] + (int64_t)(r) * R                                     \
             : ((c) < p - 1 ? (uint8_t*)0                                       \
                            : ((c) == p - 1 ? cols[k] + (int64_t)(r) * R        \
                                            : cols[k + 1] + (int64_t)(r) * R)))
    int remaining = ne * rows;
    while (remaining > 0) {
        int progress = 0;
        /* equations: e < rows -> row e; else diagonal e - rows */
        for (int e = 0; e < 2 * rows; ++e) {
            int cc[64], rr[64], n = 0, unk = -1, nunk = 0;
            if (e < rows) {
                for (int c = 0; c <= p - 1; ++c) { cc[n] = c; rr[n] = e; ++n; }
            } else {
                const int d = e - rows;
                for (int c = 0; c <= p - 1; ++c) {
                    int r = ((d - c) % p + p) % p;
                    if (r < rows) { cc[n] = c; rr[n] = r; ++n; }
                }
                cc[n] = p; rr[n] = d; ++n;
            }
            for (int t = 0; t < n; ++t)
                if (!known[cc[t]][rr[t]]) { ++nunk; unk = t; }
            if (nunk != 1) continue;
            uint8_t* dst = CELL(cc[unk], rr[unk]);
            memset(dst, 0, (size_t)R);
            for (int t = 0; t < n; ++t) {
                if (t == unk) continue;
                const uint8_t* src = CELL(cc[t], rr[t]);
                if (src) xor_into(dst, src, R);
            }
            known[cc[unk]][rr[unk]] = 1;
            --remaining;
            progress = 1;
        }
        if (!progress) return -3;
    }
#undef CELL
    return 0;
}

/* Striped geometry: each shard of (p-1)*R bytes is cut into stripes of
 * (p-1)*U bytes (the last one shorter when U does not divide R); stripe s has
 * rows of g_s = min(U, R - s*U) bytes, row r at s*(p-1)*U + r*g_s, and is coded
 * on its own.  U = 0 or U >= R is the single-stripe layout above. */
#define KVO_MAX_STRIPE_SHARDS 64
int kvo_rdp_encode_striped(const uint8_t* const* data, int k, uint8_t* P, uint8_t* Q, int p,
                           int64_t R, int64_t U) {
    if (U <= 0 || U >= R) return kvo_rdp_encode(data, k, P, Q, p, R);
    if (!is_prime(p) || p < 3 || k < 1 || k > p - 1 || k > KVO_MAX_STRIPE_SHARDS) return -1;
    const int rows = p - 1;
    const int64_t ns = (R + U - 1) / U;
    /* stripes are independent codes: one per thread at a time */
#pragma omp parallel for schedule(static)
    for (int64_t s = 0; s < ns; ++s) {
        const int64_t base = s * rows * U, g = (R - s * U < U) ? R - s * U : U;
        const uint8_t* d[KVO_MAX_STRIPE_SHARDS];
        for (int j = 0; j < k; ++j) d[j] = data[j] + base;
        rdp_encode_cols(d, k, P + base, Q + base, p, g, 0, g);
    }
    return 0;
}

int kvo_rdp_decode_striped(uint8_t* const* cols, int k, int p, int64_t R, int64_t U, int e0,
                           int e1) {
    if (U <= 0 || U >= R) return kvo_rdp_decode(cols, k, p, R, e0, e1);
    if (k < 1 || k + 2 > KVO_MAX_STRIPE_SHARDS) return -1;
    const int rows = p - 1;
    const int64_t ns = (R + U - 1) / U;
    int rc = 0;
#pragma omp parallel for schedule(static) reduction(|: rc)
    for (int64_t s = 0; s < ns; ++s) {
        const int64_t base = s * rows * U, g = (R - s * U < U) ? R - s * U : U;
        uint8_t* c[KVO_MAX_STRIPE_SHARDS];
        for (int j = 0; j < k + 2; ++j) c[j] = cols[j] + base;
        rc |= kvo_rdp_decode(c, k, p, g, e0, e1) != 0;
    }
    return rc ? -3 : 0;
}

/* ======================================================================== */
/* spec family: RS over GF(2^8), systematic Cauchy                          */
/* ======================================================================== */

int kvo_rs8_encode(const uint8_t* const* data, int k, uint8_t* const* parity, int m,
                   int64_t S) {
    uint8_t C[256 * 256 / 4];
    if (k <= 0 || m < 0 || k + m > 256 || (int64_t)k * m > (int64_t)sizeof C) return -1;
    kvo_rs8_cauchy(k, m, C);
    g8_init();
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < S; ++o) {
        for (int i = 0; i < m; ++i) {
            uint8_t acc = 0;
            for (int j = 0; j < k; ++j) {
                const uint8_t x = data[j][o], c = C[i * k + j];
                if (x && c) acc ^= g8_exp[g8_log[x] + g8_log[c]];
            }
            parity[i][o] = acc;
        }
    }
    return 0;
}

/* Decode: the first k surviving shards in index order give k equations
 * G_s . d = shard_s in the k data symbols (G = [I; C]); they are solved by
 * Gauss-Jordan elimination on the augmented k x (k+1) system for every byte
 * offset, then any erased parity shard is re-encoded from the recovered data. */
int kvo_rs8_decode(uint8_t* const* sh, int k, int m, int64_t S, const int32_t* erased,
                   int ne) {
    if (k <= 0 || m < 0 || k + m > 64) return -1;
    int is_er[64] = {0};
    for (int q = 0; q < ne; ++q) {
        if (erased[q] < 0 || erased[q] >= k + m) return -2;
        is_er[erased[q]] = 1;
    }
    int nerased = 0;
    for (int s = 0; s < k + m; ++s) nerased += is_er[s];
    if (nerased == 0) return 0;
    if (nerased > m) return -3;
    uint8_t C[64 * 64];
    kvo_rs8_cauchy(k, m, C);
    int surv[64], ns = 0;
    for (int s = 0; s < k + m && ns < k; ++s)
        if (!is_er[s]) surv[ns++] = s;
    /* coefficient rows of the chosen survivors */
    uint8_t A[64 * 64];
    for (int q = 0; q < k; ++q)
        for (int j = 0; j < k; ++j)
            A[q * k + j] = surv[q] < k ? (uint8_t)(surv[q] == j) : C[(surv[q] - k) * k + j];
    int any_data = 0;
    for (int j = 0; j < k; ++j) any_data |= is_er[j];
    if (any_data) {
#pragma omp parallel for schedule(static)
        for (int64_t o = 0; o < S; ++o) {
            uint8_t M[64 * 65];
            for (int q = 0; q < k; ++q) {
                for (int j = 0; j < k; ++j) M[q * (k + 1) + j] = A[q * k + j];
                M[q * (k + 1) + k] = sh[surv[q]][o];
            }
            for (int col = 0; col < k; ++col) {
                int piv = col;
                while (piv < k && M[piv * (k + 1) + col] == 0) ++piv;
                if (piv != col)
                    for (int c = 0; c <= k; ++c) {
                        uint8_t t = M[col * (k + 1) + c];
                        M[col * (k + 1) + c] = M[piv * (k + 1) + c];
                        M[piv * (k + 1) + c] = t;
                    }
                const uint8_t ip = kvo_gf8_inv(M[col * (k + 1) + col]);
                for (int c = 0; c <= k; ++c)
                    M[col * (k + 1) + c] = kvo_gf8_mul(M[col * (k + 1) + c], ip);
                for (int q = 0; q < k; ++q) {
                    if (q == col) continue;
                    const uint8_t f = M[q * (k + 1) + col];
                    if (!f) continue;
                    for (int c = 0; c <= k; ++c)
                        M[q * (k + 1) + c] ^= kvo_gf8_mul(f, M[col * (k + 1) + c]);
                }
            }
            for (int j = 0; j < k; ++j)
                if (is_er[j]) sh[j][o] = M[j * (k + 1) + k];
        }
    }
    /* re-encode erased parity rows from the (now complete) data */
    for (int i = 0; i < m; ++i) {
        if (!is_er[k + i]) continue;
#pragma omp parallel for schedule(static)
        for (int64_t o = 0; o < S; ++o) {
            uint8_t acc = 0;
            for (int j = 0; j < k; ++j) acc ^= kvo_gf8_mul(C[i * k + j], sh[j][o]);
            sh[k + i][o] = acc;
        }
    }
    return 0;
}

/* ======================================================================== */
/* paged KV gather                                                          */
/* ======================================================================== */

/* Semantics of the delta gather K = pool[slots, 0], V = pool[slots, 1]
 * (bench_ghostserve_rdp.py:445-458), with slots taken from a page table of
 * page_tokens-token pages: slot(b, t) = table[b][t / page_tokens] * page_tokens
 * + t % page_tokens.  The stream holds, per layer and sequence, the token
 * records (K then V, as stored in the pool) of positions tok_off.. in order:
 * [L][B][T][2][tok_bytes]. */
int kvo_kv_gather(const uint8_t* pool, int64_t pool_pages, int L, int64_t tb,
                  int page_tokens, const int32_t* pt, int B, int pps, int tok_off, int T,
                  uint8_t* stream) {
    if (L <= 0 || tb <= 0 || page_tokens <= 0 || B <= 0 || T < 0 || tok_off < 0) return -1;
    if ((int64_t)(tok_off + T) > (int64_t)pps * page_tokens) return -2;
    for (int b = 0; b < B; ++b)
        for (int j = 0; j < pps; ++j)
            if (pt[(int64_t)b * pps + j] < 0 || pt[(int64_t)b * pps + j] >= pool_pages)
                return -3;
    const int64_t layer_pool = pool_pages * page_tokens * 2 * tb;
#pragma omp parallel for collapse(2) schedule(static)
    for (int l = 0; l < L; ++l)
        for (int b = 0; b < B; ++b)
            for (int t = 0; t < T; ++t) {
                const int tt = tok_off + t;
                const int64_t slot =
                    (int64_t)pt[(int64_t)b * pps + tt / page_tokens] * page_tokens +
                    tt % page_tokens;
                for (int kv = 0; kv < 2; ++kv) {
                    const uint8_t* src = pool + l * layer_pool + (slot * 2 + kv) * tb;
                    uint8_t* dst =
                        stream + ((((int64_t)l * B + b) * (int64_t)T + t) * 2 + kv) * tb;
                    memcpy(dst, src, (size_t)tb);
                }
            }
    return 0;
}
