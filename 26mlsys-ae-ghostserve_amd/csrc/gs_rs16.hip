// gs_rs16.hip -- the reference's Reed-Solomon code over GF(2^16), bit-exact
// (benchmark/rs/kernel.cu:16-222), on its packed [(k+m), S] u16 tensors.
//
// Multiplication uses the caller's log/exp tables exactly as the reference's
// gf_mul does, but only to build per-block lookup tables: for a constant c,
// x*c = T_lo[x & 0xFF] ^ T_hi[x >> 8] with T_lo[v] = gf_mul(v, c) and
// T_hi[v] = gf_mul(v << 8, c) (the field product is GF(2)-bilinear), so the
// streaming loop does two LDS lookups per symbol and coefficient instead of
// three dependent global-table gathers.
//
// Reconstruction folds the reference's two steps (right-hand side b, then
// x = V^-1 b) into one coefficient per (output, input) pair: exact in the
// field, so the bytes are those of the two-step computation.  The inverse is
// computed per block with the reference's Gauss-Jordan (pivot order and
// zero-pivot skip included), from indices read on the device.
#include "tile_engine.h"

namespace kvec {

constexpr int kGfOrder = 65535;
constexpr int kRsMaxM = 16;           // reference limit (benchmark/rs/kernel.cu:118)
constexpr int kRsMaxTables = 48;      // coefficient tables held in LDS (48 KiB)
constexpr int kRsGrid = 2048;         // persistent blocks: tables are built once per block

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
};

// Products of the input symbols with the coefficient table set `tab`
// ([nout][nin][2][256] u16 in LDS) for 8 logical words of output o.
__device__ __forceinline__ u32x4 rs_mix_window(const RsJob& j, const uint16_t* tab, int o,
                                               int64_t w0) {
    uint32_t acc[4] = {0, 0, 0, 0};
    for (int i = 0; i < j.nin; ++i) {
        const u32x4 x = load_window16(reinterpret_cast<const uint8_t*>(j.in_rows[i] + w0));
        const uint16_t* tl = tab + (size_t(o) * j.nin + i) * 512;
        const uint16_t* th = tl + 256;
        const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t v = xs[q];
            const uint32_t lo = tl[v & 0xFF] ^ th[(v >> 8) & 0xFF];
            const uint32_t hi = tl[(v >> 16) & 0xFF] ^ th[v >> 24];
            acc[q] ^= lo | (hi << 16);
        }
    }
    return u32x4{acc[0], acc[1], acc[2], acc[3]};
}

__device__ __forceinline__ uint16_t rs_mix_word(const RsJob& j, const uint16_t* tab, int o,
                                                int64_t w) {
    uint16_t a = 0;
    for (int i = 0; i < j.nin; ++i) {
        const uint16_t x = j.in_rows[i][w];
        const uint16_t* tl = tab + (size_t(o) * j.nin + i) * 512;
        a ^= tl[x & 0xFF] ^ tl[256 + (x >> 8)];
    }
    return a;
}

// Stream every tile of the job through the tables already in LDS.
__device__ void rs_run_tiles(const RsJob& j, const uint16_t* tab, uint8_t* tile) {
    const uint64_t Sb = uint64_t(j.S) * 2;
    const uint64_t ntiles = (Sb + kTileBytes - 1) / kTileBytes;
    for (uint64_t tt = blockIdx.x; tt < ntiles; tt += gridDim.x) {
        const uint64_t t0b = tt * kTileBytes;
        const uint32_t nbytes = uint32_t(Sb - t0b < uint64_t(kTileBytes) ? Sb - t0b : kTileBytes);
        const int64_t w0 = int64_t(t0b / 2) + 8 * threadIdx.x;
        for (int o = 0; o < j.nout; ++o) {
            u32x4 acc = {0, 0, 0, 0};
            if (w0 + 8 <= j.S) {
                acc = rs_mix_window(j, tab, o, w0);
            } else if (w0 < j.S) {
                for (int q = 0; q < int(j.S - w0); ++q) {
                    const uint16_t a = rs_mix_word(j, tab, o, w0 + q);
                    acc = set_byte(set_byte(acc, 2 * q, uint8_t(a)), 2 * q + 1, uint8_t(a >> 8));
                }
            }
            *reinterpret_cast<u32x4*>(tile + 16 * threadIdx.x) = acc;
            __syncthreads();
            tile_store(reinterpret_cast<uint8_t*>(j.out_rows[o]) + t0b, tile, nbytes);
            __syncthreads();
        }
    }
}

// Fill the [nout][nin] byte-split tables for coefficient matrix `coef` (LDS).
__device__ void rs_build_tables(uint16_t* tab, const uint16_t* coef, int nout, int nin,
                                const uint16_t* ex, const uint16_t* lg) {
    const int n = nout * nin * 512;
    for (int e = threadIdx.x; e < n; e += kTB) {
        const int t = e >> 9, half = (e >> 8) & 1, v = e & 0xFF;
        const uint16_t x = half ? uint16_t(v << 8) : uint16_t(v);
        tab[e] = gf16_mul_tab(x, coef[t], ex, lg);
    }
}

// benchmark/rs/kernel.cu:67-102 parity: Par_p = XOR_i D_i * alpha^((p+1) i mod 65535).
__global__ __launch_bounds__(kTB) void rs16_encode_kernel(RsJob job, const uint16_t* ex,
                                                          const uint16_t* lg) {
    __shared__ __attribute__((aligned(16))) uint16_t tab[kRsMaxTables * 512];
    __shared__ uint16_t coef[kRsMaxTables];
    __shared__ __attribute__((aligned(16))) uint8_t tile[kTileBytes + 16];
    __shared__ RsJob j;
    if (threadIdx.x == 0) j = job;
    __syncthreads();
    for (int t = threadIdx.x; t < j.nout * j.nin; t += kTB) {
        const int p = t / j.nin, i = t % j.nin;
        coef[t] = ex[((p + 1) * i) % kGfOrder];
    }
    __syncthreads();
    rs_build_tables(tab, coef, j.nout, j.nin, ex, lg);
    __syncthreads();
    rs_run_tiles(j, tab, tile);
}

// benchmark/rs/kernel.cu:105-222 with the right-hand side folded into the
// coefficients.  Inputs: the k - m surviving data rows, then the m parity rows
// of parity_used; outputs: the m missing data rows.
__global__ __launch_bounds__(kTB) void rs16_reconstruct_kernel(uint16_t* sh, int64_t S, int k,
                                                               int mpar, int m,
                                                               const int32_t* missing,
                                                               const int32_t* pused,
                                                               const uint16_t* ex,
                                                               const uint16_t* lg) {
    __shared__ __attribute__((aligned(16))) uint16_t tab[kRsMaxTables * 512];
    __shared__ uint16_t coef[kRsMaxTables];
    __shared__ uint16_t inv[kRsMaxM * kRsMaxM];
    __shared__ int s_miss[kRsMaxM], s_pu[kRsMaxM];
    __shared__ int s_ok;
    __shared__ __attribute__((aligned(16))) uint8_t tile[kTileBytes + 16];
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
    rs_build_tables(tab, coef, m, nin, ex, lg);
    __syncthreads();
    rs_run_tiles(j, tab, tile);
}

static int rs_grid(int64_t S) {
    const int64_t tiles = (S * 2 + kTileBytes - 1) / kTileBytes;
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
    hipError_t e = hipSuccess;
    if (N_k) e = hipMemcpyAsync(out, k, uint64_t(N_k) * 2, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess && N_v)
        e = hipMemcpyAsync((uint16_t*)out + N_k, v, uint64_t(N_v) * 2, hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return set_error(KVEC_EHIP, "kvec_rs16_pack: %s", hipGetErrorString(e));
    return KVEC_OK;
}

// u16_to_fp16_split, benchmark/rs/kernel.cu:245-263: inverse of the pack.
extern "C" int kvec_rs16_split(const void* in, void* k_out, void* v_out, int64_t N_k, int64_t N_v,
                               void* stream) {
    if (N_k < 0 || N_v < 0) return set_error(KVEC_EINVAL, "kvec_rs16_split: negative size");
    if ((N_k && (!in || !k_out)) || (N_v && (!in || !v_out)))
        return set_error(KVEC_EINVAL, "kvec_rs16_split: null pointer");
    hipStream_t st = as_stream(stream);
    hipError_t e = hipSuccess;
    if (N_k) e = hipMemcpyAsync(k_out, in, uint64_t(N_k) * 2, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess && N_v)
        e = hipMemcpyAsync(v_out, (const uint16_t*)in + N_k, uint64_t(N_v) * 2, hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return set_error(KVEC_EHIP, "kvec_rs16_split: %s", hipGetErrorString(e));
    return KVEC_OK;
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
    hipError_t e = hipMemcpyAsync(shards, data_padded, uint64_t(data_shards) * S * 2,
                                  hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return set_error(KVEC_EHIP, "kvec_rs16_encode: %s", hipGetErrorString(e));
    if (parity_shards == 0) return KVEC_OK;
    RsJob j{};
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
