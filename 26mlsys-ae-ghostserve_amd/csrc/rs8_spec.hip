// rs8_spec.hip -- systematic Reed-Solomon over GF(2^8) (poly 0x11D) with the
// Cauchy parity block C[i][j] = 1 / ((k+i) ^ j), i < m, j < k.
//
// Encode and decode are the same operation: out_o = XOR_j M[o][j] * in_j over
// separate shard buffers, with M = C for encode and, for decode, the rows of
// the inverse of the surviving k x k block of [I; C] (and C times it for an
// erased parity shard), computed on the host.
//
// The constant multiply is the v_perm_b32 split-table product of gf8.h.  Per 4
// data bytes: 5 ops to extract the fields (shared by all outputs) and 3 v_perm
// + 3 XOR per coefficient, with the tables held in registers -- no LDS or
// memory lookups.
#include "gf8.h"

namespace kvec {

// The coefficient tables are staged in LDS and read at their point of use:
// held in SGPRs from the kernel arguments, 6*k*m dwords next to the shard
// buffer resources overflow the SGPR file and get spilled (and kernels that
// spilled SGPRs have given run-to-run different results).
template <int NIN, int NOUT, int V>
__global__ __launch_bounds__(kRs8BS) void gf8_mix_kernel(Ptrs<kRs8MaxK> in, Ptrs<kRs8MaxM> out,
                                                         Gf8Mix mix, uint32_t S, uint32_t nvec) {
    __shared__ uint32_t lds_tab[NIN * NOUT][6];
    for (int i = threadIdx.x; i < NIN * NOUT * 6; i += kRs8BS) lds_tab[i / 6][i % 6] = mix.t[i / 6][i % 6];
    __syncthreads();
    auto tab = [&](int c) -> const uint32_t* { return lds_tab[c]; };
    const uint32_t u0 = blockIdx.x * (kRs8BS * V) + threadIdx.x;
    u32x4 acc[V][NOUT];
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
        for (int o = 0; o < NOUT; ++o) acc[v][o] = u32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < NIN; ++j) {
        const ShardView<true> sv(in.p[j], S);
        u32x4 x[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const uint32_t u = u0 + v * kRs8BS;
            x[v] = sv.load(0, (u < nvec ? u : 0u) << 4);
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
            Gf8Fields f[4];
            gf8_fields16(x[v], f);
#pragma unroll
            for (int o = 0; o < NOUT; ++o) acc[v][o] = gf8_fma16(acc[v][o], f, tab(o * NIN + j));
        }
    }
#pragma unroll
    for (int o = 0; o < NOUT; ++o) {
        const ShardView<true> so(out.p[o], S);
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const uint32_t u = u0 + v * kRs8BS;
            if (u < nvec) so.store(0, u << 4, acc[v][o]);
        }
    }
}

// Any shape: one output at a time, inputs re-read through L2.
__global__ __launch_bounds__(kRs8BS) void gf8_mix_generic_kernel(Ptrs<kRs8MaxK> in,
                                                                 Ptrs<kRs8MaxM> out, Gf8Mix mix,
                                                                 int nin, int nout, uint64_t S,
                                                                 uint64_t nvec) {
    const uint64_t u = uint64_t(blockIdx.x) * kRs8BS + threadIdx.x;
    if (u >= nvec) return;
    for (int o = 0; o < nout; ++o) {
        u32x4 acc = {0, 0, 0, 0};
        for (int j = 0; j < nin; ++j) {
            const u32x4 x = ld16(in.p[j] + (u << 4));
            const uint32_t w[4] = {x.x, x.y, x.z, x.w};
            uint32_t r[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                r[q] = gf8_mul4(w[q] & 0x07070707u, (w[q] >> 3) & 0x07070707u,
                                (w[q] >> 6) & 0x03030303u, mix.t[o * nin + j]);
            acc ^= u32x4{r[0], r[1], r[2], r[3]};
        }
        st_stream(out.p[o], u << 4, acc);
    }
    (void)S;
}

typedef void (*MixFn)(Ptrs<kRs8MaxK>, Ptrs<kRs8MaxM>, Gf8Mix, uint32_t, uint32_t);

template <int NIN, int NOUT>
constexpr int mix_vec() {
    return NIN * NOUT <= 12 ? 2 : 1;
}

#define KVEC_MIX(NIN, NOUT) \
    if (nin == NIN && nout == NOUT) return &gf8_mix_kernel<NIN, NOUT, mix_vec<NIN, NOUT>()>;

// Shapes of the stripe configurations (RS(6,2) encode and its 1/2-erasure
// decodes, RS(5,3) and its decodes, RS(4,2), RS(8,2), RS(10,4)) are compiled
// straight-line; other shapes run the generic kernel.
static MixFn mix_fn(int nin, int nout, int* vec) {
    auto pick = [&]() -> MixFn {
        KVEC_MIX(6, 1) KVEC_MIX(6, 2)
        KVEC_MIX(5, 1) KVEC_MIX(5, 2) KVEC_MIX(5, 3)
        KVEC_MIX(4, 1) KVEC_MIX(4, 2)
        KVEC_MIX(8, 1) KVEC_MIX(8, 2)
        KVEC_MIX(10, 1) KVEC_MIX(10, 2) KVEC_MIX(10, 3) KVEC_MIX(10, 4)
        return nullptr;
    };
    MixFn f = pick();
    *vec = (nin * nout <= 12) ? 2 : 1;
    return f;
}
#undef KVEC_MIX

static int launch_mix(uint8_t* const* in, int nin, uint8_t* const* out, int nout,
                      const uint8_t* M /* nout x nin */, int64_t S, hipStream_t st,
                      const char* what) {
    Ptrs<kRs8MaxK> pi{};
    Ptrs<kRs8MaxM> po{};
    Gf8Mix mix{};
    for (int j = 0; j < nin; ++j) pi.p[j] = in[j];
    for (int o = 0; o < nout; ++o) {
        po.p[o] = out[o];
        for (int j = 0; j < nin; ++j) perm_tables(M[o * nin + j], mix.t[o * nin + j]);
    }
    if (S == 0 || nout == 0) return KVEC_OK;
    int vec = 1;
    MixFn fn = fits_buffer(uint64_t(S)) ? mix_fn(nin, nout, &vec) : nullptr;
    if (fn) {
        const uint32_t nvec = uint32_t(S / 16);
        hipLaunchKernelGGL(fn, dim3(blocks_for(nvec, kRs8BS * vec)), dim3(kRs8BS), 0, st, pi, po, mix,
                           uint32_t(S), nvec);
    } else {
        const uint64_t nvec = uint64_t(S) / 16;
        hipLaunchKernelGGL(gf8_mix_generic_kernel, dim3(unsigned((nvec + kRs8BS - 1) / kRs8BS)),
                           dim3(kRs8BS), 0, st, pi, po, mix, nin, nout, uint64_t(S), nvec);
    }
    return check_launch(what);
}

static int check_rs8(int k, int m, int64_t S, const char* fn) {
    if (k < 1 || m < 0 || k > kRs8MaxK || m > kRs8MaxM || k * m > kRs8MaxCoef)
        return set_error(KVEC_EINVAL, "%s: k=%d m=%d (k <= %d, m <= %d, k*m <= %d)", fn, k, m, kRs8MaxK,
                         kRs8MaxM, kRs8MaxCoef);
    if (S < 0 || S % 16) return set_error(KVEC_EINVAL, "%s: shard_bytes=%lld must be a multiple of 16", fn,
                                          (long long)S);
    return KVEC_OK;
}

}  // namespace kvec

using namespace kvec;

extern "C" int kvec_rs8_cauchy(int k, int m, uint8_t* C) {
    if (k < 1 || m < 0 || k + m > 256 || !C) return set_error(KVEC_EINVAL, "kvec_rs8_cauchy: k=%d m=%d", k, m);
    cauchy(k, m, C);
    return KVEC_OK;
}

extern "C" int kvec_rs8_encode(const void* const* data, int k, void* const* parity, int m,
                               int64_t shard_bytes, void* stream) {
    int rc = check_rs8(k, m, shard_bytes, "kvec_rs8_encode");
    if (rc) return rc;
    if (m == 0) return KVEC_OK;
    if (!data || !parity) return set_error(KVEC_EINVAL, "kvec_rs8_encode: null pointer array");
    uint8_t* in[kRs8MaxK];
    uint8_t* out[kRs8MaxM];
    for (int j = 0; j < k; ++j) {
        if (!data[j] || !aligned16(data[j]))
            return set_error(KVEC_EINVAL, "kvec_rs8_encode: data[%d] null or not 16-byte aligned", j);
        in[j] = (uint8_t*)data[j];
    }
    for (int i = 0; i < m; ++i) {
        if (!parity[i] || !aligned16(parity[i]))
            return set_error(KVEC_EINVAL, "kvec_rs8_encode: parity[%d] null or not 16-byte aligned", i);
        out[i] = (uint8_t*)parity[i];
    }
    {
        Span w[kRs8MaxM], r[kRs8MaxK];
        for (int i = 0; i < m; ++i) w[i] = Span{out[i], uint64_t(shard_bytes), "parity", i};
        for (int j = 0; j < k; ++j) r[j] = Span{in[j], uint64_t(shard_bytes), "data", j};
        if ((rc = check_no_alias(w, m, r, k, "kvec_rs8_encode"))) return rc;
    }
    uint8_t C[kRs8MaxM * kRs8MaxK];
    cauchy(k, m, C);
    return launch_mix(in, k, out, m, C, shard_bytes, as_stream(stream), "kvec_rs8_encode");
}

extern "C" int kvec_rs8_decode(void* const* shards, int k, int m, int64_t shard_bytes,
                               const int32_t* erased, int n_erased, void* stream) {
    int rc = check_rs8(k, m, shard_bytes, "kvec_rs8_decode");
    if (rc) return rc;
    if (!shards || (n_erased > 0 && !erased))
        return set_error(KVEC_EINVAL, "kvec_rs8_decode: null pointer");
    bool er[kRs8MaxK + kRs8MaxM] = {};
    for (int q = 0; q < n_erased; ++q) {
        if (erased[q] < 0 || erased[q] >= k + m)
            return set_error(KVEC_EINVAL, "kvec_rs8_decode: erased index %d not in [0, %d)", erased[q], k + m);
        er[erased[q]] = true;
    }
    int ne = 0;
    for (int s = 0; s < k + m; ++s) {
        if (!shards[s] || !aligned16(shards[s]))
            return set_error(KVEC_EINVAL, "kvec_rs8_decode: shard %d null or not 16-byte aligned", s);
        ne += er[s];
    }
    if (ne == 0) return KVEC_OK;
    if (ne > m) return set_error(KVEC_EDECODE, "kvec_rs8_decode: %d erasures > m=%d", ne, m);
    {
        // the rebuilt shards must not share a byte with any other shard
        Span w[kRs8MaxM], r[kRs8MaxK + kRs8MaxM];
        int nw = 0, nr = 0;
        for (int s = 0; s < k + m; ++s)
            (er[s] ? w[nw++] : r[nr++]) = Span{shards[s], uint64_t(shard_bytes), "shard", s};
        if ((rc = check_no_alias(w, nw, r, nr, "kvec_rs8_decode"))) return rc;
    }
    int surv[kRs8MaxK], outs[kRs8MaxM], no = 0;
    uint8_t M[kRs8MaxM * kRs8MaxK];
    if (!rs8_decode_rows(k, m, er, surv, outs, &no, M))
        return set_error(KVEC_EDECODE, "kvec_rs8_decode: singular survivor block");
    uint8_t* in[kRs8MaxK];
    uint8_t* out[kRs8MaxM];
    for (int o = 0; o < no; ++o) out[o] = (uint8_t*)shards[outs[o]];
    for (int q = 0; q < k; ++q) in[q] = (uint8_t*)shards[surv[q]];
    return launch_mix(in, k, out, no, M, shard_bytes, as_stream(stream), "kvec_rs8_decode");
}
