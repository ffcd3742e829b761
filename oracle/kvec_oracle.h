/*
 * kvec_oracle.h -- CPU restatement of the GhostServe KV-cache erasure-coding
 * path.  TEST INFRASTRUCTURE ONLY: the HIP kernels are compared against this
 * library.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links it.
 *
 * Two codec families:
 *   "gs"   -- bit-exact restatements of the reference kernels
 *             (benchmark/xor/kernel.cu, benchmark/rdp/kernel.cu,
 *              benchmark/rs/kernel.cu, bench_ghostserve_rdp.py:105-150).
 *   "spec" -- textbook RDP over a prime p (Corbett et al., FAST 2004) and
 *             Reed-Solomon over GF(2^8)/0x11D with a Cauchy generator.
 *
 * Every function returns 0 on success and a negative value on bad arguments
 * (or void when the reference kernel has no failure mode).
 */
#ifndef KVEC_ORACLE_H
#define KVEC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- Galois fields ---------------- */
/* GF(2^16), poly 0x1100B, alpha = 2; exp has 2*65535 entries, log 65536
 * (benchmark/rs/main.py:39-54). */
void kvo_gf16_tables(uint16_t* gf_exp, uint16_t* gf_log);
/* GF(2^8), poly 0x11D, alpha = 2; exp has 510 entries, log 256. */
void kvo_gf8_tables(uint8_t* gf_exp, uint8_t* gf_log);
uint8_t kvo_gf8_mul(uint8_t a, uint8_t b);
uint8_t kvo_gf8_inv(uint8_t a);
/* Systematic Cauchy parity block C[i][j] = inv((k+i) ^ j), i<m, j<k. */
int kvo_rs8_cauchy(int k, int m, uint8_t* C);

/* ---------------- gs family: XOR (benchmark/xor/kernel.cu) ---------------- */
void kvo_xor_encode(const uint8_t* data_padded, uint8_t* shards, int data_shards,
                    int64_t shard_size);
void kvo_xor_reconstruct(const uint8_t* encoded, uint8_t* recovered,
                         uint8_t* recovered_missing, int64_t shard_size,
                         int data_shards, const int32_t* missing_indices,
                         int missing_count);
void kvo_pack_kv(const uint16_t* k, const uint16_t* v, uint8_t* kv_bytes, int n,
                 int seq_len);
void kvo_unpack_kv(const uint8_t* kv_bytes, uint16_t* out, int n, int seq_len);

/* ---------------- gs family: RDP star-diagonal (benchmark/rdp/kernel.cu) ---- */
void kvo_gs_pack(const uint16_t* K_TN, const uint16_t* V_TN, uint16_t* shards,
                 int nd, int S, int T, int n);
void kvo_gs_parity(uint16_t* shards, int nd, int S, int star_base);
void kvo_gs_recover(uint16_t* shards, int nd, int S, int star_base, int miss_a,
                    int miss_b);
void kvo_gs_load_full(const uint16_t* shards, uint16_t* out_TN, int nd, int S,
                      int T, int n);
int kvo_gs_pack_row(const uint16_t* k_blk, const uint16_t* v_blk, uint16_t* rows,
                    int64_t words, int row, int S);

/* ---------------- gs family: RS over GF(2^16) (benchmark/rs/kernel.cu) ------ */
void kvo_rs16_encode(const uint16_t* data_padded, uint16_t* shards, int data_shards,
                     int parity_shards, int64_t shard_size, const uint16_t* gf_exp,
                     const uint16_t* gf_log);
int kvo_rs16_reconstruct(uint16_t* shards, int64_t shard_size, int data_shards,
                         int parity_shards, const int32_t* missing_data, int m,
                         const int32_t* parity_used, const uint16_t* gf_exp,
                         const uint16_t* gf_log);

/* ---------------- spec family: textbook RDP ---------------- */
/* data[0..k-1], P, Q: (p-1) row planes of R bytes each. k <= p-1. */
int kvo_rdp_encode(const uint8_t* const* data, int k, uint8_t* P, uint8_t* Q, int p,
                   int64_t R);
/* cols[0..k+1] = data..., P, Q.  e0/e1 are erased shard indices or -1. */
int kvo_rdp_decode(uint8_t* const* cols, int k, int p, int64_t R, int e0, int e1);
/* striped geometry: stripes of (p-1)*U bytes, rows of min(U, R - s*U) bytes */
int kvo_rdp_encode_striped(const uint8_t* const* data, int k, uint8_t* P, uint8_t* Q, int p,
                           int64_t R, int64_t U);
int kvo_rdp_decode_striped(uint8_t* const* cols, int k, int p, int64_t R, int64_t U, int e0,
                           int e1);

/* ---------------- spec family: RS over GF(2^8) (Cauchy) ---------------- */
int kvo_rs8_encode(const uint8_t* const* data, int k, uint8_t* const* parity, int m,
                   int64_t S);
int kvo_rs8_decode(uint8_t* const* shards, int k, int m, int64_t S,
                   const int32_t* erased, int n_erased);

/* ---------------- paged KV gather ---------------- */
/* pool: [L][pool_pages][page_tokens][2][tok_bytes]; page_table: [B][pps] int32.
 * stream: [L][B][T][2][tok_bytes] for tokens tok_off .. tok_off+T-1. */
int kvo_kv_gather(const uint8_t* pool, int64_t pool_pages, int L, int64_t tok_bytes,
                  int page_tokens, const int32_t* page_table, int B, int pps,
                  int tok_off, int T, uint8_t* stream);

/* number of OpenMP threads the oracle will use (1 without OpenMP) */
int kvo_num_threads(void);
void kvo_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
