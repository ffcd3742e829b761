/*
 * kvec.h -- C ABI of libkvec, the MI355X (gfx950) KV-cache erasure-coding
 * library.  Plain pointers and sizes only: every buffer argument is a device
 * pointer unless the comment says "host", `stream` is a hipStream_t (NULL is
 * the null stream), and every call is stream-ordered and never waits for the
 * device.  Every function returns KVEC_OK (0) or a negative KVEC_E* code;
 * kvec_last_error() gives the message of the last failure on the calling
 * thread.
 *
 * Two codec families:
 *   gs    bit-exact with the reference kernels (same arguments, same output
 *         bytes, same layouts): XOR, the star-diagonal "RDP" P/Q code and
 *         Reed-Solomon over GF(2^16).
 *   spec  textbook RDP over a prime p (Corbett et al., FAST 2004) and
 *         Reed-Solomon over GF(2^8) with polynomial 0x11D and the systematic
 *         Cauchy parity block C[i][j] = 1 / ((k+i) ^ j).  Shards are separate
 *         buffers (host array of device pointers), 16-byte aligned.
 *
 * File:line citations name the reference interface each entry point replaces
 * (project-ghostserve/26mlsys-AE-GhostServe).
 */
#ifndef KVEC_H
#define KVEC_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVEC_OK 0
#define KVEC_EINVAL (-1)      /* bad argument (shape, range, alignment, null) */
#define KVEC_EUNSUPPORTED (-2) /* valid but not built (e.g. prime too large) */
#define KVEC_EHIP (-3)        /* HIP launch/runtime error */
#define KVEC_EDECODE (-4)     /* erasure pattern cannot be decoded */

/* Library version, as 10000*major + 100*minor + patch.  The major number
 * changes with every incompatible change of the entry points or structs
 * below; a caller built against this header checks
 * kvec_version() / 10000 == KVEC_VERSION / 10000 before its first call.
 * 1.0.0: kvec_rdp_encode / kvec_rdp_decode / kvec_rdp_encode_paged take
 * unit_bytes, kvec_chunk_stripe has region_off and unit_bytes (0.1.0 had
 * neither).  1.1.0: kvec_hook_step added. */
#define KVEC_VERSION 10100
int kvec_version(void);
/* Static description of a KVEC_E* code. */
const char* kvec_strerror(int code);
/* Message of the last failing call on this thread ("" if none). */
const char* kvec_last_error(void);

/* ======================= spec family: textbook RDP ======================= */
/* No reference counterpart (the reference "RDP" is the gs star-diagonal code
 * below); this is Row-Diagonal Parity as Corbett et al. define it (FAST 2004),
 * the double-parity code of the p = 7, k = 6 KV chunk stripes.
 * Code: p prime (3..13), k data shards (1 <= k <= p-1; data columns k..p-2
 * are implicit zeros), column p-1 is the row parity P, Q holds diagonals
 * 0..p-2 over columns 0..p-1.
 * Geometry: every shard buffer holds (p-1)*row_bytes bytes, row_bytes % 16 ==
 * 0, cut into stripes of (p-1)*unit_bytes bytes (the last one shorter when
 * unit_bytes does not divide row_bytes).  Stripe s has p-1 rows of
 * g_s = min(unit_bytes, row_bytes - s*unit_bytes) bytes, row r at shard byte
 * s*(p-1)*unit_bytes + r*g_s, and every byte offset of its rows is one RDP
 * instance.  unit_bytes is 0 (one stripe: p-1 row planes of row_bytes bytes)
 * or a multiple of 1024; 65536 is the fastest on MI355X (each wave's loads of
 * a shard then stay inside one 384 KiB stripe). */

/* P, Q from data[0..k-1] (host array of k device pointers). */
int kvec_rdp_encode(const void* const* data, int k, void* P, void* Q, int p,
                    int64_t row_bytes, int64_t unit_bytes, void* stream);

/* Rebuild up to two erased shards in place.  shards = host array of k+2
 * device pointers (data..., P, Q); e0/e1 are shard indices in [0, k+1] or -1. */
int kvec_rdp_decode(void* const* shards, int k, int p, int64_t row_bytes, int64_t unit_bytes,
                    int e0, int e1, void* stream);

/* Smallest row plane size (multiple of `granule`, itself a multiple of 16) whose
 * k*(p-1) row planes hold `stream_bytes` bytes.  Host-only arithmetic. */
int64_t kvec_rdp_row_bytes(int64_t stream_bytes, int k, int p, int64_t granule);

/* ================== spec family: RS over GF(2^8), Cauchy ================== */
/* No reference counterpart (the reference RS works over GF(2^16), below); this
 * is Reed-Solomon over GF(2^8), the code of the RS(6,2) and RS(5,3) KV stripes.
 * Polynomial 0x11D, systematic
 * generator [I_k; C] with C[i][j] = 1 / ((k+i) ^ j).  Shards are separate
 * 16-byte aligned buffers of shard_bytes (% 16 == 0) bytes.
 * Limits: k <= 32, m <= 8, k*m <= 64. */

/* The m x k block C, row-major, into host memory. */
int kvec_rs8_cauchy(int k, int m, uint8_t* C);
/* parity[i] = XOR_j C[i][j] * data[j]; host arrays of device pointers. */
int kvec_rs8_encode(const void* const* data, int k, void* const* parity, int m,
                    int64_t shard_bytes, void* stream);
/* Rebuild the erased shards (host int32 array of shard indices in [0, k+m),
 * at most m of them) in place from the first k surviving shards.  shards =
 * host array of k+m device pointers (data..., parity...). */
int kvec_rs8_decode(void* const* shards, int k, int m, int64_t shard_bytes,
                    const int32_t* erased, int n_erased, void* stream);

/* ============================ paged KV gather ============================ */
/* The delta gather of the serving plugin, K = pool[slots, 0], V = pool[slots, 1]
 * (bench_ghostserve_rdp.py:440-458), over a paged pool.  Pool layout:
 * [layers][pool_pages][page_tokens][2 (K,V)][token_bytes]; page_table: device
 * int32 [batch][pages_per_seq] of pool pages.  The coding stream of a chunk
 * (positions tok_off .. tok_off+tokens-1 of every sequence) is the chunk's
 * token records in order, [layers][batch][tokens][2 (K,V)][token_bytes].
 * token_bytes % 16 == 0, page_tokens a power of two.  Page-table entries
 * outside [0, pool_pages) read as zero pages and are skipped by the scatter. */
typedef struct kvec_paged_kv {
    const void* pool;
    int64_t pool_pages;
    int layers;
    int64_t token_bytes;        /* kv_heads * head_dim * element bytes */
    int page_tokens;
    const int32_t* page_table;  /* device */
    int batch;
    int pages_per_seq;
    int tok_off;
    int tokens;
} kvec_paged_kv;

/* Bytes of the coding stream of `kv` (host arithmetic). */
int64_t kvec_kv_stream_bytes(const kvec_paged_kv* kv);
/* out[0 .. stream bytes) = the chunk's stream gathered from the pool. */
int kvec_kv_gather(const kvec_paged_kv* kv, void* out, void* stream);
/* The chunk's K halves to out_k and V halves to out_v, each in record order
 * (layer, sequence, token): with one layer and one sequence this is the
 * serving plugin's delta gather kv_pool[slots, 0] and kv_pool[slots, 1]
 * (bench_ghostserve_rdp.py:445-458) written straight into the [K | V] parity
 * row that pack_row_from_block assembles (:105-118).  Both outputs 16-byte
 * aligned; each receives stream_bytes / 2 bytes. */
int kvec_kv_gather_split(const kvec_paged_kv* kv, void* out_k, void* out_v, void* stream);
/* Inverse: write the stream `in` back into the pool pages (pool == kv->pool). */
int kvec_kv_scatter(const kvec_paged_kv* kv, void* pool, const void* in, void* stream);
/* Fused gather + spec RDP encode: the chunk's stream, cut into k data shards
 * of (p-1)*row_bytes bytes (zero padded), is written to data[0..k-1] and its
 * P, Q to P, Q (stripe geometry as kvec_rdp_encode), reading every pool byte
 * once.  row_bytes and unit_bytes must be multiples of 2*token_bytes (one
 * token record) and k*(p-1)*row_bytes >= the stream bytes. */
int kvec_rdp_encode_paged(const kvec_paged_kv* kv, void* const* data, int k, void* P, void* Q,
                          int p, int64_t row_bytes, int64_t unit_bytes, void* stream);
/* Inverse of kvec_rdp_encode_paged (the reference's recovery + load_full back
 * into K/V, benchmark/rdp/kernel.cu:305-345 and benchmark/rdp/main.py:95-126,
 * with textbook RDP and the pool as the destination): up to two erased shards
 * e0, e1 (data 0..k-1, P = k, Q = k+1, or -1) are rebuilt; lost data cells
 * are written straight into their pool pages (pool == kv->pool) and, when
 * `data` (host array of k device pointers, or NULL) is given, into the data
 * shards too; lost P / Q into P / Q.  Surviving data is read from `data` when
 * given, else from the pool.  Same geometry arguments as the encode.
 * Page-table entries of one chunk must be distinct. */
int kvec_rdp_decode_paged(const kvec_paged_kv* kv, void* pool, void* const* data, int k, void* P,
                          void* Q, int p, int64_t row_bytes, int64_t unit_bytes, int e0, int e1,
                          void* stream);

/* ================= chunked coding of a paged pool (spec family) ================= */
/* No reference function: the reference codes each prefill step's KV after an
 * fp16 conversion (bench_ghostserve_rdp.py:334-392); this codes the cache bytes
 * themselves (any dtype, e.g. fp8 e4m3), chunk by chunk, with textbook RDP(p)
 * and RS(k, m) over GF(2^8)/0x11D (Cauchy) sharing the same k data shards.
 *
 * A whole-sequence stripe set is k data shards (optional: NULL data means the
 * pool is the only copy of the data), P, Q and m RS parity shards, each
 * (p-1)*row_bytes bytes.  Chunk c owns the region of (p-1)*width bytes at
 * region_off of every shard (c*(p-1)*width for chunks in order), which is an
 * RDP stripe set in the striped geometry of kvec_rdp_encode with rows of
 * `width` bytes and unit `unit_bytes`.  The chunk's stream (the kvec_paged_kv
 * chunk), zero padded to k*(p-1)*width bytes, is cut into k pieces of
 * (p-1)*width bytes, piece j being data shard j's region.  Every code works on
 * its own stripe instances, so encoding chunk c writes only its own region,
 * reads no parity, and the per-chunk encodes together code the whole set.
 * Built: p in {3, 5, 7}, 2 <= k <= p-1, 0 <= m <= 3 (decode: k <= 6). */
typedef struct kvec_chunk_stripe {
    void* const* data;  /* host array of k device pointers, or NULL */
    int k;
    void* P;            /* RDP row parity */
    void* Q;            /* RDP diagonal parity (diagonals 0..p-2) */
    int p;
    void* const* rs;    /* host array of m device pointers (RS parity 0..m-1) */
    int m;
    int64_t row_bytes;  /* R: every shard is (p-1)*R bytes, < 4 GiB; R % 16 == 0 */
    int64_t region_off; /* this chunk's region in every shard, multiple of 16 */
    int64_t width;      /* the region's row bytes, a multiple of 2*token_bytes */
    int64_t unit_bytes; /* stripe unit of the region: 0 or a multiple of 1024 and of
                           2*token_bytes (65536 is the fastest) */
} kvec_chunk_stripe;

/* Smallest cell width (multiple of record_bytes) whose k*(p-1) cells hold
 * chunk_stream_bytes bytes.  Host-only arithmetic; -1 on bad arguments. */
int64_t kvec_chunk_width(int64_t chunk_stream_bytes, int k, int p, int64_t record_bytes);
/* One pass over the chunk's pool pages: data shards (if given), P, Q and the
 * RS parity in the chunk's region. */
int kvec_chunk_encode_paged(const kvec_paged_kv* kv, const kvec_chunk_stripe* stripe,
                            void* stream);
/* Rebuild the chunk's region of the erased shards.  erased: host int32 array of
 * shard indices, data 0..k-1, P = k, Q = k+1, RS parity i = k+2+i.  Lost data
 * cells are written into the pool pages (pool == kv->pool; surviving data is
 * read from the pool) and into the data shards when given; lost parity shards
 * are recomputed.  RS decodes when the data erasures do not exceed the
 * surviving RS parities, else RDP when data + P/Q erasures are at most two;
 * anything else is KVEC_EDECODE.  Page-table entries of one chunk must be
 * distinct (a shared page would be read and rewritten by two cells). */
int kvec_chunk_decode_paged(const kvec_paged_kv* kv, void* pool, const kvec_chunk_stripe* stripe,
                            const int32_t* erased, int n_erased, void* stream);

/* ============ gs family: XOR (benchmark/xor/kernel.cu, main.py) =========== */
/* Byte shards, packed: shards = [(data_shards + 1), shard_size] bytes. */

/* encode_xor_launcher, benchmark/xor/kernel.cu:158-171: copy the data rows of
 * data_padded [data_shards*shard_size] into shards, then P = XOR of them. */
int kvec_xor_encode(const void* data_padded, void* shards, int data_shards,
                    int64_t shard_size, void* stream);
/* forward_encode_kv, benchmark/xor/main.py:69-90 (pack_kv of K then V, each
 * kv_half_bytes raw bytes, into the data stream, zero padding to
 * data_shards*shard_size) followed by encode_xor (:158-171): one pass over K and
 * V when shards, K and V are 16-byte aligned, kv_half_bytes is a multiple of
 * 16, data_shards <= 8 and shard_size >= 4096 (else the copies, then the
 * encode).  Needs 2*kv_half_bytes <= data_shards*shard_size. */
int kvec_xor_encode_kv(const void* key_input, const void* value_input, int64_t kv_half_bytes,
                       void* shards, int data_shards, int64_t shard_size, void* stream);
/* reconstruct_xor_launcher, :173-191.  missing_indices: device int32 array of
 * missing_count entries; only missing_count == 1 does anything: a data row
 * m < data_shards is rebuilt from P, m == data_shards recomputes P.  The row is
 * written to recovered_data (may alias encoded_data) and recovered_missing. */
int kvec_xor_reconstruct(const void* encoded_data, void* recovered_data,
                         void* recovered_missing, int64_t shard_size, int data_shards,
                         const int32_t* missing_indices, int missing_count, void* stream);
/* backwards_decode_kv, benchmark/xor/main.py:159-194: missing shard rebuilt
 * in place (a data row from P and the others in one pass with the copy-out; P
 * recomputed when missing == data_shards; missing < 0: nothing rebuilt), then
 * the first out_bytes of the data rows copied to out (unpack_kv). */
int kvec_xor_recover_kv(void* shards, void* out, int data_shards, int64_t shard_size,
                        int64_t out_bytes, int missing, void* stream);
/* pack_kv_launcher / unpack_kv_launcher, :193-223: K bytes then V bytes of
 * n*seq_len 16-bit words each (little-endian split == memory order). */
int kvec_pack_kv(const void* key_input, const void* value_input, void* kv_bytes, int n,
                 int seq_len, void* stream);
int kvec_unpack_kv(const void* kv_bytes, void* dequant_kv, int n, int seq_len, void* stream);

/* ====== gs family: star-diagonal RDP (benchmark/rdp/kernel.cu, main.py) ====== */
/* u16 words, packed: shards = [(nd + 2), S]; P = row nd, Q = row nd+1.
 * Q[d] = XOR_r D_r[(d - r) mod S], skipping column (star_base + r) % S of row r. */

/* fused_backup_full_kv_launcher, benchmark/rdp/kernel.cu:366-395: K_TN, V_TN
 * are [T, n] words; data rows get K_TN || V_TN (words past row nd-1 dropped),
 * then P and Q.  The caller zero-initialises the padding words. */
int kvec_gs_rdp_backup(const void* K_TN, const void* V_TN, void* shards, int nd, int S, int T,
                       int n, int star_base, void* stream);
/* fused_recovery_full_kv_launcher, :397-521: observable semantics of the
 * reference (indices outside [0, nd) ignored; one data row is rebuilt from P;
 * for two, the lower row is rebuilt from P and the other keeps its bytes),
 * then out_TN [2*T*n] words = the data rows.  For two lost rows with
 * (star_base + a) % S < 0 (a the lower row, C's %) the reference reads and
 * writes outside row a (:268-282); that case returns KVEC_EINVAL. */
int kvec_gs_rdp_recover(void* shards, void* out_TN, int nd, int S, int T, int n, int star_base,
                        int missing_a, int missing_b, void* stream);
/* pack_row_from_block_launcher, bench_ghostserve_rdp.py:152-175:
 * rows[row*S ..] = k_blk words then v_blk words (S >= 2*words). */
int kvec_gs_pack_row(const void* k_blk, const void* v_blk, void* rows, int64_t words, int row,
                     int64_t S, void* stream);
/* compute_rdp_parity_launcher, bench_ghostserve_rdp.py:177-199: P, Q of the
 * first nd rows of `rows` (row stride S words) into rows nd and nd+1. */
int kvec_gs_rdp_parity(void* rows, int nd, int S, int star_base, void* stream);
/* No reference counterpart: the serving plugin's per-step parity
 * (bench_ghostserve_rdp.py:334-374 with the delta gather of :440-458), the
 * work its Python issues as separate torch calls, enqueued by one call.
 * rows: [world + 2, S] u16 on the device; kv: the step's delta, its page
 * table the device slot buffer ([1][n] with 1-token pages over a
 * [1][T][1][2][H][D] view of the pool).  On `stream`, in order:
 *   - wait for the event `freed` (if not NULL: the last copy out of rows);
 *   - if kv is not NULL: copy n int32 slots from slots_host (host, pinned;
 *     skipped when NULL) into kv->page_table, then gather the delta's K
 *     words and V words into row `row` (kvec_kv_gather_split);
 *   - if pq_host is not NULL: record ev[0], P and Q of rows 0..world-1 into
 *     rows world and world+1 (kvec_gs_rdp_parity), record ev[1]; then on
 *     copy_stream (NULL: `stream`), after ev[1]: record ev[2], copy the two
 *     rows (4*S bytes) to pq_host (host, pinned), record ev[3].
 * ev: 4 hipEvent_t (any may be NULL; ev[1] is required when copy_stream is
 * another stream).  Host copies make it unfit for graph capture. */
int kvec_hook_step(const kvec_paged_kv* kv, const int32_t* slots_host, void* rows, int row, int world, int S,
                   int star_base, void* pq_host, void* stream, void* copy_stream, void* freed,
                   void* const* ev);

/* ======== gs family: RS over GF(2^16) (benchmark/rs/kernel.cu, main.py) ======= */
/* u16 symbols, packed: shards = [(k + m), shard_size].  gf_exp / gf_log are
 * device tables: those of init_gf_tables() (poly 0x1100B), or any exp/log pair
 * of GF(2^16) (any primitive polynomial, any generator), for which every
 * kernel gives the reference's bytes.  Tables that are not a field's make the
 * bytes unspecified (they may differ between shapes). */

/* pack_fp16_pair_to_u16, benchmark/rs/kernel.cu:225-243: out = K || V words. */
int kvec_rs16_pack(const void* k, const void* v, void* out, int64_t N_k, int64_t N_v,
                   void* stream);
/* u16_to_fp16_split, :245-263: inverse of kvec_rs16_pack. */
int kvec_rs16_split(const void* in, void* k_out, void* v_out, int64_t N_k, int64_t N_v,
                    void* stream);
/* encode_rs_u16, :265-285: copy data rows; Par_p = XOR_i D_i * alpha^((p+1) i).
 * Any data_shards >= 1 and parity_shards >= 0 with (k - 1) * m < 2^31 (the
 * reference's int exponent) and m <= 524280; KVEC_EUNSUPPORTED beyond. */
int kvec_rs16_encode(const void* data_padded, void* shards, int data_shards, int parity_shards,
                     int shard_size, const uint16_t* gf_exp, const uint16_t* gf_log,
                     void* stream);
/* reconstruct_rs_u16_inplace, :287-312: rebuild the m data rows listed in the
 * device int32 array missing_data from the parity rows in parity_used (device,
 * m entries; m <= 16 as the reference's, any data_shards >= m).  Parity rows
 * are not rewritten.  Indices outside the tensor, or a repeated missing index,
 * make the call write nothing. */
int kvec_rs16_reconstruct(void* shards, int shard_size, int data_shards, int parity_shards,
                          const int32_t* missing_data, int m, const int32_t* parity_used,
                          const uint16_t* gf_exp, const uint16_t* gf_log, void* stream);
/* init_gf_tables, benchmark/rs/main.py:39-54, into host arrays (exp: 131070
 * entries, log: 65536). */
int kvec_gf16_tables(uint16_t* gf_exp, uint16_t* gf_log);

#ifdef __cplusplus
}
#endif
#endif /* KVEC_H */
