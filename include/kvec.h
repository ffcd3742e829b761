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

/* Library version, as 10000*major + 100*minor + patch. */
int kvec_version(void);
/* Static description of a KVEC_E* code. */
const char* kvec_strerror(int code);
/* Message of the last failing call on this thread ("" if none). */
const char* kvec_last_error(void);

/* ======================= spec family: textbook RDP ======================= */
/* No reference counterpart (the reference "RDP" is the gs star-diagonal code
 * below); this is the code BASELINE's RDP configurations name.
 * Stripe: p prime (3..13), k data shards (1 <= k <= p-1; data columns k..p-2
 * are implicit zeros), each shard buffer holds p-1 row planes of `row_bytes`
 * bytes (row r at offset r*row_bytes); row_bytes % 16 == 0.  Column p-1 is
 * the row parity P, Q holds diagonals 0..p-2 over columns 0..p-1. */

/* P, Q from data[0..k-1] (host array of k device pointers). */
int kvec_rdp_encode(const void* const* data, int k, void* P, void* Q, int p,
                    int64_t row_bytes, void* stream);

/* Rebuild up to two erased shards in place.  shards = host array of k+2
 * device pointers (data..., P, Q); e0/e1 are shard indices in [0, k+1] or -1. */
int kvec_rdp_decode(void* const* shards, int k, int p, int64_t row_bytes, int e0,
                    int e1, void* stream);

/* Smallest row plane size (multiple of `granule`, itself a multiple of 16) whose
 * k*(p-1) row planes hold `stream_bytes` bytes.  Host-only arithmetic. */
int64_t kvec_rdp_row_bytes(int64_t stream_bytes, int k, int p, int64_t granule);

#ifdef __cplusplus
}
#endif
#endif /* KVEC_H */
