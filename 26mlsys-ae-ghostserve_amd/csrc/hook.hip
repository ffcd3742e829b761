// hook.hip -- the serving hook's per-step work as one call.
//
// The reference's plugin codes every prefill step in Python: it indexes the
// KV pool with the step's slots twice, converts to fp16, packs each rank's
// row, calls compute_rdp_parity, copies P and Q to the host and synchronizes
// the device after each part (bench_ghostserve_rdp.py:334-374, :440-458).
// Issued from Python one torch call at a time, even without the
// synchronizations, that sequence costs the host more per step than the GPU
// work it enqueues.  kvec_hook_step enqueues the same work -- slot upload,
// split gather into the rank's row, P/Q, the copy of P and Q to pinned host
// memory, and the events that time them -- in one call.
#include "kvec_internal.h"

using namespace kvec;

namespace {

int hip_rc(hipError_t e, const char* fn, const char* what) {
    if (e == hipSuccess) return KVEC_OK;
    return set_error(KVEC_EHIP, "%s: %s: %s", fn, what, hipGetErrorString(e));
}

}  // namespace

extern "C" int kvec_hook_step(const kvec_paged_kv* kv, const int32_t* slots_host, void* rows, int row, int world,
                              int S, int star_base, void* pq_host, void* stream, void* copy_stream, void* freed,
                              void* const* ev) {
    static const char* fn = "kvec_hook_step";
    if (!rows) return set_error(KVEC_EINVAL, "%s: null rows", fn);
    if (world < 1 || S < 1) return set_error(KVEC_EINVAL, "%s: world=%d S=%d", fn, world, S);
    hipStream_t st = as_stream(stream);
    int rc;
    if (freed && (rc = hip_rc(hipStreamWaitEvent(st, hipEvent_t(freed), 0), fn, "wait for the row buffer")))
        return rc;
    uint8_t* base = static_cast<uint8_t*>(rows);
    const uint64_t row_bytes = uint64_t(S) * 2;
    if (kv) {
        if (row < 0 || row >= world) return set_error(KVEC_EINVAL, "%s: row=%d not in [0, %d)", fn, row, world);
        const int64_t stream_bytes = kvec_kv_stream_bytes(kv);
        if (stream_bytes < 0) return set_error(KVEC_EINVAL, "%s: bad paged-KV descriptor", fn);
        if (uint64_t(stream_bytes) != row_bytes)
            return set_error(KVEC_EINVAL, "%s: the delta has %lld bytes, a row %llu", fn, (long long)stream_bytes,
                             (unsigned long long)row_bytes);
        if (slots_host) {
            if (!kv->page_table) return set_error(KVEC_EINVAL, "%s: null page table", fn);
            const uint64_t tb = uint64_t(kv->batch) * uint64_t(kv->pages_per_seq) * 4;
            if ((rc = hip_rc(hipMemcpyAsync(const_cast<int32_t*>(kv->page_table), slots_host, tb,
                                            hipMemcpyHostToDevice, st),
                             fn, "slot upload")))
                return rc;
        }
        uint8_t* own = base + uint64_t(row) * row_bytes;
        if ((rc = kvec_kv_gather_split(kv, own, own + row_bytes / 2, stream))) return rc;
    }
    if (!pq_host) return KVEC_OK;
    hipStream_t cs = copy_stream ? as_stream(copy_stream) : st;
    if (cs != st && !(ev && ev[1]))
        return set_error(KVEC_EINVAL, "%s: a separate copy stream needs event 1 to order the copy", fn);
    if (ev && ev[0] && (rc = hip_rc(hipEventRecord(hipEvent_t(ev[0]), st), fn, "event 0"))) return rc;
    if ((rc = kvec_gs_rdp_parity(rows, world, S, star_base, stream))) return rc;
    if (ev && ev[1] && (rc = hip_rc(hipEventRecord(hipEvent_t(ev[1]), st), fn, "event 1"))) return rc;
    if (cs != st && (rc = hip_rc(hipStreamWaitEvent(cs, hipEvent_t(ev[1]), 0), fn, "copy stream wait")))
        return rc;
    if (ev && ev[2] && (rc = hip_rc(hipEventRecord(hipEvent_t(ev[2]), cs), fn, "event 2"))) return rc;
    if ((rc = hip_rc(hipMemcpyAsync(pq_host, base + uint64_t(world) * row_bytes, 2 * row_bytes,
                                    hipMemcpyDeviceToHost, cs),
                     fn, "P/Q copy")))
        return rc;
    if (ev && ev[3] && (rc = hip_rc(hipEventRecord(hipEvent_t(ev[3]), cs), fn, "event 3"))) return rc;
    return KVEC_OK;
}
