// copy.hip -- device-to-device byte copies and zero fills as kernels.
//
// The entry points' fallback paths (layouts the fused kernels do not take:
// misaligned or overlapping K/V, packs and unpacks, zero padding) copy or
// clear memory.  They do it with these kernels instead of hipMemcpyAsync /
// hipMemsetAsync, so every entry point enqueues kernels only and a caller can
// capture any of them in a HIP graph (memset nodes have given wrong results
// on graph replays on this hardware).
//
// Destination chunks are 16-byte aligned; the source window of each is read
// as one or two aligned 16-byte loads joined with v_alignbyte (load_window16),
// so any pair of alignments runs at full width.  The at most 15 bytes before
// the first and after the last aligned destination chunk are copied singly.
#include "tile_engine.h"

namespace kvec {

constexpr int kCopyBS = 256;
constexpr unsigned kCopyMaxBlocks = 8192;

__global__ __launch_bounds__(kCopyBS) void copy_bytes_kernel(uint8_t* __restrict__ dst,
                                                             const uint8_t* __restrict__ src,
                                                             uint64_t n) {
    const uintptr_t D0 = reinterpret_cast<uintptr_t>(dst);
    const uint64_t head = ((D0 + 15) & ~uintptr_t(15)) - D0;   // bytes before the first chunk
    const uint64_t h = head < n ? head : n;
    const uint64_t nch = (n - h) >> 4;
    const uint64_t tail0 = h + (nch << 4);
    const uint64_t stride = uint64_t(gridDim.x) * kCopyBS;
    for (uint64_t c = uint64_t(blockIdx.x) * kCopyBS + threadIdx.x; c < nch; c += stride) {
        const uint64_t o = h + (c << 4);
        st16(dst + o, load_window16(src + o));
    }
    if (blockIdx.x == 0) {
        const gptr<uint8_t> d = as_global(dst);
        const gptr<const uint8_t> s = as_global(src);
        const uint32_t i = threadIdx.x;
        if (i < h) d[i] = s[i];
        else if (i >= 16 && i - 16 < n - tail0) d[tail0 + (i - 16)] = s[tail0 + (i - 16)];
    }
}

__global__ __launch_bounds__(kCopyBS) void zero_bytes_kernel(uint8_t* __restrict__ dst, uint64_t n) {
    const uintptr_t D0 = reinterpret_cast<uintptr_t>(dst);
    const uint64_t head = ((D0 + 15) & ~uintptr_t(15)) - D0;
    const uint64_t h = head < n ? head : n;
    const uint64_t nch = (n - h) >> 4;
    const uint64_t tail0 = h + (nch << 4);
    const uint64_t stride = uint64_t(gridDim.x) * kCopyBS;
    for (uint64_t c = uint64_t(blockIdx.x) * kCopyBS + threadIdx.x; c < nch; c += stride)
        st16(dst + h + (c << 4), u32x4{0, 0, 0, 0});
    if (blockIdx.x == 0) {
        const gptr<uint8_t> d = as_global(dst);
        const uint32_t i = threadIdx.x;
        if (i < h) d[i] = 0;
        else if (i >= 16 && i - 16 < n - tail0) d[tail0 + (i - 16)] = 0;
    }
}

static unsigned copy_grid(uint64_t n) {
    const uint64_t chunks = n / 16 + 1;
    const uint64_t b = (chunks + kCopyBS - 1) / kCopyBS;
    return unsigned(b < kCopyMaxBlocks ? b : kCopyMaxBlocks);
}

int copy_d2d(void* dst, const void* src, uint64_t n, hipStream_t st, const char* what) {
    if (n == 0 || dst == src) return KVEC_OK;
    if (!dst || !src) return set_error(KVEC_EINVAL, "%s: null pointer", what);
    if (ranges_overlap(dst, n, src, n))
        return set_error(KVEC_EINVAL, "%s: source and destination overlap", what);
    hipLaunchKernelGGL(copy_bytes_kernel, dim3(copy_grid(n)), dim3(kCopyBS), 0, st, (uint8_t*)dst,
                       (const uint8_t*)src, n);
    return check_launch(what);
}

int zero_d(void* dst, uint64_t n, hipStream_t st, const char* what) {
    if (n == 0) return KVEC_OK;
    if (!dst) return set_error(KVEC_EINVAL, "%s: null pointer", what);
    hipLaunchKernelGGL(zero_bytes_kernel, dim3(copy_grid(n)), dim3(kCopyBS), 0, st, (uint8_t*)dst, n);
    return check_launch(what);
}

}  // namespace kvec
