// piece_walk.h -- pieces of the reference's packed row tensors, one wave per
// piece, with the row windows loaded and stored at the rows' own alignment.
//
// The tile engine (tile_engine.h) has every block own one tile of columns,
// join each misaligned window from two aligned loads and realign its outputs
// through LDS, with two block barriers per tile.  The engine here has each
// wave walk pieces of 64 windows of every row, lane t holding logical bytes
// 16t .. 16t+15 of the piece in every row.  A lane loads and stores its
// windows directly at the row's own alignment: gfx950 runs compute queues in
// unaligned-access mode, and 16-byte loads and stores at 2-byte-aligned
// addresses are exact (checked on MI355X; a 256 MiB copy took 82.0 us aligned
// and 86-90 us with the source, the destination or both misaligned).  So a piece needs no lane
// shifts, no LDS and no barrier, and a wave requests the next piece's windows
// before it codes the current one.  Only a row's last window can be partial;
// its bytes are stored one by one.
//
// Rows are addressed through one buffer resource of fewer than 2^31 bytes
// based at the 16-byte-aligned address at or below the tensor, so offsets are
// never negative and a voffset of kNoLoad reads nothing.  The resource ends at
// the 16-byte boundary at or past the tensor's end: reading further could
// touch an unmapped page.
#pragma once

#include "tile_engine.h"

namespace kvec {

constexpr uint32_t kPieceBytes = 1024;               // logical bytes per row per piece
constexpr int kPieceBS = 256;                        // threads per block
constexpr int kPieceWaves = kPieceBS / 64;           // waves per block

// Host: blocks for rows of Sb bytes, with at most max_blocks blocks.
inline uint32_t piece_grid(uint64_t Sb, uint32_t max_blocks) {
    const uint64_t pieces = (Sb + kPieceBytes - 1) / kPieceBytes;
    const uint64_t blocks = (pieces + kPieceWaves - 1) / kPieceWaves;
    return uint32_t(blocks < max_blocks ? blocks : max_blocks);
}

// The calling wave's pieces: logical columns first, first + stride, ... below
// the row length.  Consecutive waves take consecutive pieces, so the waves in
// flight sweep one compact region of every row.  Waves that each walked a
// contiguous run of their own (about 22 KiB of every row) were slower: the
// GF(2^16) encode on pieces took 339 against 295 us on the 512 MiB stream.
// Wave-uniform.
struct PieceWalk {
    uint32_t first, stride;
};
__device__ __forceinline__ PieceWalk wave_walk() {
    const uint32_t w = uint32_t(__builtin_amdgcn_readfirstlane(int(blockIdx.x * kPieceWaves + (threadIdx.x >> 6))));
    return PieceWalk{w * kPieceBytes, gridDim.x * kPieceWaves * kPieceBytes};
}

// The lane's window of the row starting at byte `row` of the resource: 16
// bytes at logical column L.  `lim` is the highest offset a 16-byte load may
// start at: the resource size less 16 for the tensor's last row, whose last
// windows reach past the resource's end (a dword only partly in range reads
// as zero), and ~0 for the other rows.  A window starting past lim is read as
// the resource's last 16 bytes shifted into place (zeros past the end).
__device__ __forceinline__ u32x4 piece_load(__amdgpu_buffer_rsrc_t rs, uint32_t row, uint32_t L, uint32_t lim) {
    const uint32_t o = row + L;
    u32x4 v = chunk_load(rs, o < lim ? o : lim);
    if (o > lim) v = o - lim < 16 ? funnel16(v, u32x4{0, 0, 0, 0}, o - lim) : u32x4{0, 0, 0, 0};
    return v;
}

// Store the lane's window v of the row starting at byte `row`, logical
// columns [L, L+16) clipped to the row length hi.
template <bool NT>
__device__ __forceinline__ void piece_store(__amdgpu_buffer_rsrc_t rs, uint32_t row, uint32_t L, uint32_t hi,
                                          u32x4 v) {
    if (L + 16 <= hi) {
        __builtin_amdgcn_raw_buffer_store_b128(v, rs, row + L, 0, NT ? kAuxStoreNT : 0);
    } else if (L < hi) {
        for (uint32_t i = 0; i < hi - L; ++i)
            __builtin_amdgcn_raw_buffer_store_b8(byte_of(v, int(i)), rs, row + L + i, 0, 0);
    }
}

}  // namespace kvec
