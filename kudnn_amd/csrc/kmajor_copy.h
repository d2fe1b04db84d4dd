// Address arithmetic of the ping-pong kernel's copies of a K-major B (a weight stored [K][N], N contiguous, row pitch
// ldb bytes). Shared by the kernel (gemm_pingpong.hip) and a CPU test of its bounds (tests/cpp/test_kmajor_bounds.cpp),
// so the test checks the arithmetic the kernel runs.
//
// A k-tile of B is 64 k-rows of the tile's 256 columns (512 bytes of 16-bit elements a row). Copy q (0..31) of k-tile
// kt moves 1 KB: k-rows 64 kt + 2q and 64 kt + 2q + 1. Lane l reads the 16-byte chunk (l % 32) ^ (4 (row % 4)) of row
// 2q + l / 32, so the LDS writes stay linear while the tile lands swizzled.
//
// The copies go through raw buffer resources (base, size). The hardware range check applies to the vector offset
// only; the scalar offset is added outside it. So a resource that starts at the k-tile's first byte and reaches the
// k-rows through the scalar offset blanks nothing past the operand's end: on a tile that crosses column N, the last
// k-row's copy would read up to 496 bytes past the operand. Such tiles take a resource per copy that starts at the
// copy's first row (block_off) with size bytes - block_off and scalar offset 0: then a chunk past the operand fails the
// range check and reads zero. With N a multiple of 8 every 16-byte chunk lies wholly inside or wholly past the end.
#ifndef KUDNN_KMAJOR_COPY_H
#define KUDNN_KMAJOR_COPY_H

#include <stdint.h>

#if defined(__HIPCC__)
#define KUDNN_KM_FN __host__ __device__ __forceinline__
#else
#define KUDNN_KM_FN inline
#endif

namespace kudnn_km {

constexpr uint32_t kTileCols = 256;  // columns of a tile
constexpr uint32_t kTileRows = 64;   // k-rows of a k-tile
constexpr uint32_t kCopies = 32;     // 1 KB copies per k-tile

// Lane l's vector offset (bytes from the copy's first row) in copy q: row l / 32 of the two, source chunk
// (l % 32) ^ (4 (row % 4)) where row % 4 = 2 (q % 2) + l / 32.
KUDNN_KM_FN uint32_t lane_voff(uint32_t ldb, uint32_t lane, uint32_t q)
{
    const uint32_t row = lane >> 5, slot = lane & 31u;
    return row * ldb + ((slot ^ (4u * (2u * (q & 1u) + row))) * 16u);
}

// Byte offset of k-tile kt's first row at column byte n0b.
KUDNN_KM_FN uint32_t tile_off(uint32_t ldb, uint32_t n0b, uint32_t kt) { return kt * kTileRows * ldb + n0b; }

// Byte offset of copy q's first row in k-tile kt at column byte n0b.
KUDNN_KM_FN uint32_t block_off(uint32_t ldb, uint32_t n0b, uint32_t kt, uint32_t q)
{
    return (kt * kTileRows + 2u * q) * ldb + n0b;
}

// Scalar offset of copy q from its k-tile's first row (the whole-tile form).
KUDNN_KM_FN uint32_t tile_soff(uint32_t ldb, uint32_t q) { return 2u * q * ldb; }

// Resource size for a resource that starts `off` bytes into an operand of `bytes` bytes (0 past its end).
KUDNN_KM_FN uint32_t remain(uint32_t bytes, uint32_t off) { return off < bytes ? bytes - off : 0u; }

// Whether a tile whose first column byte is n0b reads its k-rows through one resource per k-tile (the scalar-offset
// form): only when the tile's 256 columns lie inside every k-row, so no copy reaches past the operand's end.
KUDNN_KM_FN bool whole_tile(uint32_t n0, uint32_t N) { return n0 + kTileCols <= N; }

}  // namespace kudnn_km

#endif  // KUDNN_KMAJOR_COPY_H
