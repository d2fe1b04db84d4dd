// CPU check of the ping-pong kernel's K-major B copy addresses (kudnn_amd/csrc/kmajor_copy.h, the arithmetic the
// kernel runs). For every copy of every k-tile of every tile column, and every lane, it applies the raw-buffer rule
// (a 16-byte load is performed when its vector offset + 16 <= the resource size; the scalar offset is not checked)
// and verifies:
//   1. no byte past the operand's last byte, (K - 1) * ldb + 2 N, is ever read;
//   2. every performed load reads its lane's nominal row and chunk, and every element (k, n) with n < N of the tile's
//      columns is covered by a performed load (nothing the MFMAs need is blanked);
// and, as a check that (1) can fail, that the whole-tile form (scalar row offsets) applied to an edge tile would read
// past the end. Exit status 0 when every shape passes.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "kmajor_copy.h"

namespace {

struct Result {
    uint64_t maxEnd = 0;      // one past the largest byte read
    uint64_t missing = 0;     // in-matrix elements of the tile no performed load covered
    uint64_t misplaced = 0;   // performed loads whose address is not their nominal row and chunk
};

// All copies of tile column n0 in one form (wholeTile: one resource per k-tile, rows in the scalar offset). A lane's
// nominal element block is row 64 kt + 2q + lane / 32 of the k-tile and columns 8 c .. 8 c + 7 of the tile with
// c = (lane % 32) ^ (4 (row % 4)), as the kernel's LDS layout expects.
Result Walk(uint32_t K, uint32_t N, uint32_t ldb, uint32_t n0, bool wholeTile)
{
    const uint32_t es = 2, bytes = (K - 1) * ldb + N * es, n0b = n0 * es;
    Result r;
    std::vector<uint8_t> seen(static_cast<size_t>(K) * kudnn_km::kTileCols, 0);
    for (uint32_t kt = 0; kt < K / kudnn_km::kTileRows; ++kt) {
        for (uint32_t q = 0; q < kudnn_km::kCopies; ++q) {
            const uint32_t base = wholeTile ? kudnn_km::tile_off(ldb, n0b, kt) : kudnn_km::block_off(ldb, n0b, kt, q);
            const uint32_t size = kudnn_km::remain(bytes, base);
            const uint32_t soff = wholeTile ? kudnn_km::tile_soff(ldb, q) : 0u;
            for (uint32_t lane = 0; lane < 64; ++lane) {
                const uint32_t row = 2 * q + lane / 32, k = kt * kudnn_km::kTileRows + row;
                const uint32_t c = (lane % 32) ^ (4 * (row % 4));
                const uint32_t voff = kudnn_km::lane_voff(ldb, lane, q);
                if (voff + 16u > size) {
                    continue;  // range check: reads zero
                }
                const uint64_t addr = static_cast<uint64_t>(base) + soff + voff;
                r.maxEnd = addr + 16 > r.maxEnd ? addr + 16 : r.maxEnd;
                r.misplaced += addr != static_cast<uint64_t>(n0b) + static_cast<uint64_t>(k) * ldb + c * 16;
                for (uint32_t e = 0; e < 8; ++e) {
                    if (n0 + 8 * c + e < N) {
                        seen[k * kudnn_km::kTileCols + 8 * c + e] = 1;
                    }
                }
            }
        }
    }
    for (uint32_t k = 0; k < K; ++k) {
        for (uint32_t c = 0; c < kudnn_km::kTileCols && n0 + c < N; ++c) {
            r.missing += seen[k * kudnn_km::kTileCols + c] == 0;
        }
    }
    return r;
}

}  // namespace

int main()
{
    struct Shape {
        uint32_t K, N, pad;  // row pitch = N + pad elements
    } shapes[] = {{640, 136, 0}, {640, 264, 0}, {640, 520, 0}, {1280, 1160, 0}, {64, 8, 0},   {128, 256, 0},
                  {192, 1032, 0}, {640, 264, 8},  {640, 520, 24}, {4096, 4104, 0}, {5120, 13824, 0}};
    int failed = 0, edgeTiles = 0, detected = 0;
    for (const Shape &s : shapes) {
        const uint32_t ldb = (s.N + s.pad) * 2, bytes = (s.K - 1) * ldb + s.N * 2;
        for (uint32_t n0 = 0; n0 < s.N; n0 += kudnn_km::kTileCols) {
            const bool whole = kudnn_km::whole_tile(n0, s.N);
            const Result r = Walk(s.K, s.N, ldb, n0, whole);  // the form the kernel takes for this tile
            const bool ok = r.maxEnd <= bytes && r.missing == 0 && r.misplaced == 0;
            if (!ok) {
                std::printf("FAIL K=%u N=%u ldb=%u n0=%u (%s): max byte end %llu of %u, missing %llu, misplaced %llu\n",
                            s.K, s.N, ldb, n0, whole ? "whole-tile" : "per-copy", (unsigned long long)r.maxEnd, bytes,
                            (unsigned long long)r.missing, (unsigned long long)r.misplaced);
                ++failed;
            }
            if (!whole) {
                // the form the kernel must not take here reads past the end whenever the pitch equals the row
                ++edgeTiles;
                const Result bad = Walk(s.K, s.N, ldb, n0, true);
                detected += bad.maxEnd > bytes;
            }
        }
    }
    std::printf("%d edge tiles; the whole-tile form would overrun on %d of them; %d failures\n", edgeTiles, detected,
                failed);
    return failed == 0 && detected > 0 ? 0 : 1;
}
