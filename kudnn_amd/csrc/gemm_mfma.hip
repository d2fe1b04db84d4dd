// bf16, f16, s8 and fp32 GEMM on gfx950 MFMA with the fused epilogue.
//
// Computes, per batch, Y = epilogue(A[M][K] x B[N][K]^T) with both operands contiguous along K
// (A = activations/X rows, B = nn.Linear-style weight rows). This is the kernel behind cblas_sbgemm /
// cblas_bgemm (bf16), cblas_hgemm / cblas_shgemm (f16), cblas_gemm_s8s8s32 (s8 -> s32) and cblas_sgemm (fp32) in the
// reference (src/dnn/src/kudnn_gemm.cpp:157-264) plus its post-op passes.
//
// Design (one workgroup of 4 waves per BM x BN output tile, waves arranged 2 x 2):
//  - k-tiles of 128 bytes per row (64 bf16 / 32 fp32) go straight from global memory into LDS with
//    gfx950's global_load_lds_dwordx4 (no staging registers) through an ST-stage ring: the loads of tile k+ST-1
//    are issued right after the barrier that opens tile k (ST = 2 for 256 x 256, up to 4 where the tiles are
//    small enough, so that a small grid is not bound by one memory latency per k-tile). The copies are inline asm
//    (dma16) and the ring's waits are explicit (wait_tiles), so they stay in flight during the k-tile's MFMAs.
//  - A wave's LDS DMA instruction fills 8 rows x 128 bytes; lane l writes 16-byte slot l, and fetches the
//    global chunk that the XOR swizzle (chunk ^ (row & 7)) assigns to that slot, so the ds_read_b128 of
//    32 consecutive rows at one logical k-chunk hits every bank once.
//  - MFMA fragments of k16-substep s+1 are read from LDS while substep s's MFMAs issue.
//  - bf16: v_mfma_f32_32x32x16_bf16; f16: v_mfma_f32_32x32x16_f16; s8: v_mfma_i32_32x32x32_i8 (int32 accumulators,
//    kept in the same registers as bit patterns); fp32: v_mfma_f32_32x32x2f32 fed from one 16-byte LDS read per lane
//    (four k values; MFMA q consumes element q of both lane halves, which covers every k exactly once). The 16- and
//    8-bit instructions all take 16 bytes of one row per lane, lane half h holding bytes 16h .. 16h+15 of each
//    32-byte k step for both operands, so one data path serves all three: the sum over k does not depend on how the
//    hardware orders the k values inside a lane, as long as both operands use the same order.
//  - The operands are swapped (weight tile as the first MFMA operand): each lane then owns, per 32x32
//    sub-tile, one output row m and four runs of four consecutive columns n.
//  - Epilogue: the accumulators pass through LDS, one 32-column strip per wave at a time, and are read
//    back row-major so each lane applies bias / activation / residual to 8 consecutive columns and
//    writes them with one 16-byte store (a wave writes 16 rows x 64 contiguous bytes per instruction).
//  - Blocks are remapped so consecutive tiles run on the same XCD and walked in groups of tile-rows.
//  - The activation and the epilogue's tensor types are template arguments (see the forms in device_common.h):
//    full tiles in the bf16 / f32 forms run short straight-line code; other tiles and the generic form go one
//    element at a time.
//  - Split-K for grids too small to fill the chip, in one launch: grid.z splits the k-tiles; every split stores its
//    accumulators in its slot of the workspace and takes a ticket from the tile's arrival counter, and the split that
//    draws the last ticket sums the slots in split order (the same bits whichever split finishes last) and runs the
//    epilogue. No workgroup waits for another.
//  - fp32 weights stored [K][N] (N contiguous) are read in place (BKM): each k-tile of B is copied as 32 k-rows of the
//    tile's columns and read one float per k (see the kernel's comment).
// Requirements (the dispatcher packs operands otherwise): K a multiple of the k-tile, rows 16-byte
// aligned. Rows past M / N are clamped (read but never stored).
#include <algorithm>
#include <type_traits>
#include <utility>

#include "device_common.h"
#include "kernels.h"

using namespace kudnn_dev;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kChunks = 8;   // 16-byte chunks per 128-byte LDS row
constexpr int kStagePitch = 36;  // epilogue staging row pitch in floats (32 columns + 4 pad)

__device__ __forceinline__ int swz(int row, int chunk) { return (chunk ^ (row & 7)); }

// s_waitcnt vmcnt(N) with N a compile-time constant (expcnt / lgkmcnt unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Waits until at most `ahead` tiles of PER DMA instructions each are outstanding (ahead < ST - 1).
template <int PER, int ST>
__device__ __forceinline__ void wait_tiles(int ahead)
{
    if constexpr (ST >= 4) {
        if (ahead >= 2) {
            wait_vmcnt<2 * PER>();
            return;
        }
    }
    if constexpr (ST >= 3) {
        if (ahead >= 1) {
            wait_vmcnt<PER>();
            return;
        }
    }
    wait_vmcnt<0>();
}

// LDS byte address of a __shared__ element.
__device__ __forceinline__ uint32_t lds_byte(const uint4 *p)
{
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void *)p));
}

// One LDS DMA copy: lane l's 16 bytes at src land in LDS at lds + 16 l. It is issued through inline asm so that the
// compiler does not track it. With the builtin (__builtin_amdgcn_global_load_lds) the compiler cannot tell the ring's
// stages apart, so it waited for every copy in flight (vmcnt(0)) before the first fragment read of each k-tile, which
// also waited for the copy just issued for k-tile kt + ST - 1 and left no copy in flight during the MFMAs. The waits
// are the kernel's own instead: wait_tiles before each k-tile's barrier. The s_nop before the M0 write covers the
// wait states after the v_readfirstlane that produced its operand, the one after it those of the copy reading M0.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds)
{
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_nop 4\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
                 : "memory", "m0");
}

// Calls f(std::integral_constant<int, I>) for I = 0 .. N-1 (a loop whose index is a compile-time constant).
template <int... I, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, I...>, F &&f)
{
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f)
{
    static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

// Split-K state of a launch with grid.z > 1: slots of BM x BN accumulators, tile-major then split, and one arrival
// counter per tile, zero before the launch and left at zero by it.
struct SplitArgs {
    float *part;
    uint32_t *cnt;
};

// The configurations a launch may split along K: the ones the dispatcher gives small grids. The split code is a
// separate instance of the kernel (SPLIT), so it adds no register pressure to the kernels of large grids.
template <int CT, int BM, int BN>
constexpr bool kSplittable = (CT == KUDNN_DT_F32 && BM == 64 && BN == 64) ||
                             ((CT == KUDNN_DT_BF16 || CT == KUDNN_DT_F16) && BM == 128 && BN == 128);

// CT: compute (operand) type, KUDNN_DT_F32 / BF16 / F16 / S8. SPLIT: grid.z splits K (see SplitArgs).
// BKM (fp32 only): B is stored [K][N] (N contiguous, k-row pitch ldb) and read in place. A k-tile of B is then 32
// k-rows of the tile's BN columns; the LDS DMA copies them as they lie, k-row k's 128-byte column segments in the
// order seg ^ ((k >> 2) & 1), and a lane reads its column's 4 consecutive k as 4 single floats (gfx950 has no 32-bit
// transposing LDS read). The segment order puts the two lane halves' reads (k and k + 4, see read_frags) in different
// halves of the 64 banks, so each ds_read_b32 is conflict-free. Needs K a multiple of 32, N of 4 (columns past N are
// clamped to the last whole chunk, read but never stored), 16-byte aligned k-rows and batches.
template <int CT, int BM, int BN, int WM, int WN, int ST, int ACT, int FORM, bool SPLIT = false, bool BKM = false>
__global__ __launch_bounds__(WM *WN * 64, 1) void gemm_mfma_kernel(GemmOperands op, EpiParams ep, int tilesM,
                                                                  int tilesN, int group, SplitArgs sa)
{
    constexpr bool F32 = CT == KUDNN_DT_F32;
    static_assert(!BKM || (F32 && BN >= 64), "the in-place K-major B is an fp32 path with at least two column segments");
    using T = typename std::conditional<F32, float, typename std::conditional<CT == KUDNN_DT_S8, int8_t, uint16_t>::type>::type;
    constexpr int EPC = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte chunk
    constexpr int kBK = kChunks * EPC;                      // k-tile in elements
    constexpr int NW = WM * WN;                             // waves
    constexpr int TM = BM / WM;   // wave tile rows (m)
    constexpr int TN = BN / WN;   // wave tile cols (n)
    constexpr int FM = TM / 32;   // 32x32 sub-tiles per wave along m
    constexpr int FN = TN / 32;   // ... along n
    constexpr int GA = BM / 8 / NW;  // 8-row LDS DMA groups per wave per A tile
    constexpr int GB = BN / 8 / NW;
    static_assert(GA >= 1 && GB >= 1, "tile too small for the wave count");
    static_assert(NW * TM * kStagePitch * 4 <= (BM + BN) * kChunks * 16 * ST, "epilogue staging exceeds LDS");

    // one LDS array: ST A stages, then ST B stages; reused as epilogue staging after the k-loop
    __shared__ uint4 lds[ST * (BM + BN) * kChunks];
    uint4(*sA)[BM * kChunks] = reinterpret_cast<uint4(*)[BM * kChunks]>(lds);
    uint4(*sB)[BN * kChunks] = reinterpret_cast<uint4(*)[BN * kChunks]>(lds + ST * BM * kChunks);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN;
    const int wn = wave % WN;

    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, gridDim.x), tilesM, tilesN, group, tm, tn);
    const int64_t m0 = static_cast<int64_t>(tm) * BM;
    const int64_t n0 = static_cast<int64_t>(tn) * BN;

    const int64_t batch = blockIdx.y;
    const int64_t i2 = batch % ep.bdim[2];
    const int64_t i1 = (batch / ep.bdim[2]) % ep.bdim[1];
    const int64_t i0 = batch / (ep.bdim[2] * ep.bdim[1]);
    const T *A = static_cast<const T *>(op.a) + i0 * op.a_bs[0] + i1 * op.a_bs[1] + i2 * op.a_bs[2];
    const T *B = static_cast<const T *>(op.b) + i0 * op.b_bs[0] + i1 * op.b_bs[1] + i2 * op.b_bs[2];
    const int64_t M = op.M, N = op.N, K = op.K;

    // This lane's source in every DMA group: row (8-row group base) + lane/8, logical chunk chosen so that
    // LDS slot (lane % 8) of the row holds swizzled chunk (lane % 8).
    const int lrow8 = lane >> 3;
    const int lchunk = (lane & 7) ^ lrow8;
    const T *pa[GA];
    const T *pb[GB];
#pragma unroll
    for (int j = 0; j < GA; ++j) {
        int64_t r = m0 + (wave * GA + j) * 8 + lrow8;
        r = r < M ? r : M - 1;
        pa[j] = A + r * op.lda + lchunk * EPC;
    }
#pragma unroll
    for (int j = 0; j < GB; ++j) {
        if constexpr (BKM) {
            // LDS chunk p of the B tile holds k-row p / (BN / 4), segment position (p % (BN / 4)) / 8, chunk p % 8
            constexpr int kCpr = BN / 4;  // 16-byte chunks per k-row of the tile
            const int p = (wave * GB + j) * 64 + lane;
            const int k = p / kCpr, rem = p % kCpr;
            const int seg = (rem >> 3) ^ ((k >> 2) & 1);
            int64_t n = n0 + seg * 32 + (rem & 7) * 4;
            n = n + 4 <= N ? n : N - 4;
            pb[j] = B + k * op.ldb + n;
        } else {
            int64_t r = n0 + (wave * GB + j) * 8 + lrow8;
            r = r < N ? r : N - 1;
            pb[j] = B + r * op.ldb + lchunk * EPC;
        }
    }

    // LDS byte addresses of stage 0's A and B tiles (stage s adds s * BM (BN) rows of 128 bytes)
    const uint32_t ldsA = lds_byte(&sA[0][0]), ldsB = lds_byte(&sB[0][0]);
    auto issue_tile = [&](int buf, int64_t k0) {
#pragma unroll
        for (int j = 0; j < GA; ++j) {
            dma16(pa[j] + k0, ldsA + static_cast<uint32_t>((buf * BM * kChunks + (wave * GA + j) * 64) * 16));
        }
#pragma unroll
        for (int j = 0; j < GB; ++j) {
            dma16(pb[j] + (BKM ? k0 * op.ldb : k0), ldsB + static_cast<uint32_t>((buf * BN * kChunks + (wave * GB + j) * 64) * 16));
        }
    };

    f32x16_t acc[FN][FM];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;
        }
    }

    const int lrow = lane & 31;
    const int lhalf = lane >> 5;
    // k-tiles of this launch: all of them, or split z's share of a split-K launch
    const int KTall = static_cast<int>(K / kBK);
    const int kt0 = static_cast<int>(static_cast<int64_t>(KTall) * blockIdx.z / gridDim.z);
    const int kt1 = static_cast<int>(static_cast<int64_t>(KTall) * (blockIdx.z + 1) / gridDim.z);
    const int KT = kt1 - kt0;

    // ST-stage pipeline: tiles kt+1 .. kt+ST-1 are in flight while tile kt is computed. Each tile is GA + GB
    // DMA instructions per wave and they complete in order, so "tile kt landed" is vmcnt <= (tiles issued after
    // it) * (GA + GB).
#pragma unroll
    for (int s = 0; s < ST - 1; ++s) {
        if (s < KT) {
            issue_tile(s, static_cast<int64_t>(kt0 + s) * kBK);
        }
    }
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt % ST;
        const int ahead = KT - 1 - kt < ST - 2 ? KT - 1 - kt : ST - 2;  // tiles issued after tile kt so far
        wait_tiles<GA + GB, ST>(ahead);
        // the barrier makes every wave's tile kt visible and guarantees every wave finished reading the buffer
        // of tile kt - 1, which the issue below refills
        __syncthreads();
        if (kt + ST - 1 < KT) {
            issue_tile((kt + ST - 1) % ST, static_cast<int64_t>(kt0 + kt + ST - 1) * kBK);
        }
        uint4 va[2][FM], vb[2][FN];
        auto read_frags = [&](int slot, int s) {
            const int c = s * 2 + lhalf;  // lane half h reads 16-byte chunk 2s+h of its row
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int row = wm * TM + i * 32 + lrow;
                va[slot][i] = sA[cur][row * kChunks + swz(row, c)];
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if constexpr (BKM) {
                    // column wn TN + j 32 + lrow at k = 8 s + 4 h + q, q = 0..3: segment wn TN / 32 + j, stored at
                    // position segment ^ h in k-rows 8 s + 4 h .. + 3
                    const float *col = reinterpret_cast<const float *>(&sB[cur][0]) + (8 * s + 4 * lhalf) * BN +
                                       (((wn * TN) / 32 + j) ^ lhalf) * 32 + lrow;
                    vb[slot][j] = make_uint4(__builtin_bit_cast(uint32_t, col[0]), __builtin_bit_cast(uint32_t, col[BN]),
                                             __builtin_bit_cast(uint32_t, col[2 * BN]), __builtin_bit_cast(uint32_t, col[3 * BN]));
                } else {
                    const int row = wn * TN + j * 32 + lrow;
                    vb[slot][j] = sB[cur][row * kChunks + swz(row, c)];
                }
            }
        };
        read_frags(0, 0);
#pragma unroll
        for (int s = 0; s < kChunks / 2; ++s) {
            if (s + 1 < kChunks / 2) {
                read_frags((s + 1) & 1, s + 1);
            }
            // Keep the next substep's LDS reads ahead of this substep's MFMAs (the scheduler would
            // otherwise sink them next to their uses and expose the LDS latency every few MFMAs).
            __builtin_amdgcn_sched_barrier(0);
            const int sl = s & 1;
            if constexpr (F32) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
#pragma unroll
                        for (int i = 0; i < FM; ++i) {
                            const f32x4_t a4 = __builtin_bit_cast(f32x4_t, va[sl][i]);
                            const f32x4_t b4 = __builtin_bit_cast(f32x4_t, vb[sl][j]);
                            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(b4[q], a4[q], acc[j][i], 0, 0, 0);
                        }
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        if constexpr (CT == KUDNN_DT_BF16) {
                            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(bf16x8_t, vb[sl][j]), __builtin_bit_cast(bf16x8_t, va[sl][i]), acc[j][i], 0, 0, 0);
                        } else if constexpr (CT == KUDNN_DT_F16) {
                            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                                __builtin_bit_cast(f16x8_t, vb[sl][j]), __builtin_bit_cast(f16x8_t, va[sl][i]), acc[j][i], 0, 0, 0);
                        } else {
                            acc[j][i] = __builtin_bit_cast(
                                f32x16_t, __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, vb[sl][j]),
                                                                               __builtin_bit_cast(i32x4_t, va[sl][i]),
                                                                               __builtin_bit_cast(i32x16_t, acc[j][i]), 0, 0, 0));
                        }
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Split-K: this split's accumulators go to its slot with agent-scope atomic stores (coherent across the XCDs' L2
    // caches access by access; a device-scope fence would write back and invalidate a whole L2), every wave waits for
    // its stores, and one ticket per split is drawn. The holder of the last ticket rebuilds the sum in split order.
    if constexpr (SPLIT) {
        {
            constexpr int QPW = FN * FM * 4;  // 16-byte quads of accumulators per lane
            constexpr int64_t kSlot = static_cast<int64_t>(BM) * BN / 2;  // uint64 per slot
            uint64_t *tileSlots = reinterpret_cast<uint64_t *>(sa.part) + static_cast<int64_t>(blockIdx.x) * gridDim.z * kSlot;
            auto at = [&](uint64_t *slot, int qd) { return slot + 2 * ((wave * QPW + qd) * 64 + lane); };
            uint64_t *mine = tileSlots + static_cast<int64_t>(blockIdx.z) * kSlot;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
#pragma unroll
                for (int i = 0; i < FM; ++i) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        uint64_t *d = at(mine, (j * FM + i) * 4 + g);
                        // the elements are copied out first: __builtin_bit_cast applied to an element of an
                        // ext_vector_type reads element 0 with this compiler
                        const float e0 = acc[j][i][4 * g], e1 = acc[j][i][4 * g + 1];
                        const float e2 = acc[j][i][4 * g + 2], e3 = acc[j][i][4 * g + 3];
                        const uint64_t lo = static_cast<uint64_t>(__builtin_bit_cast(uint32_t, e0)) |
                                            (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, e1)) << 32);
                        const uint64_t hi = static_cast<uint64_t>(__builtin_bit_cast(uint32_t, e2)) |
                                            (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, e3)) << 32);
                        __hip_atomic_store(d, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_store(d + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's part has reached the coherence point
            __syncthreads();                     // also: every wave is past the k-loop's LDS reads
            uint32_t *ticket = reinterpret_cast<uint32_t *>(lds);
            if (tid == 0) {
                // system scope: the add is performed past the XCDs' private L2 caches
                ticket[0] = __hip_atomic_fetch_add(&sa.cnt[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            __syncthreads();
            if (ticket[0] != gridDim.z - 1) {
                return;  // another split finishes this tile
            }
            // CH slots are loaded together (as many as the registers allow), then added in split order
            constexpr int NACC = FN * FM * 16;
            constexpr int CH = NACC <= 16 ? 4 : (NACC <= 64 ? 2 : 1);
            const int splits = static_cast<int>(gridDim.z);
            for (int z0 = 0; z0 < splits; z0 += CH) {
                uint64_t buf[CH][FN][FM][4][2];
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    if (z0 + c < splits) {
                        uint64_t *part = tileSlots + static_cast<int64_t>(z0 + c) * kSlot;
#pragma unroll
                        for (int j = 0; j < FN; ++j) {
#pragma unroll
                            for (int i = 0; i < FM; ++i) {
#pragma unroll
                                for (int g = 0; g < 4; ++g) {
                                    uint64_t *src = at(part, (j * FM + i) * 4 + g);
                                    buf[c][j][i][g][0] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                    buf[c][j][i][g][1] = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                }
                            }
                        }
                    }
                }
#pragma unroll
                for (int c = 0; c < CH; ++c) {
                    if (z0 + c < splits) {
#pragma unroll
                        for (int j = 0; j < FN; ++j) {
#pragma unroll
                            for (int i = 0; i < FM; ++i) {
#pragma unroll
                                for (int g = 0; g < 4; ++g) {
                                    const uint64_t lo = buf[c][j][i][g][0], hi = buf[c][j][i][g][1];
                                    const float o[4] = {__builtin_bit_cast(float, static_cast<uint32_t>(lo)),
                                                        __builtin_bit_cast(float, static_cast<uint32_t>(lo >> 32)),
                                                        __builtin_bit_cast(float, static_cast<uint32_t>(hi)),
                                                        __builtin_bit_cast(float, static_cast<uint32_t>(hi >> 32))};
#pragma unroll
                                    for (int e = 0; e < 4; ++e) {
                                        acc[j][i][4 * g + e] = z0 + c == 0 ? o[e] : acc[j][i][4 * g + e] + o[e];
                                    }
                                }
                            }
                        }
                    }
                }
            }
            if (tid == 0) {
                __hip_atomic_store(&sa.cnt[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);  // next launch
            }
        }
    }

    // Epilogue through LDS, one 32-column strip of each wave tile at a time. The strip index is a
    // compile-time constant (static_for) so the accumulators stay in registers. Lanes then read the strip
    // back row-major: 4 lanes per row, 8 columns per lane, 16 rows per pass.
    float *stage = reinterpret_cast<float *>(lds) + wave * (TM * kStagePitch);
    const EpiBatch ob = epi_batch_offsets(ep, batch);
    const bool full = m0 + BM <= M && n0 + BN <= N;
    const int col8 = (lane & 3) * 8;
    static_for<FN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        __syncthreads();  // previous strip fully read back (and, for j = 0, the k-loop's last LDS reads done)
#pragma unroll
        for (int i = 0; i < FM; ++i) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float *dst = stage + (i * 32 + lrow) * kStagePitch + g * 8 + lhalf * 4;
                *reinterpret_cast<float4 *>(dst) =
                    make_float4(acc[j][i][4 * g + 0], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]);
            }
        }
        __syncthreads();
        const int64_t n = n0 + wn * TN + j * 32 + col8;
        if constexpr (FORM == EPI_FORM_I32) {
#pragma unroll 1
            for (int r = lane >> 2; r < TM; r += 16) {
                const int64_t m = m0 + wm * TM + r;
                const float *src = stage + r * kStagePitch + col8;
                if (ep.fast8 && (full || (m < M && n + 7 < N))) {
                    const float4 lo = *reinterpret_cast<const float4 *>(src);
                    const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
                    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                    epi_i32_8(ep, ob, m, n, v);
                } else if (m < M) {
#pragma unroll 1
                    for (int q = 0; q < 8; ++q) {
                        if (n + q < N) {
                            epi_i32_1(ep, ob, m, n + q, src[q]);
                        }
                    }
                }
            }
        } else if constexpr (FORM == EPI_FORM_GENERIC) {
#pragma unroll 1
            for (int r = lane >> 2; r < TM; r += 16) {
                const int64_t m = m0 + wm * TM + r;
                if (m >= M) {
                    continue;
                }
                const float *src = stage + r * kStagePitch + col8;
#pragma unroll 1
                for (int q = 0; q < 8; ++q) {
                    if (n + q < N) {
                        epi_apply(ep, ob, m, n + q, src[q]);
                    }
                }
            }
        } else {
#pragma unroll 1
            for (int r = lane >> 2; r < TM; r += 16) {
                const int64_t m = m0 + wm * TM + r;
                const float *src = stage + r * kStagePitch + col8;
                if (full || (m < M && n + 7 < N)) {
                    const Pre8 pre = epi_prefetch8<FORM>(ep, ob, m, n);
                    const float4 lo = *reinterpret_cast<const float4 *>(src);
                    const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
                    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                    epi_fast8<ACT, FORM>(ep, ob, m, n, v, pre);
                } else if (m < M) {
#pragma unroll 1
                    for (int q = 0; q < 8; ++q) {
                        if (n + q < N) {
                            epi_elem<ACT, FORM>(ep, ob, m, n + q, src[q]);
                        }
                    }
                }
            }
        }
    });
}

// Split-K factor of a launch: the tiles cover less than half of the 256 CUs and each split keeps at least 4 k-tiles.
// A split launch therefore has fewer than kSplitMaxTiles tiles, one arrival counter each.
int splitk_splits(const GemmOperands &op, int64_t batches, int BM, int BN, int kBK)
{
    const int64_t tiles = ((op.M + BM - 1) / BM) * ((op.N + BN - 1) / BN) * batches;
    const int64_t KT = op.K / kBK;
    if (batches != 1 || tiles >= KUDNN_SPLIT_MAX_TILES || KT < 8) {
        return 1;
    }
    return static_cast<int>(std::min<int64_t>(KT / 4, (384 + tiles - 1) / tiles));
}

// Launches the variant of the kernel that the epilogue's activation and tensor types select.
template <int CT, int BM, int BN, int WM, int WN, int ST, bool SPLIT, bool BKM = false>
int launch_kernel(const GemmOperands &op, const EpiParams &ep, dim3 grid, int group, int tilesM, int tilesN,
                  const SplitArgs &sa, hipStream_t stream)
{
    decltype(&gemm_mfma_kernel<CT, BM, BN, WM, WN, ST, 0, EPI_FORM_GENERIC, SPLIT, BKM>) kernel = nullptr;
    // the fixed form compiled for this compute type
    constexpr int kForm = CT == KUDNN_DT_F32 ? EPI_FORM_F32 : (CT == KUDNN_DT_F16 ? EPI_FORM_F16 : EPI_FORM_BF16);
    if (epi_form(ep) == kForm) {
        switch (ep.act) {
            case KUDNN_ACT_UNIMPLEMENTED:
                kernel = gemm_mfma_kernel<CT, BM, BN, WM, WN, ST, KUDNN_ACT_UNIMPLEMENTED, kForm, SPLIT, BKM>;
                break;
            case KUDNN_ACT_RELU: kernel = gemm_mfma_kernel<CT, BM, BN, WM, WN, ST, KUDNN_ACT_RELU, kForm, SPLIT, BKM>; break;
            case KUDNN_ACT_SWISH: kernel = gemm_mfma_kernel<CT, BM, BN, WM, WN, ST, KUDNN_ACT_SWISH, kForm, SPLIT, BKM>; break;
            case KUDNN_ACT_GELU_TANH:
                kernel = gemm_mfma_kernel<CT, BM, BN, WM, WN, ST, KUDNN_ACT_GELU_TANH, kForm, SPLIT, BKM>;
                break;
            case KUDNN_ACT_GELU_ERF:
                kernel = gemm_mfma_kernel<CT, BM, BN, WM, WN, ST, KUDNN_ACT_GELU_ERF, kForm, SPLIT, BKM>;
                break;
            default: break;
        }
    }
    if (kernel == nullptr) {
        kernel = gemm_mfma_kernel<CT, BM, BN, WM, WN, ST, 0, EPI_FORM_GENERIC, SPLIT, BKM>;  // activation read at run time
    }
    hipLaunchKernelGGL(kernel, grid, dim3(WM * WN * 64), 0, stream, op, ep, tilesM, tilesN, group, sa);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int CT, int BM, int BN, int WM, int WN, int ST>
int launch_cfg(const GemmOperands &op, const EpiParams &ep, int64_t batches, int group, void *ws, uint32_t *counters,
               hipStream_t stream)
{
    constexpr int kBK = CT == KUDNN_DT_F32 ? 32 : (CT == KUDNN_DT_S8 ? 128 : 64);
    if (op.K % kBK != 0) {
        return -1;  // the dispatcher pads K by packing
    }
    const int tilesM = static_cast<int>((op.M + BM - 1) / BM);
    const int tilesN = static_cast<int>((op.N + BN - 1) / BN);
    dim3 block(WM * WN * 64);
    dim3 grid(static_cast<unsigned>(tilesM * tilesN), static_cast<unsigned>(batches));
    if constexpr (CT == KUDNN_DT_S8) {
        // integer accumulators: no split-K (its partials are f32), one epilogue
        if (epi_form(ep) != EPI_FORM_I32) {
            return -1;
        }
        hipLaunchKernelGGL((gemm_mfma_kernel<CT, BM, BN, WM, WN, ST, 0, EPI_FORM_I32>), grid, block, 0, stream, op, ep,
                           tilesM, tilesN, group, SplitArgs{});
        return hipGetLastError() == hipSuccess ? 0 : -1;
    } else {
        // split-K: grid.z splits, slots in the workspace, one arrival counter per tile
        const int splits = kSplittable<CT, BM, BN> && ws != nullptr && counters != nullptr
                               ? splitk_splits(op, batches, BM, BN, kBK) : 1;
        SplitArgs sa{};
        if (splits > 1) {
            grid.z = static_cast<unsigned>(splits);
            sa.part = static_cast<float *>(ws);
            sa.cnt = counters;
        }
        if constexpr (CT == KUDNN_DT_F32) {
            if (op.b_kmajor) {
                // the weight read in place as [K][N] (the planner checked the kernel's requirements)
                if constexpr (kSplittable<CT, BM, BN>) {
                    if (splits > 1) {
                        return launch_kernel<CT, BM, BN, WM, WN, ST, true, true>(op, ep, grid, group, tilesM, tilesN, sa, stream);
                    }
                }
                return launch_kernel<CT, BM, BN, WM, WN, ST, false, true>(op, ep, grid, group, tilesM, tilesN, sa, stream);
            }
        } else if (op.b_kmajor) {
            return -1;  // only the ping-pong kernel reads a 16-bit K-major weight
        }
        if constexpr (kSplittable<CT, BM, BN>) {
            if (splits > 1) {
                return launch_kernel<CT, BM, BN, WM, WN, ST, true>(op, ep, grid, group, tilesM, tilesN, sa, stream);
            }
        }
        return launch_kernel<CT, BM, BN, WM, WN, ST, false>(op, ep, grid, group, tilesM, tilesN, sa, stream);
    }
}

}  // namespace

size_t kudnn_gemm_workspace_bytes(const GemmOperands &op, int64_t batches, int cfg, int ct)
{
    if (ct == KUDNN_DT_S8) {
        return 0;  // integer launches are never split
    }
    int bm = 0, bn = 0, bk = 0;
    switch (cfg) {  // the configurations that may split (kSplittable)
        case KUDNN_CFG_BF16_128x128: bm = 128; bn = 128; bk = 64; break;
        case KUDNN_CFG_F32_64x64: bm = 64; bn = 64; bk = 32; break;
        default: return 0;
    }
    if ((ct == KUDNN_DT_F32) != (cfg == KUDNN_CFG_F32_64x64)) {
        return 0;
    }
    const int splits = splitk_splits(op, batches, bm, bn, bk);
    const int64_t tiles = ((op.M + bm - 1) / bm) * ((op.N + bn - 1) / bn);
    return splits > 1 ? static_cast<size_t>(tiles) * splits * bm * bn * sizeof(float) : 0;
}

namespace {

template <int CT>
int launch_lowp(const GemmOperands &op, const EpiParams &ep, int64_t batches, int cfg, void *ws, uint32_t *counters,
                hipStream_t stream)
{
    switch (cfg) {
        case KUDNN_CFG_BF16_256x256: return launch_cfg<CT, 256, 256, 2, 2, 2>(op, ep, batches, 8, ws, counters, stream);
        case KUDNN_CFG_BF16_256x128: return launch_cfg<CT, 256, 128, 2, 2, 3>(op, ep, batches, 8, ws, counters, stream);
        case KUDNN_CFG_BF16_128x128: return launch_cfg<CT, 128, 128, 2, 2, 4>(op, ep, batches, 8, ws, counters, stream);
        default: return -1;
    }
}

}  // namespace

int kudnn_launch_gemm_mfma(const GemmOperands &op, const EpiParams &ep, int64_t batches, int cfg, int ct, void *ws,
                           uint32_t *counters, hipStream_t stream)
{
    switch (ct) {
        case KUDNN_DT_BF16: return launch_lowp<KUDNN_DT_BF16>(op, ep, batches, cfg, ws, counters, stream);
        case KUDNN_DT_F16: return launch_lowp<KUDNN_DT_F16>(op, ep, batches, cfg, ws, counters, stream);
        case KUDNN_DT_S8: return launch_lowp<KUDNN_DT_S8>(op, ep, batches, cfg, nullptr, nullptr, stream);
        default: return -1;
    }
}

int kudnn_launch_gemm_f32(const GemmOperands &op, const EpiParams &ep, int64_t batches, int cfg, void *ws,
                          uint32_t *counters, hipStream_t stream)
{
    switch (cfg) {
        // 128 x 128 serves grids of >= 256 tiles: two stages keep two workgroups per CU, which hides latency better
        // than a deeper ring at one workgroup per CU
        case KUDNN_CFG_F32_128x128:
            return launch_cfg<KUDNN_DT_F32, 128, 128, 2, 2, 2>(op, ep, batches, 8, ws, counters, stream);
        case KUDNN_CFG_F32_64x64: return launch_cfg<KUDNN_DT_F32, 64, 64, 2, 2, 4>(op, ep, batches, 8, ws, counters, stream);
        default: return -1;
    }
}
