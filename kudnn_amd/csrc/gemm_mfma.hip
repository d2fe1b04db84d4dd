// bf16 and fp32 GEMM on gfx950 MFMA with the fused epilogue.
//
// Computes, per batch, Y = epilogue(A[M][K] x B[N][K]^T) with both operands contiguous along K
// (A = activations/X rows, B = nn.Linear-style weight rows). This is the kernel behind cblas_sbgemm /
// cblas_bgemm (bf16) and cblas_sgemm (fp32) in the reference (src/dnn/src/kudnn_gemm.cpp:157-241) plus
// its post-op passes.
//
// Design (one workgroup per BM x BN output tile, 4 waves as 2 x 2):
//  - A and B k-tiles of 128 bytes per row (64 bf16 / 32 fp32) are staged global -> registers -> LDS,
//    double buffered: the global loads of tile k+1 are in flight while the MFMAs of tile k run; one
//    barrier per k-tile.
//  - LDS rows are 128 B with the 16-byte chunk index XOR-swizzled by (row & 7), so the ds_read_b128 of
//    32 consecutive rows at one k-chunk hits every bank once.
//  - bf16: v_mfma_f32_32x32x16_bf16; fp32: v_mfma_f32_32x32x2f32 fed from one 16-byte LDS read per lane
//    (four k values; MFMA q consumes element q of both lane halves, which covers every k exactly once).
//  - The operands are swapped (weight tile as the first MFMA operand): each lane then owns, per 32x32
//    sub-tile, one output row m and four runs of four consecutive columns n, so the epilogue issues
//    8-byte (bf16) / 16-byte (f32) stores and residual loads.
//  - Blocks are remapped so consecutive tiles run on the same XCD and walked in groups of tile-rows.
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

using namespace kudnn_dev;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kChunks = 8;   // 16-byte chunks per 128-byte LDS row

__device__ __forceinline__ int swz(int row, int chunk) { return (chunk ^ (row & 7)); }

template <bool F32, int BM, int BN, int WM, int WN, bool KTAIL>
__global__ __launch_bounds__(WM *WN * 64, 1) void gemm_mfma_kernel(GemmOperands op, EpiParams ep, int tilesM,
                                                                  int tilesN, int group)
{
    using T = typename std::conditional<F32, float, uint16_t>::type;
    constexpr int EPC = 16 / static_cast<int>(sizeof(T));  // elements per 16-byte chunk
    constexpr int kBK = kChunks * EPC;                      // k-tile in elements
    constexpr int NT = WM * WN * 64;
    constexpr int TM = BM / WM;   // wave tile rows (m)
    constexpr int TN = BN / WN;   // wave tile cols (n)
    constexpr int FM = TM / 32;   // 32x32 sub-tiles per wave along m
    constexpr int FN = TN / 32;   // ... along n
    constexpr int CA = BM * kChunks / NT;  // 16-byte chunks per thread per A tile
    constexpr int CB = BN * kChunks / NT;
    constexpr int ROWS_PER_PASS = NT / kChunks;

    __shared__ uint4 sA[2][BM * kChunks];
    __shared__ uint4 sB[2][BN * kChunks];

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

    // Per-thread global source rows (clamped into range; out-of-range rows are never stored).
    const int chunk = tid & (kChunks - 1);
    const int rowBase = tid / kChunks;
    const T *pa[CA];
    const T *pb[CB];
#pragma unroll
    for (int j = 0; j < CA; ++j) {
        int64_t r = m0 + rowBase + j * ROWS_PER_PASS;
        r = r < M ? r : M - 1;
        pa[j] = A + r * op.lda + chunk * EPC;
    }
#pragma unroll
    for (int j = 0; j < CB; ++j) {
        int64_t r = n0 + rowBase + j * ROWS_PER_PASS;
        r = r < N ? r : N - 1;
        pb[j] = B + r * op.ldb + chunk * EPC;
    }

    uint4 ra[CA], rb[CB];
    auto load_tile = [&](int64_t k0) {
        const bool inK = !KTAIL || (k0 + chunk * EPC < K);
#pragma unroll
        for (int j = 0; j < CA; ++j) {
            ra[j] = inK ? *reinterpret_cast<const uint4 *>(pa[j] + k0) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            rb[j] = inK ? *reinterpret_cast<const uint4 *>(pb[j] + k0) : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int j = 0; j < CA; ++j) {
            int row = rowBase + j * ROWS_PER_PASS;
            sA[buf][row * kChunks + swz(row, chunk)] = ra[j];
        }
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            int row = rowBase + j * ROWS_PER_PASS;
            sB[buf][row * kChunks + swz(row, chunk)] = rb[j];
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

    const int KT = static_cast<int>((K + kBK - 1) / kBK);
    load_tile(0);
    store_tile(0);
    __syncthreads();

    const int lrow = lane & 31;
    const int lhalf = lane >> 5;
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) {
            load_tile(static_cast<int64_t>(kt + 1) * kBK);
        }
#pragma unroll
        for (int s = 0; s < kChunks / 2; ++s) {
            // lane half h reads 16-byte chunk 2s+h of its row
            const int c = s * 2 + lhalf;
            uint4 va[FM], vb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                int row = wm * TM + i * 32 + lrow;
                va[i] = sA[cur][row * kChunks + swz(row, c)];
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                int row = wn * TN + j * 32 + lrow;
                vb[j] = sB[cur][row * kChunks + swz(row, c)];
            }
            if constexpr (F32) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
#pragma unroll
                        for (int i = 0; i < FM; ++i) {
                            f32x4_t a4 = __builtin_bit_cast(f32x4_t, va[i]);
                            f32x4_t b4 = __builtin_bit_cast(f32x4_t, vb[j]);
                            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x2f32(b4[q], a4[q], acc[j][i], 0, 0, 0);
                        }
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vb[j]),
                                                                            __builtin_bit_cast(bf16x8_t, va[i]),
                                                                            acc[j][i], 0, 0, 0);
                    }
                }
            }
        }
        if (kt + 1 < KT) {
            store_tile(cur ^ 1);
        }
        __syncthreads();
    }

    // Epilogue. Sub-tile (j, i): lane holds output row m = ... + (lane & 31) and, for register group g,
    // columns n = ... + 8g + 4*(lane >> 5) + {0,1,2,3}.
    const EpiBatch ob = epi_batch_offsets(ep, batch);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int64_t m = m0 + wm * TM + i * 32 + lrow;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int64_t n = n0 + wn * TN + j * 32 + g * 8 + lhalf * 4;
                if (n >= N) continue;
                float v[4] = {acc[j][i][4 * g + 0], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]};
                epi_apply4(ep, ob, m, n, N, v);
            }
        }
    }
}

template <bool F32, int BM, int BN, int WM, int WN>
int launch_cfg(const GemmOperands &op, const EpiParams &ep, int64_t batches, int group, hipStream_t stream)
{
    constexpr int kBK = F32 ? 32 : 64;
    int tilesM = static_cast<int>((op.M + BM - 1) / BM);
    int tilesN = static_cast<int>((op.N + BN - 1) / BN);
    dim3 grid(static_cast<unsigned>(tilesM * tilesN), static_cast<unsigned>(batches));
    dim3 block(WM * WN * 64);
    if (op.K % kBK == 0) {
        hipLaunchKernelGGL((gemm_mfma_kernel<F32, BM, BN, WM, WN, false>), grid, block, 0, stream, op, ep, tilesM,
                           tilesN, group);
    } else {
        hipLaunchKernelGGL((gemm_mfma_kernel<F32, BM, BN, WM, WN, true>), grid, block, 0, stream, op, ep, tilesM,
                           tilesN, group);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int kudnn_launch_gemm_bf16(const GemmOperands &op, const EpiParams &ep, int64_t batches, int cfg, hipStream_t stream)
{
    switch (cfg) {
        case KUDNN_CFG_BF16_256x256: return launch_cfg<false, 256, 256, 2, 2>(op, ep, batches, 8, stream);
        case KUDNN_CFG_BF16_256x128: return launch_cfg<false, 256, 128, 2, 2>(op, ep, batches, 8, stream);
        case KUDNN_CFG_BF16_128x128: return launch_cfg<false, 128, 128, 2, 2>(op, ep, batches, 8, stream);
        default: return -1;
    }
}

int kudnn_launch_gemm_f32(const GemmOperands &op, const EpiParams &ep, int64_t batches, int cfg, hipStream_t stream)
{
    switch (cfg) {
        case KUDNN_CFG_F32_128x128: return launch_cfg<true, 128, 128, 2, 2>(op, ep, batches, 8, stream);
        case KUDNN_CFG_F32_64x64: return launch_cfg<true, 64, 64, 2, 2>(op, ep, batches, 8, stream);
        default: return -1;
    }
}
