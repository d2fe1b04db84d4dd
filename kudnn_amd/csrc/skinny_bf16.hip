// Skinny-M (M <= 16) bf16 Linear for decode-shaped calls: Y = epilogue(X[M][K] x W[N][K]^T).
//
// The reference reaches cblas_sgemv for m == 1 (src/dnn/src/kudnn_gemm.cpp:164-173) and cblas_sbgemm /
// cblas_bgemm otherwise (:208-241). On MI355X this shape is bound by streaming W from HBM once, so the
// kernel is organised around the weight stream, not around compute:
//  - a workgroup owns 16 weight rows (n) and all of K; its KW waves split K into KW contiguous ranges;
//  - each lane loads 16-byte chunks of W straight from global memory into the register layout of
//    v_mfma_f32_16x16x32_bf16 (lane l: row l%16, k-chunk l/16; a wave instruction reads 16 rows x 64
//    contiguous bytes), UNR k-steps are issued back to back to keep enough bytes in flight;
//  - X rows (m < M, tiny and cache-resident) form the second MFMA operand; lanes with m >= M feed zeros;
//  - the KW partial 16x16 tiles are summed through LDS and wave 0 runs the fused epilogue.
#include "device_common.h"
#include "kernels.h"

using namespace kudnn_dev;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int KW, int UNR, bool KTAIL>
__global__ __launch_bounds__(KW * 64) void skinny_bf16_kernel(GemmOperands op, EpiParams ep)
{
    __shared__ f32x4_t part[KW][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t M = op.M, N = op.N, K = op.K;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;

    const int64_t batch = blockIdx.y;
    const int64_t i2 = batch % ep.bdim[2];
    const int64_t i1 = (batch / ep.bdim[2]) % ep.bdim[1];
    const int64_t i0 = batch / (ep.bdim[2] * ep.bdim[1]);
    const uint16_t *X = static_cast<const uint16_t *>(op.a) + i0 * op.a_bs[0] + i1 * op.a_bs[1] + i2 * op.a_bs[2];
    const uint16_t *W = static_cast<const uint16_t *>(op.b) + i0 * op.b_bs[0] + i1 * op.b_bs[1] + i2 * op.b_bs[2];

    const int r16 = lane & 15;
    const int q = lane >> 4;  // k-chunk within a 32-wide k step
    int64_t wrow = n0 + r16;
    wrow = wrow < N ? wrow : N - 1;
    const bool xrow_ok = r16 < M;
    const uint16_t *wp = W + wrow * op.ldb + q * 8;
    const uint16_t *xp = X + (xrow_ok ? r16 : 0) * op.lda + q * 8;

    // k-steps of 32 owned by this wave
    const int64_t steps = (K + 31) / 32;
    const int64_t sBeg = steps * wave / KW;
    const int64_t sEnd = steps * (wave + 1) / KW;

    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t s = sBeg; s < sEnd; s += UNR) {
        u32x4_t wv[UNR], xv[UNR];
        const u32x4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int64_t k = (s + u) * 32 + q * 8;
            const bool ok = (s + u < sEnd) && (!KTAIL || k < K);
            wv[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(wp + (s + u) * 32)) : zero;
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int64_t k = (s + u) * 32 + q * 8;
            const bool ok = xrow_ok && (s + u < sEnd) && (!KTAIL || k < K);
            xv[u] = ok ? *reinterpret_cast<const u32x4_t *>(xp + (s + u) * 32) : zero;
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, wv[u]),
                                                          __builtin_bit_cast(bf16x8_t, xv[u]), acc, 0, 0, 0);
        }
    }

    part[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) {
        return;
    }
    f32x4_t sum = part[0][lane];
#pragma unroll
    for (int w = 1; w < KW; ++w) {
        f32x4_t p = part[w][lane];
        sum[0] += p[0];
        sum[1] += p[1];
        sum[2] += p[2];
        sum[3] += p[3];
    }
    // lane holds D[n = n0 + 4*q + r][m = r16], r = 0..3
    if (r16 >= M) {
        return;
    }
    const int64_t n = n0 + 4 * q;
    if (n >= N) {
        return;
    }
    const EpiBatch ob = epi_batch_offsets(ep, batch);
    const float v[4] = {sum[0], sum[1], sum[2], sum[3]};
    epi_apply4(ep, ob, r16, n, N, v);
}

template <int KW, int UNR>
int launch(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream)
{
    dim3 grid(static_cast<unsigned>((op.N + 15) / 16), static_cast<unsigned>(batches));
    dim3 block(KW * 64);
    if (op.K % 32 == 0) {
        hipLaunchKernelGGL((skinny_bf16_kernel<KW, UNR, false>), grid, block, 0, stream, op, ep);
    } else {
        hipLaunchKernelGGL((skinny_bf16_kernel<KW, UNR, true>), grid, block, 0, stream, op, ep);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int kudnn_launch_skinny_bf16(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream)
{
    if (op.M > 16) {
        return -1;
    }
    // Few weight row-groups: split K over 8 waves per workgroup to keep more loads in flight.
    const int64_t groups = (op.N + 15) / 16 * batches;
    if (groups < 1024) {
        return launch<8, 8>(op, ep, batches, stream);
    }
    return launch<4, 8>(op, ep, batches, stream);
}
