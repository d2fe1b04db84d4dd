// f32 GEMM for grids too small to fill the chip with output tiles (the fp32 Linear of the reference's
// LinearActivationTests, 128 x 1024 x 1024, is 32 tiles of 64 x 64): one workgroup per 16 x 32 output tile, its NW
// waves splitting K into interleaved 16-element chunks (chunk c goes to wave c % NW). Each wave accumulates the whole
// 16 x 32 tile on v_mfma_f32_16x16x4_f32 from operands loaded straight into registers, the NW partial tiles are summed
// through LDS in wave order, and the generic epilogue stores the tile. There is no workspace and no hand-off between
// workgroups, so the kernel's latency is one pass of loads and MFMAs plus one LDS reduction.
//
// Operand layout: A [M][K] and B [N][K], both contiguous along K, 16-byte aligned rows, K a multiple of 16 (the
// planner packs otherwise, with zero padding up to a whole number of 32-element k-tiles).
//
// MFMA operand order. v_mfma_f32_16x16x4_f32 takes one A element (row lane % 16, k lane / 16) and one B element
// (column lane % 16, k lane / 16) per lane. A lane loads 4 consecutive k of its row as one 16-byte access: lane
// (r, q) = (lane % 16, lane / 16) holds k = 16c + 4q + s, s = 0..3, of A row r and of B rows j and j + 16. MFMA step s
// feeds element s of those vectors, so step s sums over k = 16c + 4q + s, q = 0..3, and the four steps cover the chunk's
// 16 k once each (the same permutation on both operands).
#include <hip/hip_runtime.h>

#include "device_common.h"
#include "kernels.h"

namespace {

using namespace kudnn_dev;

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTM = 16, kTN = 32;  // output tile
constexpr int kChunk = 16;         // k per chunk (one 16-byte load per lane per operand row group)
constexpr int kAhead = 2;          // chunks per batch of loads (two batches in flight; more in flight measured slower)

// ACT / FORM: a fixed epilogue form (the activation and the tensor types compiled in) or EPI_FORM_GENERIC. The generic
// epilogue is a long chain of run-time branches whose first pass on each CU misses the instruction cache: for a
// kernel this short that is a large part of its time, so the common forms are compiled out.
template <int NW, int ACT, int FORM>
__device__ __forceinline__ void kslice_body(const GemmOperands &op, const EpiParams &ep, int tilesN)
{
    constexpr int kPer = kTM * kTN / (NW * 64);  // output elements per thread in the epilogue
    static_assert(kPer * NW * 64 == kTM * kTN, "the tile must divide over the threads");
    __shared__ f32x4_t part[NW][2][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: the K loop's branches are scalar
    const int tm = static_cast<int>(blockIdx.x) / tilesN, tn = static_cast<int>(blockIdx.x) % tilesN;
    const int64_t m0 = static_cast<int64_t>(tm) * kTM, n0 = static_cast<int64_t>(tn) * kTN;
    const int64_t batch = blockIdx.y;
    int64_t aoff = 0, boff = 0;
    if (gridDim.y > 1) {
        const int64_t i2 = batch % ep.bdim[2];
        const int64_t i1 = (batch / ep.bdim[2]) % ep.bdim[1];
        const int64_t i0 = batch / (ep.bdim[2] * ep.bdim[1]);
        aoff = i0 * op.a_bs[0] + i1 * op.a_bs[1] + i2 * op.a_bs[2];
        boff = i0 * op.b_bs[0] + i1 * op.b_bs[1] + i2 * op.b_bs[2];
    }
    // A fixed form's epilogue operands (f32 bias and binary operand) of this thread's output elements, loaded now so
    // that their latency overlaps the K loop. No branch guards these loads: a missing tensor reads A's first element
    // instead (a valid address; the value is not used) and an element outside the tile's valid range reads the
    // nearest valid one. Element t of the tile is D[4 * (l / 16) + e][16 * h + l % 16] with l = t % 64,
    // e = (t / 64) % 4, h = t / 256: the layout the partial tiles are summed in below.
    const EpiBatch ob = gridDim.y > 1 ? epi_batch_offsets(ep, batch) : EpiBatch{0, 0, 0, 0, 0, 0};
    EpiPre1 pre[kPer];
    if constexpr (FORM != EPI_FORM_GENERIC) {
        const float *fa = static_cast<const float *>(op.a);
        const float *pbias = ep.bias != nullptr ? static_cast<const float *>(ep.bias) : fa;
        const float *psrc = ep.bin != KUDNN_BINARY_NONE ? static_cast<const float *>(ep.src) : fa;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int t = threadIdx.x + i * NW * 64;
            const int l = t & 63, e = (t >> 6) & 3, h = t >> 8;
            const int64_t m = min(m0 + 4 * (l >> 4) + e, op.M - 1), n = min(n0 + 16 * h + (l & 15), op.N - 1);
            const int64_t bi = ep.bias != nullptr ? ob.bias + m * ep.bias_sm + n * ep.bias_sn : 0;
            const int64_t si = ep.bin != KUDNN_BINARY_NONE ? ob.src + m * ep.src_sm + n * ep.src_sn : 0;
            pre[i] = EpiPre1{0u, __float_as_uint(pbias[bi]), __float_as_uint(psrc[si])};
        }
    }

    const int r = lane & 15, q = lane >> 4;
    // rows past M or N load the last row (in bounds; their results are not stored)
    const int64_t ar = m0 + r < op.M ? m0 + r : op.M - 1;
    const int64_t b0 = n0 + r < op.N ? n0 + r : op.N - 1;
    const int64_t b1 = n0 + 16 + r < op.N ? n0 + 16 + r : op.N - 1;
    const float *pa = static_cast<const float *>(op.a) + aoff + ar * op.lda + 4 * q;
    const float *pb0 = static_cast<const float *>(op.b) + boff + b0 * op.ldb + 4 * q;
    const float *pb1 = static_cast<const float *>(op.b) + boff + b1 * op.ldb + 4 * q;

    const int chunks = static_cast<int>(op.K / kChunk);
    constexpr int kStep = NW * kAhead;  // chunks between a wave's consecutive batches
    f32x4_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    // batch at chunk c0: chunks c0 + u * NW, u < kAhead; chunks past K are skipped (`wave` is uniform, so the test is
    // a scalar branch and the waits before the MFMAs still count only the loads they need)
    auto load = [&](int c0, f32x4_t (&va)[kAhead], f32x4_t (&vb0)[kAhead], f32x4_t (&vb1)[kAhead]) {
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            const int c = c0 + u * NW;
            if (c < chunks) {
                const int64_t k = static_cast<int64_t>(c) * kChunk;
                va[u] = *reinterpret_cast<const f32x4_t *>(pa + k);
                vb0[u] = *reinterpret_cast<const f32x4_t *>(pb0 + k);
                vb1[u] = *reinterpret_cast<const f32x4_t *>(pb1 + k);
            }
        }
    };
    auto compute = [&](int c0, const f32x4_t (&va)[kAhead], const f32x4_t (&vb0)[kAhead],
                       const f32x4_t (&vb1)[kAhead]) {
#pragma unroll
        for (int u = 0; u < kAhead; ++u) {
            if (c0 + u * NW < chunks) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    // D[i][j] += sum_k A[i][k] B[j][k]: the MFMA's first operand gives D's rows
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(va[u][s], vb0[u][s], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(va[u][s], vb1[u][s], acc1, 0, 0, 0);
                }
            }
        }
    };
    // two register sets alternate: the next batch's loads are in flight while the current batch is multiplied
    f32x4_t a0[kAhead], p0[kAhead], q0[kAhead], a1[kAhead], p1[kAhead], q1[kAhead];
    load(wave, a0, p0, q0);
    for (int c = wave; c < chunks; c += 2 * kStep) {
        load(c + kStep, a1, p1, q1);
        compute(c, a0, p0, q0);
        if (c + kStep >= chunks) {
            break;
        }
        load(c + 2 * kStep, a0, p0, q0);
        compute(c + kStep, a1, p1, q1);
    }

    // lane holds D[4 * (lane / 16) + e][lane % 16] (+ 16 columns for acc1), e = 0..3. Element t of the tile is then
    // D[4 * (l / 16) + e][16 * h + l % 16] with l = t % 64, e = (t / 64) % 4, h = t / 256.
    part[wave][0][lane] = acc0;
    part[wave][1][lane] = acc1;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int t = threadIdx.x + i * NW * 64;
        const int l = t & 63, e = (t >> 6) & 3, h = t >> 8;  // source lane, element, column half
        float v = part[0][h][l][e];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            v += part[w][h][l][e];
        }
        const int64_t m = m0 + 4 * (l >> 4) + e, n = n0 + 16 * h + (l & 15);
        if (m < op.M && n < op.N) {
            if constexpr (FORM == EPI_FORM_GENERIC) {
                epi_apply(ep, ob, m, n, v);
            } else {
                epi_elem_pre<ACT, FORM>(ep, ob, m, n, v, pre[i]);
            }
        }
    }
}

// Any call: the whole GemmOperands and EpiParams as arguments.
template <int NW, int ACT, int FORM>
__global__ __launch_bounds__(NW * 64) void gemm_f32_kslice_kernel(GemmOperands op, EpiParams ep, int tilesN)
{
    kslice_body<NW, ACT, FORM>(op, ep, tilesN);
}

// A single-batch call in the f32 form: the fields it uses (120 bytes instead of 380). A smaller argument block
// shortens every launch of this latency-bound kernel.
struct KsArgs {
    const void *a, *b, *bias, *src;
    void *y;
    int64_t M, N, K, lda, ldb;
    int64_t bias_sm, bias_sn, src_sm, y_sm;
    float alpha, gamma, act_alpha;
    int bin, tilesN;
};

template <int NW, int ACT>
__global__ __launch_bounds__(NW * 64) void gemm_f32_kslice_compact_kernel(KsArgs r)
{
    GemmOperands op{};
    op.a = r.a;
    op.b = r.b;
    op.M = r.M;
    op.N = r.N;
    op.K = r.K;
    op.lda = r.lda;
    op.ldb = r.ldb;
    // the epilogue helpers read an EpiParams: the fields the f32 form uses, the rest zero
    EpiParams ep{};
    ep.alpha = r.alpha;
    ep.gamma = r.gamma;
    ep.act_alpha = r.act_alpha;
    ep.act = ACT;
    ep.bin = r.bin;
    ep.c_dt = ep.bias_dt = ep.src_dt = ep.y_dt = KUDNN_DT_F32;
    ep.bias = r.bias;
    ep.src = r.src;
    ep.y = r.y;
    ep.bias_sm = r.bias_sm;
    ep.bias_sn = r.bias_sn;
    ep.src_sm = r.src_sm;
    ep.src_sn = 1;
    ep.y_sm = r.y_sm;
    ep.y_sn = 1;
    ep.bdim[0] = ep.bdim[1] = ep.bdim[2] = 1;
    kslice_body<NW, ACT, EPI_FORM_F32>(op, ep, r.tilesN);
}

}  // namespace

bool kudnn_kslice_eligible(const GemmOperands &op)
{
    return op.K > 0 && op.K % kChunk == 0 && op.lda % 4 == 0 && op.ldb % 4 == 0 &&
           reinterpret_cast<uintptr_t>(op.a) % 16 == 0 && reinterpret_cast<uintptr_t>(op.b) % 16 == 0;
}

int kudnn_launch_gemm_f32_kslice(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream)
{
    if (!kudnn_kslice_eligible(op) || op.M <= 0 || op.N <= 0 || batches < 1 || batches > 65535) {
        return -1;
    }
    const int64_t tilesM = (op.M + kTM - 1) / kTM, tilesN = (op.N + kTN - 1) / kTN;
    if (tilesM * tilesN > 0x7fffffff) {
        return -1;
    }
    const dim3 grid(static_cast<unsigned>(tilesM * tilesN), static_cast<unsigned>(batches));
    constexpr int NW = 4;
    const bool f32Form = epi_form(ep, false) == EPI_FORM_F32;
    if (f32Form && batches == 1 && (ep.bin == KUDNN_BINARY_NONE || ep.src_sn == 1) && ep.y_sn == 1) {
        decltype(&gemm_f32_kslice_compact_kernel<NW, 0>) ck = nullptr;
        switch (ep.act) {
            case KUDNN_ACT_UNIMPLEMENTED: ck = gemm_f32_kslice_compact_kernel<NW, KUDNN_ACT_UNIMPLEMENTED>; break;
            case KUDNN_ACT_RELU: ck = gemm_f32_kslice_compact_kernel<NW, KUDNN_ACT_RELU>; break;
            case KUDNN_ACT_SWISH: ck = gemm_f32_kslice_compact_kernel<NW, KUDNN_ACT_SWISH>; break;
            case KUDNN_ACT_GELU_TANH: ck = gemm_f32_kslice_compact_kernel<NW, KUDNN_ACT_GELU_TANH>; break;
            case KUDNN_ACT_GELU_ERF: ck = gemm_f32_kslice_compact_kernel<NW, KUDNN_ACT_GELU_ERF>; break;
            default: break;
        }
        if (ck != nullptr) {
            const KsArgs r{op.a,   op.b,       ep.bias,    ep.src,    ep.y,    op.M,     op.N,     op.K,
                           op.lda, op.ldb,     ep.bias_sm, ep.bias_sn, ep.src_sm, ep.y_sm, ep.alpha, ep.gamma,
                           ep.act_alpha, ep.bin, static_cast<int>(tilesN)};
            hipLaunchKernelGGL(ck, grid, dim3(NW * 64), 0, stream, r);
            return hipGetLastError() == hipSuccess ? 0 : -1;
        }
    }
    decltype(&gemm_f32_kslice_kernel<NW, 0, EPI_FORM_GENERIC>) kernel = gemm_f32_kslice_kernel<NW, 0, EPI_FORM_GENERIC>;
    if (f32Form) {
        switch (ep.act) {
            case KUDNN_ACT_UNIMPLEMENTED:
                kernel = gemm_f32_kslice_kernel<NW, KUDNN_ACT_UNIMPLEMENTED, EPI_FORM_F32>;
                break;
            case KUDNN_ACT_RELU: kernel = gemm_f32_kslice_kernel<NW, KUDNN_ACT_RELU, EPI_FORM_F32>; break;
            case KUDNN_ACT_SWISH: kernel = gemm_f32_kslice_kernel<NW, KUDNN_ACT_SWISH, EPI_FORM_F32>; break;
            case KUDNN_ACT_GELU_TANH: kernel = gemm_f32_kslice_kernel<NW, KUDNN_ACT_GELU_TANH, EPI_FORM_F32>; break;
            case KUDNN_ACT_GELU_ERF: kernel = gemm_f32_kslice_kernel<NW, KUDNN_ACT_GELU_ERF, EPI_FORM_F32>; break;
            default: break;
        }
    }
    hipLaunchKernelGGL(kernel, grid, dim3(NW * 64), 0, stream, op, ep, static_cast<int>(tilesN));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
