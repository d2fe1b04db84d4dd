// Skinny-M (M <= 16) bf16 / f16 Linear for decode-shaped calls: Y = epilogue(X[M][K] x W[N][K]^T). Every kernel here is
// templated on the operand type CT (KUDNN_DT_BF16 or KUDNN_DT_F16): the MFMA (v_mfma_f32_16x16x32_bf16 / _f16) or the
// conversion of the VALU dot product changes, nothing else.
//
// The reference reaches cblas_sgemv for m == 1 (src/dnn/src/kudnn_gemm.cpp:164-173) and cblas_sbgemm /
// cblas_bgemm otherwise (:208-241). On MI355X this shape is bound by streaming W from HBM once, so the kernels are
// organised around the weight stream, not around compute:
//  - 1 <= M <= 5, gemv_multi_(compact_)kernel: one wave per weight row, 1 KB of the row per load instruction, X's M
//    rows staged once per 4- or 8-row workgroup in LDS, M accumulators per lane fed by v_dot2_f32_bf16, reduced across
//    the wave;
//  - M = 1 with an operand of 2^31 bytes or more, gemv_bf16_(compact_)kernel: the same row stream with 64-bit
//    addressing, X loaded by every wave;
//  - 6 <= M <= 16, skinny_rows_(compact_)kernel: 16 weight rows per workgroup, K split over its waves in blocks of
//    256; whole-row loads go through a per-wave LDS tile into the operand layout of v_mfma_f32_16x16x32_bf16, X (rows
//    m < M, cache-resident) is the second operand (in the 2-wave form also loaded by whole rows through a second
//    tile), and the waves' partial 16 x 16 tiles are summed through LDS;
//  - operands of 2^31 bytes or more, skinny_bf16_kernel: loads straight into the MFMA operand layout (16 rows x 64
//    bytes per instruction) with 64-bit addressing, UNR k-steps in flight.
// Wave 0 (lane m of each wave for the GEMV kernels) runs the fused epilogue.
#include <algorithm>
#include <cstdlib>
#include <utility>

#include "device_common.h"
#include "kernels.h"

using namespace kudnn_dev;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16x16 MFMA step of the skinny kernels on 16-byte operand fragments of type CT.
template <int CT>
__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t acc)
{
    if constexpr (CT == KUDNN_DT_F16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), acc, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
    }
}

template <int CT, int KW, int UNR, bool KTAIL>
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
            acc = mfma16<CT>(wv[u], xv[u], acc);
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

// M = 1 with an operand of 2^31 bytes or more (the staged GEMV further below takes the others): one wave per weight row,
// 64-bit addresses. Lane l reads 16-byte chunks l, l + 64, ... of the row, so every load instruction of a wave reads
// 1 KB of one row contiguously. (The MFMA operand layout of the kernel above reads 16 rows x 64 bytes per
// instruction; at M = 1, where the multiply is negligible, the memory system serves that pattern at about 4.9 TB/s
// against 6.4 TB/s for whole rows, measured on MI355X with the weight streamed from HBM.) K is walked in blocks of
// 4096 (512 chunks, 8 per lane): X's chunks of the block are loaded first, then the row's, all in flight together;
// products are summed in f32 with FMA per lane, then across the wave. Lane 0 runs the epilogue, whose operands are
// loaded during the row. The activation and the epilogue's tensor types are template arguments (as in the MFMA
// kernels) so the kernel's tail is short; batch indices are only decomposed when there is more than one batch.
constexpr int kGemvCh = 8;  // chunks per lane per K block

template <int CT, bool FULL>
__device__ __forceinline__ float gemv_block(const uint16_t *X, const uint16_t *W, int c0, int chunks, int lane)
{
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const v4 zero = {0u, 0u, 0u, 0u};
    v4 xv[kGemvCh], wv[kGemvCh];
#pragma unroll
    for (int c = 0; c < kGemvCh; ++c) {
        const int ch = c0 + c * 64 + lane;
        xv[c] = (FULL || ch < chunks) ? *reinterpret_cast<const v4 *>(X + static_cast<int64_t>(ch) * 8) : zero;
    }
#pragma unroll
    for (int c = 0; c < kGemvCh; ++c) {
        const int ch = c0 + c * 64 + lane;
        wv[c] = (FULL || ch < chunks) ? __builtin_nontemporal_load(reinterpret_cast<const v4 *>(W + static_cast<int64_t>(ch) * 8))
                                      : zero;
    }
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < kGemvCh; ++c) {
        const uint32_t w[4] = {wv[c][0], wv[c][1], wv[c][2], wv[c][3]};
        const uint32_t x[4] = {xv[c][0], xv[c][1], xv[c][2], xv[c][3]};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (CT == KUDNN_DT_F16) {
                sum = fmaf(f16_to_f32(static_cast<uint16_t>(w[j])), f16_to_f32(static_cast<uint16_t>(x[j])), sum);
                sum = fmaf(f16_to_f32(static_cast<uint16_t>(w[j] >> 16)), f16_to_f32(static_cast<uint16_t>(x[j] >> 16)), sum);
            } else {
                sum = fmaf(u2f(w[j] << 16), u2f(x[j] << 16), sum);
                sum = fmaf(u2f(w[j] & 0xffff0000u), u2f(x[j] & 0xffff0000u), sum);
            }
        }
    }
    return sum;
}

template <int CT, int ACT, int FORM>
__global__ __launch_bounds__(256) void gemv_bf16_kernel(GemmOperands op, EpiParams ep)
{
    const int lane = threadIdx.x & 63;
    const int n = static_cast<int>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (n >= op.N) {
        return;  // no barrier or LDS below: a wave past the last row just ends
    }
    int64_t aoff = 0, boff = 0;
    EpiBatch ob{0, 0, 0, 0};
    if (gridDim.y > 1) {
        const int64_t batch = blockIdx.y;
        const int64_t i2 = batch % ep.bdim[2];
        const int64_t i1 = (batch / ep.bdim[2]) % ep.bdim[1];
        const int64_t i0 = batch / (ep.bdim[2] * ep.bdim[1]);
        aoff = i0 * op.a_bs[0] + i1 * op.a_bs[1] + i2 * op.a_bs[2];
        boff = i0 * op.b_bs[0] + i1 * op.b_bs[1] + i2 * op.b_bs[2];
        ob = epi_batch_offsets(ep, batch);
    }
    const uint16_t *X = static_cast<const uint16_t *>(op.a) + aoff;
    const uint16_t *W = static_cast<const uint16_t *>(op.b) + boff + static_cast<int64_t>(n) * op.ldb;
    // rows are 16-byte aligned with a zero-padded or exact multiple-of-8 length (the planner packs otherwise), so whole
    // 16-byte chunks up to ceil(K / 8) are in bounds; the launcher guarantees ceil(K / 8) < 2^31
    const int chunks = static_cast<int>((op.K + 7) / 8);
    const EpiPre1 pre = epi_prefetch1<FORM>(ep, ob, 0, n);
    float sum = 0.0f;
    int c0 = 0;
    for (; c0 + kGemvCh * 64 <= chunks; c0 += kGemvCh * 64) {
        sum += gemv_block<CT, true>(X, W, c0, chunks, lane);
    }
    if (c0 < chunks) {
        sum += gemv_block<CT, false>(X, W, c0, chunks, lane);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        sum += __shfl_xor(sum, o);
    }
    if (lane == 0) {
        if constexpr (FORM == EPI_FORM_GENERIC) {
            epi_apply_pre(ep, ob, 0, n, sum, pre);
        } else {
            epi_elem_pre<ACT, FORM>(ep, ob, 0, n, sum, pre);
        }
    }
}

// The single-batch, fixed-form launch takes only what it reads (about 100 bytes instead of the 380 of GemmOperands +
// EpiParams): the kernel-argument block is copied and read on every launch, which costs about 0.25 us per launch at
// the larger size, measured on MI355X, against a decode step of 7-19 us.
struct GemvArgs {
    const uint16_t *x;
    const uint16_t *w;
    const void *bias;
    const void *src;
    void *y;
    int64_t ldb;
    int64_t bias_sn, src_sn, y_sn;
    int n, chunks;
    float alpha, gamma, act_alpha;
    int bin;
};

template <int CT, int ACT, int FORM>
__global__ __launch_bounds__(256) void gemv_bf16_compact_kernel(GemvArgs a)
{
    const int lane = threadIdx.x & 63;
    const int n = static_cast<int>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (n >= a.n) {
        return;
    }
    // the epilogue helpers read an EpiParams: the fields a fixed-form M = 1 epilogue uses, the rest zero
    EpiParams ep{};
    ep.alpha = a.alpha;
    ep.gamma = a.gamma;
    ep.act_alpha = a.act_alpha;
    ep.bin = a.bin;
    ep.bias = a.bias;
    ep.src = a.src;
    ep.y = a.y;
    ep.bias_sn = a.bias_sn;
    ep.src_sn = a.src_sn;
    ep.y_sn = a.y_sn;
    const EpiBatch ob{0, 0, 0, 0};
    const EpiPre1 pre = epi_prefetch1<FORM>(ep, ob, 0, n);
    const uint16_t *W = a.w + static_cast<int64_t>(n) * a.ldb;
    float sum = 0.0f;
    int c0 = 0;
    for (; c0 + kGemvCh * 64 <= a.chunks; c0 += kGemvCh * 64) {
        sum += gemv_block<CT, true>(a.x, W, c0, a.chunks, lane);
    }
    if (c0 < a.chunks) {
        sum += gemv_block<CT, false>(a.x, W, c0, a.chunks, lane);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        sum += __shfl_xor(sum, o);
    }
    if (lane == 0) {
        epi_elem_pre<ACT, FORM>(ep, ob, 0, n, sum, pre);
    }
}

// 32-bit row and chunk indices
bool gemv_eligible(const GemmOperands &op)
{
    return op.M == 1 && op.N < (int64_t(1) << 31) / 4 && (op.K + 7) / 8 < (int64_t(1) << 31);
}

template <int CT>
int launch_gemv(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream)
{
    decltype(&gemv_bf16_kernel<CT, 0, EPI_FORM_GENERIC>) kernel = nullptr;
    const int form = epi_form(ep, false);
    auto pick = [&](auto formc) {
        constexpr int F = decltype(formc)::value;
        switch (ep.act) {
            case KUDNN_ACT_UNIMPLEMENTED: kernel = gemv_bf16_kernel<CT, KUDNN_ACT_UNIMPLEMENTED, F>; break;
            case KUDNN_ACT_RELU: kernel = gemv_bf16_kernel<CT, KUDNN_ACT_RELU, F>; break;
            case KUDNN_ACT_SWISH: kernel = gemv_bf16_kernel<CT, KUDNN_ACT_SWISH, F>; break;
            case KUDNN_ACT_GELU_TANH: kernel = gemv_bf16_kernel<CT, KUDNN_ACT_GELU_TANH, F>; break;
            case KUDNN_ACT_GELU_ERF: kernel = gemv_bf16_kernel<CT, KUDNN_ACT_GELU_ERF, F>; break;
            default: break;
        }
    };
    dim3 grid(static_cast<unsigned>((op.N + 3) / 4), static_cast<unsigned>(batches));
    constexpr int kForm16 = CT == KUDNN_DT_F16 ? EPI_FORM_F16 : EPI_FORM_BF16;  // the 16-bit form of this operand type
    if (batches == 1 && (form == kForm16 || form == EPI_FORM_F32)) {
        decltype(&gemv_bf16_compact_kernel<CT, 0, EPI_FORM_BF16>) ck = nullptr;
        auto pickc = [&](auto formc) {
            constexpr int F = decltype(formc)::value;
            switch (ep.act) {
                case KUDNN_ACT_UNIMPLEMENTED: ck = gemv_bf16_compact_kernel<CT, KUDNN_ACT_UNIMPLEMENTED, F>; break;
                case KUDNN_ACT_RELU: ck = gemv_bf16_compact_kernel<CT, KUDNN_ACT_RELU, F>; break;
                case KUDNN_ACT_SWISH: ck = gemv_bf16_compact_kernel<CT, KUDNN_ACT_SWISH, F>; break;
                case KUDNN_ACT_GELU_TANH: ck = gemv_bf16_compact_kernel<CT, KUDNN_ACT_GELU_TANH, F>; break;
                case KUDNN_ACT_GELU_ERF: ck = gemv_bf16_compact_kernel<CT, KUDNN_ACT_GELU_ERF, F>; break;
                default: break;
            }
        };
        if (form == kForm16) {
            pickc(std::integral_constant<int, kForm16>{});
        } else {
            pickc(std::integral_constant<int, EPI_FORM_F32>{});
        }
        if (ck != nullptr) {
            GemvArgs a{};
            a.x = static_cast<const uint16_t *>(op.a);
            a.w = static_cast<const uint16_t *>(op.b);
            a.bias = ep.bias;
            a.src = ep.src;
            a.y = ep.y;
            a.ldb = op.ldb;
            a.bias_sn = ep.bias_sn;
            a.src_sn = ep.src_sn;
            a.y_sn = ep.y_sn;
            a.n = static_cast<int>(op.N);
            a.chunks = static_cast<int>((op.K + 7) / 8);
            a.alpha = ep.alpha;
            a.gamma = ep.gamma;
            a.act_alpha = ep.act_alpha;
            a.bin = ep.bin;
            hipLaunchKernelGGL(ck, grid, dim3(256), 0, stream, a);
            return hipGetLastError() == hipSuccess ? 0 : -1;
        }
    }
    if (form == kForm16) {
        pick(std::integral_constant<int, kForm16>{});
    } else if (form == EPI_FORM_F32) {
        pick(std::integral_constant<int, EPI_FORM_F32>{});
    }
    if (kernel == nullptr) {
        // the other activation kinds, and the other tensor types, read everything at run time
        kernel = gemv_bf16_kernel<CT, 0, EPI_FORM_GENERIC>;
    }
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, op, ep);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Bytes a kernel reads from an operand of `rows` rows of `chunks` 16-byte chunks at a pitch of `ld` 16-bit elements:
// through the last row's last chunk. A row count of one has a pitch of 0 in the descriptors (and a strided descriptor
// may repeat a row with pitch 0), so the count times the pitch is not the extent.
__host__ __device__ inline int64_t operand_extent(int64_t rows, int64_t ld, int64_t chunks)
{
    return (rows - 1) * ld * 2 + chunks * 16;
}

// 2 <= M <= 16: 16 weight rows per workgroup, KW waves splitting K into blocks of 256 (block b goes to wave b % KW).
// A wave loads a block of all 16 rows two rows per instruction (lanes 0-31 one row, 32-63 the next: 512 contiguous
// bytes per row, whole cache lines; the MFMA operand layout would read 16 rows x 64 bytes per instruction, which the
// memory system streams at about 4.9 TB/s against 6.4 TB/s for whole rows, measured at M = 1), writes it to a
// per-wave LDS tile (16 rows x 32 chunks of 16 bytes, row pitch 33 chunks: the row-wise writes and the reads of 16 rows
// at one chunk both touch every bank once, and every access is a per-lane base plus an immediate offset), and reads
// it back in the operand layout of v_mfma_f32_16x16x32_bf16, weight rows first, X (rows m < M, cache-resident) second.
// Loads go through buffer resources and are issued by every lane: a lane with nothing to load (a chunk past K, an X
// row m >= M) gets an offset past the resource's range, which reads zero, so no branch separates the loads of a block.
// The weight loads are non-temporal: measured on MI355X, a plain stream of 8 KB weight rows from HBM reads at 6.2 TB/s
// without the hint and 6.6 TB/s with it (the row kernel's M = 4 and 16 steps at N = 14336 went 5-6 % faster).
// With PIPE, a wave issues the weight loads of its next block before the current block goes through LDS and the MFMAs,
// into a second set of registers (the two sets alternate). The KW partial 16 x 16 tiles are summed through LDS and
// wave 0 runs the epilogue on runs of 4 consecutive columns.
// The body of the row kernel. ACT / FORM: a fixed epilogue form (EPI_FORM_BF16 or EPI_FORM_F32, activation compiled
// in) or EPI_FORM_GENERIC (everything read at run time).
template <int CT, int KW, bool PIPE, int ACT, int FORM>
__device__ __forceinline__ void skinny_rows_body(const GemmOperands &op, const EpiParams &ep)
{
    constexpr int kPitch = 33;  // chunks per LDS row
    // XR: X's rows are loaded like the weight's (two rows of 512 contiguous bytes per instruction) and go through a
    // second LDS tile into the MFMA operand layout, instead of being loaded in that layout (16 rows x 64 bytes per
    // instruction). Measured on MI355X at M = 16, N = 14336: the operand-layout X loads cost 6.4 of the kernel's 27 us
    // (20.6 us with them removed, 26.8 us with all of them reading one cache-resident block: the instructions, not
    // the bytes), since the vector memory path serves 64-byte row pieces at half the rate of whole lines.
    constexpr bool XR = PIPE;
    __shared__ u32x4_t tile[KW][16 * kPitch];
    __shared__ u32x4_t xtile[XR ? KW : 1][XR ? 16 * kPitch : 1];
    __shared__ f32x4_t part[KW][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t M = op.M, N = op.N;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    int64_t aoff = 0, boff = 0;
    const int64_t batch = blockIdx.y;
    if (gridDim.y > 1) {
        const int64_t i2 = batch % ep.bdim[2];
        const int64_t i1 = (batch / ep.bdim[2]) % ep.bdim[1];
        const int64_t i0 = batch / (ep.bdim[2] * ep.bdim[1]);
        aoff = i0 * op.a_bs[0] + i1 * op.a_bs[1] + i2 * op.a_bs[2];
        boff = i0 * op.b_bs[0] + i1 * op.b_bs[1] + i2 * op.b_bs[2];
    }
    const uint16_t *X = static_cast<const uint16_t *>(op.a) + aoff;
    const uint16_t *W = static_cast<const uint16_t *>(op.b) + boff;
    const int r16 = lane & 15;
    const int q = lane >> 4;
    const int half = lane >> 5, c32 = lane & 31;
    // rows are 16-byte aligned with a zero-padded or exact multiple-of-8 length (the planner packs otherwise), so whole
    // chunks up to ceil(K / 8) are in bounds; the launcher guarantees both operands' extents are below 2^31 bytes
    const int chunks = static_cast<int>((op.K + 7) / 8);
    const int blocks = (chunks + 31) / 32;
    constexpr uint32_t kOut = 0xFFFFFFF0u;  // past any range below
    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)W, (short)0, static_cast<int>(operand_extent(N, op.ldb, chunks)), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)X, (short)0, static_cast<int>(operand_extent(M, op.lda, chunks)), 0x00020000);
    const uint32_t rowBytes = static_cast<uint32_t>(op.ldb) * 2u;
    const uint32_t xrow = static_cast<uint32_t>(r16) * static_cast<uint32_t>(op.lda) * 2u;
    // byte offset of this lane's row within instruction i (rows 2i, 2i+1; rows past N load row N-1, never stored)
    uint32_t wrow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t row = n0 + 2 * i + half;
        wrow[i] = static_cast<uint32_t>(row < N ? row : N - 1) * rowBytes;
    }
    u32x4_t *tw = tile[wave];
    u32x4_t *tx = xtile[XR ? wave : 0];
    const uint32_t xpitch = static_cast<uint32_t>(op.lda) * 2u;

    // wave 0 runs the epilogue: its bias and binary operand are loaded right after its first block's loads, so their
    // latency overlaps that block's instead of following the K loop
    const EpiBatch ob = epi_batch_offsets(ep, batch);
    const int64_t nq = n0 + 4 * q;  // lane holds D[n = nq + i][m = r16], i = 0..3, after the K loop
    EpiPre4 pre{make_uint2(0u, 0u), make_uint2(0u, 0u), make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
    const bool epiLane = wave == 0 && r16 < M && nq < N;

    // weight loads of block b (a block past the last one loads nothing: every lane gets the out-of-range offset)
    auto load_w = [&](int b, u32x4_t (&wv)[8]) {
        const int c0 = b * 32;
        const bool win = b < blocks && c0 + c32 < chunks;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            wv[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, win ? wrow[i] + static_cast<uint32_t>(c0 + c32) * 16u : kOut, 0, 2);
        }
    };
    // one block: X's loads of block b, then the weight loads of the wave's next block into wn (so they stay in flight
    // through this block's LDS pass and MFMAs: the waits for wv and xv leave the 8 younger loads outstanding), then wv
    // through the LDS tile into the MFMAs
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    auto block = [&](int b, const u32x4_t (&wv)[8], u32x4_t (&wn)[8]) {
        const int c0 = b * 32;
        u32x4_t xv[8];
        if constexpr (XR) {
            // rows 2i + half of X, chunk c0 + c32 (rows m >= M read zero)
            const bool kin = c0 + c32 < chunks;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int m = 2 * i + half;
                xv[i] = __builtin_amdgcn_raw_buffer_load_b128(
                    xrs, kin && m < M ? static_cast<uint32_t>(m) * xpitch + static_cast<uint32_t>(c0 + c32) * 16u : kOut, 0, 0);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {  // k-step k of the block: chunk c0 + 4k + q
                const int kc = c0 + 4 * k + q;
                const bool in = r16 < M && kc < chunks;
                xv[k] = __builtin_amdgcn_raw_buffer_load_b128(xrs, in ? xrow + static_cast<uint32_t>(kc) * 16u : kOut, 0, 0);
            }
        }
        if constexpr (PIPE) {
            load_w(b + KW, wn);
        }
        // the previous block's tile reads have returned (their MFMAs consumed them); order the rewrite after them
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < 8; ++i) tw[(2 * i + half) * kPitch + c32] = wv[i];
        if constexpr (XR) {
#pragma unroll
            for (int i = 0; i < 8; ++i) tx[(2 * i + half) * kPitch + c32] = xv[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const u32x4_t wf = tw[r16 * kPitch + 4 * k + q];
            if constexpr (XR) {
                acc = mfma16<CT>(wf, tx[r16 * kPitch + 4 * k + q], acc);
            } else {
                acc = mfma16<CT>(wf, xv[k], acc);
            }
        }
    };
    u32x4_t w0[8], w1[8];
    load_w(wave, w0);
    if (epiLane) {
        pre = epi_prefetch4(ep, ob, r16, nq, N);
    }
    if constexpr (PIPE) {
        // two named buffers alternate, so no register copy waits on a load in flight
        for (int b = wave; b < blocks; b += 2 * KW) {
            block(b, w0, w1);
            if (b + KW >= blocks) {
                break;
            }
            block(b + KW, w1, w0);
        }
    } else {
        for (int b = wave; b < blocks; b += KW) {
            if (b != wave) {
                load_w(b, w0);
            }
            block(b, w0, w1);
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
        const f32x4_t p = part[w][lane];
        sum[0] += p[0];
        sum[1] += p[1];
        sum[2] += p[2];
        sum[3] += p[3];
    }
    if (r16 >= M || nq >= N) {
        return;
    }
    const float v[4] = {sum[0], sum[1], sum[2], sum[3]};
    if constexpr (FORM == EPI_FORM_GENERIC) {
        epi_apply4_pre(ep, ob, r16, nq, N, v, pre);
    } else {
        epi_fixed4<ACT, FORM>(ep, ob, r16, nq, N, v, pre);
    }
}

// Any row-kernel call: the whole GemmOperands and EpiParams (380 bytes of arguments), the generic epilogue.
template <int CT, int KW, bool PIPE>
__global__ __launch_bounds__(KW * 64) void skinny_rows_kernel(GemmOperands op, EpiParams ep)
{
    skinny_rows_body<CT, KW, PIPE, 0, EPI_FORM_GENERIC>(op, ep);
}

// A single-batch call in a fixed epilogue form: the fields it uses, 128 bytes, and an epilogue with the activation and
// the tensor types compiled in. Measured on MI355X at K = 4096, this cut 0.7-1.4 us from the steps of the decode
// shapes against the generic kernel (the argument block alone about 1.2 us at N = 4096).
struct RowsArgs {
    const void *a, *b, *bias, *src;
    void *y;
    int64_t M, N, K, lda, ldb;
    int64_t bias_sm, bias_sn, src_sm, y_sm;
    float alpha, gamma, act_alpha;
    int bin, fast4;
};

// The GemmOperands and EpiParams of a compact call: the fields a fixed-form epilogue reads, the rest zero.
template <int ACT, int FORM>
__device__ __forceinline__ void unpack_rows_args(const RowsArgs &r, GemmOperands &op, EpiParams &ep)
{
    op = GemmOperands{};
    op.a = r.a;
    op.b = r.b;
    op.M = r.M;
    op.N = r.N;
    op.K = r.K;
    op.lda = r.lda;
    op.ldb = r.ldb;
    constexpr int DT = FORM == EPI_FORM_BF16 ? KUDNN_DT_BF16 : KUDNN_DT_F32;
    ep = EpiParams{};
    ep.alpha = r.alpha;
    ep.gamma = r.gamma;
    ep.act_alpha = r.act_alpha;
    ep.act = ACT;
    ep.bin = r.bin;
    ep.c_dt = ep.bias_dt = ep.src_dt = ep.y_dt = DT;
    ep.fast4 = r.fast4;
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
}

template <int CT, int KW, bool PIPE, int ACT, int FORM>
__global__ __launch_bounds__(KW * 64) void skinny_rows_compact_kernel(RowsArgs r)
{
    GemmOperands op;
    EpiParams ep;
    unpack_rows_args<ACT, FORM>(r, op, ep);
    skinny_rows_body<CT, KW, PIPE, ACT, FORM>(op, ep);
}

// The compact instance kernelOf(activation, form) for a single-batch call in a fixed epilogue form (bf16 or f32
// tensors) with one of the compiled activations; nullptr otherwise, for the generic kernel.
template <typename KernelOf>
auto pick_compact(const EpiParams &ep, bool single, KernelOf kernelOf)
    -> decltype(kernelOf(std::integral_constant<int, KUDNN_ACT_UNIMPLEMENTED>{}, std::integral_constant<int, EPI_FORM_BF16>{}))
{
    decltype(kernelOf(std::integral_constant<int, KUDNN_ACT_UNIMPLEMENTED>{}, std::integral_constant<int, EPI_FORM_BF16>{})) ck =
        nullptr;
    auto pick = [&](auto formc) {
        switch (ep.act) {
            case KUDNN_ACT_UNIMPLEMENTED: ck = kernelOf(std::integral_constant<int, KUDNN_ACT_UNIMPLEMENTED>{}, formc); break;
            case KUDNN_ACT_RELU: ck = kernelOf(std::integral_constant<int, KUDNN_ACT_RELU>{}, formc); break;
            case KUDNN_ACT_SWISH: ck = kernelOf(std::integral_constant<int, KUDNN_ACT_SWISH>{}, formc); break;
            case KUDNN_ACT_GELU_TANH: ck = kernelOf(std::integral_constant<int, KUDNN_ACT_GELU_TANH>{}, formc); break;
            case KUDNN_ACT_GELU_ERF: ck = kernelOf(std::integral_constant<int, KUDNN_ACT_GELU_ERF>{}, formc); break;
            default: break;
        }
    };
    const int form = epi_form(ep, false);
    if (single && form == EPI_FORM_BF16) {
        pick(std::integral_constant<int, EPI_FORM_BF16>{});
    } else if (single && form == EPI_FORM_F32) {
        pick(std::integral_constant<int, EPI_FORM_F32>{});
    }
    return ck;
}

// The fields of a compact call.
inline RowsArgs rows_args(const GemmOperands &op, const EpiParams &ep)
{
    return RowsArgs{op.a,    op.b,   ep.bias,    ep.src,     ep.y,      op.M,    op.N,     op.K,
                    op.lda,  op.ldb, ep.bias_sm, ep.bias_sn, ep.src_sm, ep.y_sm, ep.alpha, ep.gamma,
                    ep.act_alpha, ep.bin, ep.fast4};
}

// A call that can take a compact kernel: one batch, contiguous 4-element runs, a binary operand contiguous along n.
inline bool compact_call(const EpiParams &ep, dim3 grid)
{
    return grid.y == 1 && ep.fast4 && (ep.bin == KUDNN_BINARY_NONE || ep.src_sn == 1);
}

// 1 <= M <= 5 (up to 8 forced): one wave per weight row (lane l reads 16-byte chunks l, l + 64, ... of its row, 1 KB of
// the row per load instruction), with M accumulators per lane. The waves of a workgroup stage X's rows into LDS
// together, in blocks of 512 chunks (4096 elements of K, M x 8 KB), so X is read from L2 once per workgroup instead of
// once per weight row; each wave then reads the chunks it needs from LDS (16 contiguous bytes per lane: no bank
// conflicts). Products are summed with v_dot2_f32_bf16 / _f16 (two products and the accumulator per instruction, no
// conversions), then across the wave; lane m runs the epilogue of output (m, n), its operands loaded before the K loop.
// Measured on MI355X (K = 4096, weight streamed from HBM, per step): M = 4, N = 14336 19.9 us against 22.2 us for the
// 16-row MFMA kernel, N = 4096 8.0 against 8.6 us; M = 1, N = 14336 18.4 against 18.9 us for the GEMV that loads X
// in every wave. From M = 6 on the X reads from LDS (M x 8 KB per row) make it slower than the MFMA kernel; two rows per
// wave sharing each X read, and 16 waves per workgroup, were slower at every M.
constexpr int kMgChunks = 512;  // 16-byte chunks of K per staged X block
constexpr int kMgWaves = 8;     // waves (weight rows) per workgroup

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <int CT>
__device__ __forceinline__ float dot_chunk(u32x4_t w, u32x4_t x, float acc)
{
    // elements are copied out before the bit cast (a bit cast of a vector element reads element 0 with this compiler)
    const uint32_t wa[4] = {w[0], w[1], w[2], w[3]};
    const uint32_t xa[4] = {x[0], x[1], x[2], x[3]};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if constexpr (CT == KUDNN_DT_F16) {
            acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, wa[j]), __builtin_bit_cast(f16x2_t, xa[j]), acc, false);
        } else {
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wa[j]), __builtin_bit_cast(bf16x2_t, xa[j]),
                                                  acc, false);
        }
    }
    return acc;
}

// The body: MR = M rows of X; FORM = EPI_FORM_GENERIC reads the epilogue's types and activation at run time and takes
// batches on grid y.
template <int CT, int MR, int WV, int ACT, int FORM>
__device__ __forceinline__ void gemv_multi_body(const GemmOperands &op, const EpiParams &ep)
{
    constexpr int kLanes = WV * 64;
    constexpr int kXPer = MR * kMgChunks / kLanes;  // staged X chunks per lane and block
    static_assert(kXPer * kLanes == MR * kMgChunks, "the staging covers a block exactly");
    __shared__ u32x4_t xs[MR * kMgChunks];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t N = op.N;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * WV + wave;
    int64_t aoff = 0, boff = 0;
    EpiBatch ob{0, 0, 0, 0, 0, 0};
    if (FORM == EPI_FORM_GENERIC && gridDim.y > 1) {
        const int64_t batch = blockIdx.y;
        const int64_t i2 = batch % ep.bdim[2];
        const int64_t i1 = (batch / ep.bdim[2]) % ep.bdim[1];
        const int64_t i0 = batch / (ep.bdim[2] * ep.bdim[1]);
        aoff = i0 * op.a_bs[0] + i1 * op.a_bs[1] + i2 * op.a_bs[2];
        boff = i0 * op.b_bs[0] + i1 * op.b_bs[1] + i2 * op.b_bs[2];
        ob = epi_batch_offsets(ep, batch);
    }
    // rows are 16-byte aligned with a zero-padded or exact multiple-of-8 length (the planner packs otherwise), so whole
    // chunks up to ceil(K / 8) are in bounds; the launcher guarantees both operands' extents are below 2^31 bytes
    const int chunks = static_cast<int>((op.K + 7) / 8);
    constexpr uint32_t kOut = 0xFFFFFFF0u;  // past any range below: reads zero
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(static_cast<const uint16_t *>(op.b) + boff), (short)0,
        static_cast<int>(operand_extent(N, op.ldb, chunks)), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(static_cast<const uint16_t *>(op.a) + aoff), (short)0,
        static_cast<int>(operand_extent(MR, op.lda, chunks)), 0x00020000);
    // a wave past the last row streams row N - 1 (it takes part in the staging and its barriers) and stores nothing
    const uint32_t wrow = static_cast<uint32_t>(n < N ? n : N - 1) * static_cast<uint32_t>(op.ldb) * 2u;
    const uint32_t xpitch = static_cast<uint32_t>(op.lda) * 2u;

    const bool epiLane = lane < MR && n < N;
    EpiPre1 pre{0u, 0u, 0u};
    if (epiLane) {
        pre = epi_prefetch1<FORM>(ep, ob, lane, n);
    }
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;

    for (int c0 = 0; c0 < chunks; c0 += kMgChunks) {
        // X's share of this lane first, then the row's 8 chunks: the wait for X leaves the weight loads in flight
        u32x4_t xv[kXPer];
#pragma unroll
        for (int i = 0; i < kXPer; ++i) {
            const int idx = i * kLanes + tid;
            const int m = idx / kMgChunks, ch = c0 + idx % kMgChunks;
            xv[i] = __builtin_amdgcn_raw_buffer_load_b128(
                xrs, ch < chunks ? static_cast<uint32_t>(m) * xpitch + static_cast<uint32_t>(ch) * 16u : kOut, 0, 0);
        }
        // keeps the X loads ahead of the weight loads: loads complete in order, so an X load the scheduler moved behind
        // them would make the LDS write wait for the whole weight stream (it did at M = 4: 9.1 against 8.0 us per step)
        __builtin_amdgcn_sched_barrier(0);
        u32x4_t wv[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int ch = c0 + c * 64 + lane;
            wv[c] = __builtin_amdgcn_raw_buffer_load_b128(wrs, ch < chunks ? wrow + static_cast<uint32_t>(ch) * 16u : kOut, 0, 2);
        }
        __builtin_amdgcn_sched_barrier(0);  // and all of them issued before the LDS writes wait for X
        if (c0 != 0) {
            __syncthreads();  // every wave has read the previous block
        }
#pragma unroll
        for (int i = 0; i < kXPer; ++i) xs[i * kLanes + tid] = xv[i];
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            // the chunk's MR X reads first, then their products: the compiler otherwise recycles one register set
            // and waits for every read before its products (it did at M = 4)
            u32x4_t xm[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) xm[m] = xs[m * kMgChunks + c * 64 + lane];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[m] = dot_chunk<CT>(wv[c], xm[m], acc[m]);
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc[m] += __shfl_xor(acc[m], o);
    }
    if (!epiLane) {
        return;
    }
    float v = acc[0];
#pragma unroll
    for (int m = 1; m < MR; ++m) v = lane == m ? acc[m] : v;
    if constexpr (FORM == EPI_FORM_GENERIC) {
        epi_apply_pre(ep, ob, lane, n, v, pre);
    } else {
        epi_elem_pre<ACT, FORM>(ep, ob, lane, n, v, pre);
    }
}

// A single-batch bf16 call in a fixed form: the 128-byte RowsArgs and a compiled-in epilogue.
template <int CT, int MR, int WV, int ACT, int FORM>
__global__ __launch_bounds__(WV * 64) void gemv_multi_compact_kernel(RowsArgs r)
{
    GemmOperands op;
    EpiParams ep;
    unpack_rows_args<ACT, FORM>(r, op, ep);
    gemv_multi_body<CT, MR, WV, ACT, FORM>(op, ep);
}

// Any other call: the whole GemmOperands and EpiParams, batches on grid y.
template <int CT, int MR, int WV>
__global__ __launch_bounds__(WV * 64) void gemv_multi_kernel(GemmOperands op, EpiParams ep)
{
    gemv_multi_body<CT, MR, WV, 0, EPI_FORM_GENERIC>(op, ep);
}

template <int CT, int MR, int WV>
void launch_gemv_multi_wv(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream)
{
    const dim3 grid(static_cast<unsigned>((op.N + WV - 1) / WV), static_cast<unsigned>(batches));
    decltype(&gemv_multi_compact_kernel<CT, MR, WV, 0, EPI_FORM_BF16>) ck = nullptr;
    if constexpr (CT == KUDNN_DT_BF16) {
        ck = pick_compact(ep, compact_call(ep, grid), [](auto actc, auto formc) {
            return gemv_multi_compact_kernel<CT, MR, WV, decltype(actc)::value, decltype(formc)::value>;
        });
    }
    if (ck != nullptr) {
        hipLaunchKernelGGL(ck, grid, dim3(WV * 64), 0, stream, rows_args(op, ep));
    } else {
        hipLaunchKernelGGL((gemv_multi_kernel<CT, MR, WV>), grid, dim3(WV * 64), 0, stream, op, ep);
    }
}

// Workgroups of 8 waves, or of 4 for M = 1 and for M = 2 from 10240 rows on. Measured on MI355X at K = 4096 over
// N = 4096 .. 28672: M = 1 with 4 waves 7.2 / 11.7 / 14.8 / 18.4 / 34.7 us at N = 4096 / 8192 / 11008 / 14336 / 28672
// (8 waves 7.2 / 11.8 / 15.4 / 19.2 / 37.4); M = 2 with 8 waves ahead below 10240 rows (7.3 against 7.5 us at 4096),
// with 4 from 11008 on (34.2 against 37.2 us at 28672); M = 4 with 8 waves ahead at every N (19.99 against 21.6 us at
// 14336), as X's share of the workgroup's reads grows with M.
template <int CT, int MR>
void launch_gemv_multi(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream)
{
    if constexpr (MR <= 2) {
        if (MR == 1 || op.N * batches >= 10240) {
            launch_gemv_multi_wv<CT, MR, 4>(op, ep, batches, stream);
            return;
        }
    }
    launch_gemv_multi_wv<CT, MR, kMgWaves>(op, ep, batches, stream);
}

// 2 <= M <= 16, K <= 4096, one batch: the K-split GEMV. The weight is read once, by whole rows, and X stays in
// registers:
//  - A workgroup of 8 waves splits K into 8 slices of at most 16 steps of 32 (512 elements). Wave w keeps the X
//    fragments of its slice (lane: row lane % 16, 8 elements at 32 s + 8 (lane / 16); 64 VGPRs) for every weight row
//    it reduces. It loads them once, one 1 KB row slice per instruction, through its LDS tile.
//  - The workgroups (one per CU) take the rows in rounds of 16 G: in round j workgroup b takes the 16 rows from
//    16 (j G + b), so each round's loads cover one contiguous part of the weight; a last partial round is divided
//    evenly in whole quads. For each of its rows, wave w loads the row's slice (1 KB, one instruction, non-temporal),
//    writes the group's 16 rows into its LDS tile and reads them back in the operand layout of
//    v_mfma_f32_16x16x32_bf16: one MFMA per step sums 32 k of 16 weight rows against 16 rows of X.
//  - Two groups' loads stay in flight: the registers of a group's rows take the loads of the group two ahead as
//    soon as the rows are in the tile.
//  - Each wave keeps its partial 16 x 16 tile of every group in registers; the waves stream without a barrier and
//    sum their tiles once, through LDS, at the end; then all 512 threads run the epilogue on runs of 4 columns, its
//    operands loaded at the start.
// Rows past a slot's count, rows m >= M of X and chunks past K load through an out-of-range buffer offset, which reads
// zero and fetches nothing.
// Measured on MI355X at K = 4096 (bench.py --only decode-sweep): M = 16, N = 14336 21.7 us against 23.8 us for the
// 16-row kernel below (X reloaded per 16 weight rows: as many X bytes as weight bytes); M = 4 loses to the GEMV with
// X staged in LDS. Variants measured and dropped: the weight loaded straight into the operand layout (16 rows x 64
// bytes per instruction, 24.4 us), 16 waves with 8-step slices (23.0 us), fewer rows per workgroup for less X per
// weight byte (each CU's stream is the limit: 192 workgroups 26.2 us). A v_dot2 GEMV does not fit these M: 16 rows
// of products at N = 14336 are about 13 us of VALU issue against a 17.6 us weight stream.
constexpr int kKgWaves = 8;        // waves per workgroup: K slices
constexpr int kKgStepsAll = 128;   // 32-element k-steps of a workgroup at most: K <= 4096, KW waves x KS steps
constexpr int kKgGroups = 8;       // rounds (16-row groups) per workgroup at most

template <int... I, typename F>
__device__ __forceinline__ void sfor_kg_impl(std::integer_sequence<int, I...>, F &&f)
{
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sfor_kg(F &&f)
{
    sfor_kg_impl(std::make_integer_sequence<int, N>{}, f);
}

template <int CT, int KW, int NG, int ACT, int FORM>
__device__ __forceinline__ void kgemv_body(const GemmOperands &op, const EpiParams &ep, int interleave)
{
    // LDS: a tile of 16 rows x kXPitch chunks per wave (133 KB), which stages the wave's X slice, then each group's
    // weight rows, then the waves' partial tiles; and the result tile (NG groups x 16 rows x 16 floats)
    constexpr int KS = kKgStepsAll / KW;        // k-steps per wave at most
    constexpr int kSliceCh = 4 * KS;           // chunks of a row in a wave's slice
    constexpr int RPI = 64 / kSliceCh;         // rows per load instruction (1 KB per instruction)
    constexpr int kXPitch = kSliceCh + 1;      // chunks per tile row: the 16 rows of a fragment read hit distinct banks
    __shared__ u32x4_t wtile[KW * 16 * kXPitch];
    __shared__ float res[NG * 16][16];
    u32x4_t *lds = wtile;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, q = lane >> 4;
    const int M = static_cast<int>(op.M);
    const int chunks = static_cast<int>((op.K + 7) / 8);
    const int steps = (chunks + 3) / 4;
    const int s0 = steps * wave / KW, ns = steps * (wave + 1) / KW - s0;  // ns <= KS (host-checked)
    // Slot g of the workgroup holds rows n0(g) .. n0(g) + cnt(g) - 1 (cnt 0: none), every slot starting on a whole quad
    // (each run of 4 columns keeps the alignment the vector epilogue assumes). Two ways to deal the rows:
    //  - contiguous (interleave 0): workgroup b takes quads Q b / G .. Q (b + 1) / G - 1 (G = gridDim.x), slot g the
    //    16 rows from the range's start + 16 g;
    //  - in rounds (interleave 1): in round j workgroup b takes the 16 rows from 16 (j G + b), so each round's loads
    //    cover one contiguous part of the weight across the GPU; the rows of a last partial round are divided evenly
    //    in whole quads. The host takes it when each workgroup's range would span a multiple of 128 KB: workgroups
    //    walking such ranges in step load a few memory channels at a time (N = 8192, K = 4096: 17.3 us contiguous
    //    against 13.8-14.9 in rounds; N = 14336: 21.7 against 22.2).
    const int64_t G = gridDim.x, b = blockIdx.x;
    const int64_t quads = (op.N + 3) / 4;
    const int64_t rbeg = quads * b / G * 4, rend = min(quads * (b + 1) / G * 4, op.N);
    const int64_t full = op.N / (16 * G);                     // whole rounds
    const int64_t remQuads = (op.N - full * 16 * G + 3) / 4;  // quads of the last partial round (at most 4 G)
    auto slot = [&](int g, int64_t &n0, int64_t &cnt) __attribute__((always_inline)) {
        if (!interleave) {
            n0 = rbeg + 16 * g;
            cnt = max(min(rend - n0, int64_t(16)), int64_t(0));
        } else if (g < full) {
            n0 = 16 * (g * G + b);
            cnt = 16;
        } else if (g == full && remQuads > 0) {
            const int64_t q0 = remQuads * b / G, q1 = remQuads * (b + 1) / G;
            n0 = full * 16 * G + 4 * q0;
            cnt = min(4 * (q1 - q0), op.N - n0);
        } else {
            n0 = 0;
            cnt = 0;
        }
    };
    constexpr uint32_t kOut = 0xFFFFFFF0u;  // past any range below: reads zero
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(op.b), (short)0, static_cast<int>(operand_extent(op.N, op.ldb, chunks)), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(op.a), (short)0, static_cast<int>(operand_extent(op.M, op.lda, chunks)), 0x00020000);
    const uint32_t wpitch = static_cast<uint32_t>(op.ldb) * 2u, xpitch = static_cast<uint32_t>(op.lda) * 2u;

    // the epilogue's runs of 4 columns: run t is row t % M, quad (t / M) % 4 of slot t / (4 M); the first KW x 64 runs
    // (all of them at the decode shapes) load their operands before the loop, right behind the first two groups'
    // weight loads (their addresses take 64-bit divisions, which ahead of the loads delayed the weight stream: M = 16,
    // N = 8192 15.9 against 15.0 us, N = 14336 22.7 against 22.4 us)
    const int runs = 4 * M * NG;
    const EpiBatch ob{0, 0, 0, 0, 0, 0};
    auto run_at = [&](int t, int &m, int64_t &n, int64_t &lim) __attribute__((always_inline)) {
        int64_t n0, cnt;
        slot(t / (4 * M), n0, cnt);
        m = t % M;
        n = n0 + 4 * ((t / M) % 4);
        lim = n0 + cnt;
    };
    EpiPre4 pre{make_uint2(0u, 0u), make_uint2(0u, 0u), make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};

    // the weight loads of slot g: instruction i reads rows RPI i .. RPI i + RPI - 1 of the slot over the slice, one
    // chunk per lane (lane -> row RPI i + lane / kSliceCh, chunk lane % kSliceCh: 1 KB of whole rows per instruction);
    // rows past the slot's count load nothing
    const int lrow = lane / kSliceCh, lch = lane % kSliceCh;
    const int wkc = 4 * s0 + lch;
    const uint32_t wcol = lch < 4 * ns && wkc < chunks ? static_cast<uint32_t>(wkc) * 16u : kOut;
    auto load_w = [&](int g, u32x4_t (&w)[KS]) __attribute__((always_inline)) {
        int64_t n0, cnt;
        slot(g, n0, cnt);
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            const int r = RPI * i + lrow;
            const bool in = r < cnt && wcol != kOut;
            w[i] = __builtin_amdgcn_raw_buffer_load_b128(wrs, in ? static_cast<uint32_t>(n0 + r) * wpitch + wcol : kOut, 0, 2);
        }
    };
    // X fragments of this wave's slice, loaded once: each of the slice's 16 rows by one instruction (the slice's up to 64
    // chunks of the row, one per lane, whole cache lines), through the wave's LDS area into the operand layout (lane:
    // row lane % 16, chunk 4 s + lane / 16). Loading the fragments directly reads 16 rows x 64 bytes per instruction,
    // which the memory path serves at half the rate of whole lines.
    u32x4_t xf[KS], w0[KS], w1[KS];
    {
        u32x4_t xrow[KS];
#pragma unroll
        for (int i = 0; i < KS; ++i) {
            const int m = RPI * i + lrow;
            xrow[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, wcol != kOut && m < M ? static_cast<uint32_t>(m) * xpitch + wcol : kOut,
                                                           0, 0);
        }
        // the first two groups' weight loads go out behind X's: waiting for X (the older loads) leaves them in flight;
        // the wave's tile takes X first, then (after the fragment reads below) the weight rows
        __builtin_amdgcn_sched_barrier(0);
        load_w(0, w0);
        load_w(1, w1);
        __builtin_amdgcn_sched_barrier(0);
        if (tid < runs) {
            int em;
            int64_t en, elim;
            run_at(tid, em, en, elim);
            if (en < elim) {
                pre = epi_prefetch4(ep, ob, em, en, elim);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        u32x4_t *xs = lds + wave * 16 * kXPitch;
#pragma unroll
        for (int i = 0; i < KS; ++i) xs[(RPI * i + lrow) * kXPitch + lch] = xrow[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int s = 0; s < KS; ++s) xf[s] = xs[r16 * kXPitch + 4 * s + q];
        // the first group's weight rows overwrite the tile after these reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // one group: its rows (in flight since two groups earlier) through the wave's LDS tile into the operand layout
    // (lane: row lane % 16, chunk 4 s + lane / 16); as soon as the rows are in the tile their registers take the loads
    // of the group two ahead, so two groups' loads stay in flight through this group's fragment reads and MFMAs. Each
    // wave keeps its partial tile of every group in registers: the waves stream independently, with no barrier until
    // the end.
    f32x4_t acc[NG];
    auto group = [&](int g, f32x4_t &a, u32x4_t (&wc)[KS]) __attribute__((always_inline)) {
        a = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        u32x4_t *wt = wtile + wave * 16 * kXPitch;
#pragma unroll
        for (int i = 0; i < KS; ++i) wt[(RPI * i + lrow) * kXPitch + lch] = wc[i];
        // the loads are issued before any fragment read or MFMA of this group (the scheduler otherwise sank them below
        // the MFMAs and reused their registers, which made each group wait for the one before)
        __builtin_amdgcn_sched_barrier(0);
        if (g + 2 < NG) {
            load_w(g + 2, wc);
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        u32x4_t wf[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) wf[s] = wt[r16 * kXPitch + 4 * s + q];
#pragma unroll
        for (int s = 0; s < KS; ++s) a = mfma16<CT>(wf[s], xf[s], a);
        // the next group's tile writes come after these reads (the MFMAs consumed them)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // NG groups, unrolled and unconditional (a slot without rows loads nothing and stores nothing): two named register
    // sets alternate, and with straight-line code the compiler's wait counts stay exact (at a loop head, or after a
    // skipped group, it waited for every load in flight, the next group's included)
    sfor_kg<NG>([&](auto gc) __attribute__((always_inline)) {
        constexpr int g = decltype(gc)::value;
        if constexpr (g % 2 == 0) {
            group(g, acc[g], w0);
        } else {
            group(g, acc[g], w1);
        }
    });
    // the waves' partial tiles, in the tiles' place once every wave is done with its own; then their sum per element
    // (lane l of a partial tile holds D[n = 4 (l / 16) + i][m = l % 16] in component i) into the result tile
    __syncthreads();
    f32x4_t(*part)[KW][64] = reinterpret_cast<f32x4_t(*)[KW][64]>(wtile);
    static_assert(sizeof(wtile) >= sizeof(f32x4_t) * NG * KW * 64, "partial tiles fit the weight tiles");
#pragma unroll
    for (int g = 0; g < NG; ++g) part[g][wave][lane] = acc[g];
    __syncthreads();
    for (int t = tid; t < NG * 256; t += KW * 64) {
        const int g = t >> 8, l = (t >> 2) & 63, i = t & 3;
        float sum = part[g][0][l][i];
#pragma unroll
        for (int w = 1; w < KW; ++w) sum += part[g][w][l][i];
        res[16 * g + 4 * (l >> 4) + i][l & 15] = sum;
    }
    __syncthreads();
    for (int t = tid; t < runs; t += KW * 64) {
        int m;
        int64_t n, lim;
        run_at(t, m, n, lim);
        if (n >= lim) {
            continue;
        }
        const int r = 16 * (t / (4 * M)) + 4 * ((t / M) % 4);  // the run's first row in the result tile
        const float v[4] = {res[r][m], res[r + 1][m], res[r + 2][m], res[r + 3][m]};
        const EpiPre4 p = t == tid ? pre : epi_prefetch4(ep, ob, m, n, lim);
        if constexpr (FORM == EPI_FORM_GENERIC) {
            epi_apply4_pre(ep, ob, m, n, lim, v, p);
        } else {
            epi_fixed4<ACT, FORM>(ep, ob, m, n, lim, v, p);
        }
    }
}

template <int CT, int KW, int NG, int ACT, int FORM>
__global__ __launch_bounds__(KW * 64) void kgemv_compact_kernel(RowsArgs r, int interleave)
{
    GemmOperands op;
    EpiParams ep;
    unpack_rows_args<ACT, FORM>(r, op, ep);
    kgemv_body<CT, KW, NG, ACT, FORM>(op, ep, interleave);
}

template <int CT, int KW, int NG>
__global__ __launch_bounds__(KW * 64) void kgemv_kernel(GemmOperands op, EpiParams ep, int interleave)
{
    kgemv_body<CT, KW, NG, 0, EPI_FORM_GENERIC>(op, ep, interleave);
}

// Whether the K-split GEMV takes the call: one batch, 2 <= M <= 16, at most kKgStepsAll k-steps (K <= 4096),
// operands with 32-bit offsets.
bool kgemv_eligible(const GemmOperands &op, int64_t batches)
{
    const int64_t chunks = (op.K + 7) / 8;
    return batches == 1 && op.M >= 2 && op.M <= 16 && (chunks + 3) / 4 <= kKgStepsAll &&
           operand_extent(op.N, op.ldb, chunks) < (int64_t(1) << 31) && operand_extent(op.M, op.lda, chunks) < (int64_t(1) << 31);
}

template <int CT, int KW, int NG>
void launch_kgemv_ng(const GemmOperands &op, const EpiParams &ep, dim3 grid, int interleave, hipStream_t stream)
{
    decltype(&kgemv_compact_kernel<CT, KW, NG, 0, EPI_FORM_BF16>) ck = nullptr;
    if constexpr (CT == KUDNN_DT_BF16) {
        ck = pick_compact(ep, compact_call(ep, grid), [](auto actc, auto formc) {
            return kgemv_compact_kernel<CT, KW, NG, decltype(actc)::value, decltype(formc)::value>;
        });
    }
    if (ck != nullptr) {
        hipLaunchKernelGGL(ck, grid, dim3(KW * 64), 0, stream, rows_args(op, ep), interleave);
    } else {
        hipLaunchKernelGGL((kgemv_kernel<CT, KW, NG>), grid, dim3(KW * 64), 0, stream, op, ep, interleave);
    }
}

template <int CT>
int launch_kgemv(const GemmOperands &op, const EpiParams &ep, hipStream_t stream)
{
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
        (void)hipGetLastError();
        cus = 256;
    }
    // one workgroup per CU (8 waves of about 210 VGPRs and 133 KB of LDS fill a CU), more when N needs more than
    // kKgGroups rounds of 16 rows each; never more workgroups than quads of rows
    const int64_t quads = (op.N + 3) / 4;
    const int64_t G = std::min<int64_t>(quads, std::max<int64_t>(cus, (op.N + 16 * kKgGroups - 1) / (16 * kKgGroups)));
    const dim3 grid(static_cast<unsigned>(G));
    // rows dealt in rounds when each workgroup's contiguous range would span a multiple of 128 KB (the kernel's slot
    // rule); slots: the whole rounds plus one for a partial round, or the range's 16-row groups; instances for 1-4, 8
    const int64_t rows = (quads + G - 1) / G * 4;
    const int interleave = (rows * op.ldb * 2) % (int64_t(128) << 10) == 0 ? 1 : 0;
    const int64_t full = op.N / (16 * G);
    const int64_t ng = interleave ? full + (op.N > full * 16 * G ? 1 : 0) : (rows + 15) / 16;
    switch (ng) {
        case 1: launch_kgemv_ng<CT, kKgWaves, 1>(op, ep, grid, interleave, stream); break;
        case 2: launch_kgemv_ng<CT, kKgWaves, 2>(op, ep, grid, interleave, stream); break;
        case 3: launch_kgemv_ng<CT, kKgWaves, 3>(op, ep, grid, interleave, stream); break;
        case 4: launch_kgemv_ng<CT, kKgWaves, 4>(op, ep, grid, interleave, stream); break;
        default: launch_kgemv_ng<CT, kKgWaves, kKgGroups>(op, ep, grid, interleave, stream); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Launches the row kernel of form (KW, PIPE): the compact kernel when the call is single-batch in a fixed form with one
// of the compiled activations, the generic kernel otherwise.
template <int CT, int KW, bool PIPE>
void launch_rows(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream)
{
    const dim3 grid(static_cast<unsigned>((op.N + 15) / 16), static_cast<unsigned>(batches));
    decltype(&skinny_rows_compact_kernel<CT, KW, PIPE, 0, EPI_FORM_BF16>) ck = nullptr;
    if constexpr (CT == KUDNN_DT_BF16) {
        ck = pick_compact(ep, compact_call(ep, grid), [](auto actc, auto formc) {
            return skinny_rows_compact_kernel<CT, KW, PIPE, decltype(actc)::value, decltype(formc)::value>;
        });
    }
    if (ck != nullptr) {
        hipLaunchKernelGGL(ck, grid, dim3(KW * 64), 0, stream, rows_args(op, ep));
    } else {
        hipLaunchKernelGGL((skinny_rows_kernel<CT, KW, PIPE>), grid, dim3(KW * 64), 0, stream, op, ep);
    }
}

template <int CT, int KW, int UNR>
int launch(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream)
{
    dim3 grid(static_cast<unsigned>((op.N + 15) / 16), static_cast<unsigned>(batches));
    dim3 block(KW * 64);
    if (op.K % 32 == 0) {
        hipLaunchKernelGGL((skinny_bf16_kernel<CT, KW, UNR, false>), grid, block, 0, stream, op, ep);
    } else {
        hipLaunchKernelGGL((skinny_bf16_kernel<CT, KW, UNR, true>), grid, block, 0, stream, op, ep);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int CT>
int launch_skinny(const GemmOperands &op, const EpiParams &ep, int64_t batches, int cfg, hipStream_t stream)
{
    if (op.M > 16) {
        return -1;
    }
    const int64_t chunks = (op.K + 7) / 8;
    const bool fits = operand_extent(op.N, op.ldb, chunks) < (int64_t(1) << 31) &&
                      operand_extent(op.M, op.lda, chunks) < (int64_t(1) << 31);
    // M = 1 (any configuration) and the staged configuration up to M = 8: the GEMV with X staged in LDS; an M = 1
    // operand of 2^31 bytes or more takes the GEMV with 64-bit addressing
    if (fits && (op.M == 1 || (cfg == KUDNN_CFG_GEMV_MULTI_BF16 && op.M <= 8)) && op.N <= (int64_t(1) << 31) - kMgWaves) {
        switch (op.M) {
            case 1: launch_gemv_multi<CT, 1>(op, ep, batches, stream); break;
            case 2: launch_gemv_multi<CT, 2>(op, ep, batches, stream); break;
            case 3: launch_gemv_multi<CT, 3>(op, ep, batches, stream); break;
            case 4: launch_gemv_multi<CT, 4>(op, ep, batches, stream); break;
            case 5: launch_gemv_multi<CT, 5>(op, ep, batches, stream); break;
            case 6: launch_gemv_multi<CT, 6>(op, ep, batches, stream); break;
            case 7: launch_gemv_multi<CT, 7>(op, ep, batches, stream); break;
            default: launch_gemv_multi<CT, 8>(op, ep, batches, stream); break;
        }
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if (gemv_eligible(op)) {
        return launch_gemv<CT>(op, ep, batches, stream);
    }
    if (cfg == KUDNN_CFG_GEMV_KSPLIT_BF16 && kgemv_eligible(op, batches)) {
        return launch_kgemv<CT>(op, ep, stream);
    }
    if (fits) {
        // fewer than 2 row groups per CU: split K over 16 waves (one workgroup per CU); otherwise 8 (two per CU)
        const int64_t groups = (op.N + 15) / 16 * batches;
        // measured at K = 4096: with more than 8 rows of X, 2-wave workgroups with the next block's weights in flight
        // and X's rows through an LDS tile (169 VGPRs, 36 KB of LDS: 4 workgroups per CU) beat the 8- and 16-wave
        // forms (M = 16, N = 14336: 23.9 against 27.0 us); at M = 7 and 8 they win from 512 row groups on (M = 8,
        // N = 8192: 13.4 against 15.0 us) and lose at 256 (N = 4096: 9.4 against 9.0 us); at M = 6 they are even
        if ((op.M > 8 && groups >= 256) || (op.M >= 7 && groups >= 512)) {
            launch_rows<CT, 2, true>(op, ep, batches, stream);
        } else if (groups < 512) {
            launch_rows<CT, 16, false>(op, ep, batches, stream);
        } else {
            launch_rows<CT, 8, false>(op, ep, batches, stream);
        }
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    // Few weight row-groups: split K over 8 waves per workgroup to keep more loads in flight.
    const int64_t groups = (op.N + 15) / 16 * batches;
    if (groups < 1024) {
        return launch<CT, 8, 8>(op, ep, batches, stream);
    }
    return launch<CT, 4, 8>(op, ep, batches, stream);
}

}  // namespace

int kudnn_launch_skinny(const GemmOperands &op, const EpiParams &ep, int64_t batches, int ct, int cfg, hipStream_t stream)
{
    switch (ct) {
        case KUDNN_DT_BF16: return launch_skinny<KUDNN_DT_BF16>(op, ep, batches, cfg, stream);
        case KUDNN_DT_F16: return launch_skinny<KUDNN_DT_F16>(op, ep, batches, cfg, stream);
        default: return -1;
    }
}
