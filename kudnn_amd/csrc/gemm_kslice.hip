// f32 GEMM for grids too small to fill the chip with output tiles (the fp32 Linear of the reference's
// LinearActivationTests, 128 x 1024 x 1024, is 32 tiles of 64 x 64): one workgroup per 16 x 32 output tile, its NW
// waves splitting K. Each wave accumulates the whole 16 x 32 tile on v_mfma_f32_16x16x4_f32, the NW partial tiles are
// summed through LDS in wave order, and the epilogue stores the tile. There is no workspace and no hand-off between
// workgroups, so the kernel's latency is one pass of loads and MFMAs plus one LDS reduction. Two forms (kslice_body):
// K = 256 c for c = 1, 2, 3, 4, 6, 8, 12, 16 (C1 included), 8 waves loading whole 128-byte lines through a per-wave
// LDS tile; otherwise 4 waves loading interleaved 16-element chunks (chunk c goes to wave c % NW) straight into the
// operand layout.
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

#include <type_traits>

#include "device_common.h"
#include "kernels.h"
#include "kslice.h"

namespace {

using namespace kudnn_dev;

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTM = 16, kTN = 32;  // output tile
constexpr int kChunk = 16;         // k per chunk (one 16-byte load per lane per operand row group)
constexpr int kAhead = 2;          // chunks per batch of loads (two batches in flight; more in flight measured slower)

// ACT / FORM: a fixed epilogue form (the activation and the tensor types compiled in) or EPI_FORM_GENERIC. The generic
// epilogue is a long chain of run-time branches whose first pass on each CU misses the instruction cache: for a
// kernel this short that is a large part of its time, so the common forms are compiled out.
// CPW > 0 (K = 16 NW CPW, CPW even): K is cut into pairs of chunks (32 k: one 128-byte line of each row) and wave w
// takes pairs w, w + NW, w + 2 NW, ... (at any time the waves read neighbouring lines of each row). A pair is loaded
// as whole lines: instruction i reads 8 of the wave's 48 rows (A's 16, then B's 32), lane -> row lane / 8, 16-byte
// piece lane % 8. A wave's first 8 pairs of loads are issued before its first MFMA, as straight-line code, so the
// compiler's wait before each pair counts only that pair's loads; past 8 pairs (K > 2048), 6 pairs stay in flight:
// pair p + 6 is issued into pair p's registers once pair p is in LDS. Each pair then goes through the wave's own LDS tile (48 rows x
// 8 pieces, piece j of row r in slot j ^ (r % 8): the row-wise writes and the operand-layout reads are both
// conflict-free) into the MFMA operand layout. Measured on C1 (graph-replayed), with the MFMAs removed the operand
// layout's loads (16 rows x 64 bytes per instruction) took 7.35 us and whole lines 4.15 us; the kernel went from 8.0
// to 6.0-6.1 us (4 waves with contiguous K ranges 6.8, a barrier between the waves' pairs of loads 6.4, 16 waves 6.3).
// Past the first pair's arrival the MFMAs bound it: C1 is 4096 cycles of v_mfma_f32_16x16x4_f32 per SIMD.
// CPW = 0: any K, two batches of kAhead interleaved chunks in flight per wave, loaded in the operand layout.
// BKM (whole-line form only): B is stored [K][N] (N contiguous, k-row pitch ldb) and read in place. A pair's B lines
// are then its 32 k-rows x the tile's 32 columns (128 bytes each): instruction i = 2..5 reads k-rows 8 (i - 2) + lane / 8,
// columns 4 (lane % 8) .. + 3 (past N: clamped to the last whole chunk, read but never stored). They go to a second
// region of the LDS tile, 32 k-rows at a pitch of 36 floats, and a lane reads its column's 4 consecutive k as 4 floats:
// the 36-float pitch puts the four k-rows 4 q + s (q = 0..3) of one read in four different 16-bank groups, so each
// ds_read_b32 is conflict-free. The MFMAs get the same k values in the same order as from a packed [N][K] weight.
template <int NW, int CPW, int ACT, int FORM, bool BKM = false>
__device__ __forceinline__ void kslice_body(const GemmOperands &op, const EpiParams &ep, int tilesN)
{
    static_assert(!BKM || CPW > 0, "only the whole-line form reads a [K][N] weight in place");
    constexpr int kElems = kTM * kTN;
    // output elements per thread in the epilogue (with more threads than elements, the first kElems take one each)
    constexpr int kPer = kElems > NW * 64 ? kElems / (NW * 64) : 1;
    static_assert(kPer * NW * 64 == kElems || (kPer == 1 && NW * 64 > kElems), "the tile must divide over the threads");
    __shared__ f32x4_t part[NW][2][64];
    constexpr int kRows = kTM + 2 * 16;  // a wave's rows: A's 16, B's 32
    constexpr int kBkmPitch = 36;        // floats per k-row of a [K][N] weight's region
    constexpr int kTileQuads = BKM ? kTM * 8 + 32 * kBkmPitch / 4 : kRows * 8;
    __shared__ f32x4_t tile[CPW > 0 ? NW : 1][kTileQuads];

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
            const int t = min(static_cast<int>(threadIdx.x) + i * NW * 64, kElems - 1);
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
    if constexpr (CPW > 0) {
        static_assert(CPW % 2 == 0, "whole chunk pairs");
        constexpr int NP = CPW / 2;  // pairs of chunks: 32 k, one 128-byte line of each row
        const int lr = lane >> 3, lp = lane & 7;
        // the rows of load instruction i: A rows 8 i + lr (i < 2), B rows 8 (i - 2) + lr; past M / N: the last row.
        // Pair p of this wave covers k from 32 (wave + NW p): rowp[i] + pstep[i] p is its line's first byte
        const float *rowp[6];
        int64_t pstep[6];
#pragma unroll
        for (int i = 0; i < 6; ++i) {
            if (i < 2) {
                const int64_t m = m0 + 8 * i + lr;
                rowp[i] = static_cast<const float *>(op.a) + aoff + (m < op.M ? m : op.M - 1) * op.lda + 32 * wave + 4 * lp;
                pstep[i] = 32 * NW;
            } else if constexpr (BKM) {
                int64_t n = n0 + 4 * lp;
                n = n + 4 <= op.N ? n : op.N - 4;
                rowp[i] = static_cast<const float *>(op.b) + boff + (32 * wave + 8 * (i - 2) + lr) * op.ldb + n;
                pstep[i] = 32 * NW * op.ldb;
            } else {
                const int64_t n = n0 + 8 * (i - 2) + lr;
                rowp[i] = static_cast<const float *>(op.b) + boff + (n < op.N ? n : op.N - 1) * op.ldb + 32 * wave + 4 * lp;
                pstep[i] = 32 * NW;
            }
        }
        // up to 8 pairs in flight per wave (192 VGPRs): all of them when NP <= 8; otherwise 6, pair p + 6 issued into
        // pair p's registers as soon as pair p is in the LDS tile
        constexpr int WIN = NP <= 8 ? NP : 6;
        f32x4_t ld[WIN][6];
        auto issue = [&](int p, f32x4_t (&dst)[6]) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < 6; ++i) dst[i] = *reinterpret_cast<const f32x4_t *>(rowp[i] + pstep[i] * p);
        };
#pragma unroll
        for (int p = 0; p < WIN; ++p) issue(p, ld[p]);
        __builtin_amdgcn_sched_barrier(0);
        f32x4_t *t = tile[wave];
        const int sw = r & 7;  // the swizzle of operand row r (and of rows 16 + r, 32 + r)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            // row 8 i + lr, piece lp -> slot lp ^ lr (8 i is a multiple of 8); a [K][N] weight's k-row 8 (i - 2) + lr,
            // columns 4 lp .. + 3 -> its region at pitch kBkmPitch
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                if (BKM && i >= 2) {
                    t[kTM * 8 + ((8 * (i - 2) + lr) * kBkmPitch + 4 * lp) / 4] = ld[p % WIN][i];
                } else {
                    t[(8 * i + lr) * 8 + (lp ^ lr)] = ld[p % WIN][i];
                }
            }
            if (p + WIN < NP) {
                __builtin_amdgcn_sched_barrier(0);
                issue(p + WIN, ld[p % WIN]);
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // chunk h of the pair: lane (r, q) takes piece 4 h + q of A row r and of B rows r and 16 + r
            f32x4_t fa[2], fb0[2], fb1[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int slot = (4 * h + q) ^ sw;
                fa[h] = t[r * 8 + slot];
                if constexpr (BKM) {
                    // column r (and 16 + r) at k = 16 h + 4 q + s, s = 0..3
                    const float *kb = reinterpret_cast<const float *>(t + kTM * 8) + (16 * h + 4 * q) * kBkmPitch + r;
                    fb0[h] = f32x4_t{kb[0], kb[kBkmPitch], kb[2 * kBkmPitch], kb[3 * kBkmPitch]};
                    fb1[h] = f32x4_t{kb[16], kb[kBkmPitch + 16], kb[2 * kBkmPitch + 16], kb[3 * kBkmPitch + 16]};
                } else {
                    fb0[h] = t[(16 + r) * 8 + slot];
                    fb1[h] = t[(32 + r) * 8 + slot];
                }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[h][s], fb0[h][s], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[h][s], fb1[h][s], acc1, 0, 0, 0);
                }
            }
            // the next pair's writes come after these reads
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    } else {
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
    }

    // lane holds D[4 * (lane / 16) + e][lane % 16] (+ 16 columns for acc1), e = 0..3. Element t of the tile is then
    // D[4 * (l / 16) + e][16 * h + l % 16] with l = t % 64, e = (t / 64) % 4, h = t / 256.
    part[wave][0][lane] = acc0;
    part[wave][1][lane] = acc1;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int t = threadIdx.x + i * NW * 64;
        if (t >= kElems) {
            break;
        }
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
template <int NW, int CPW, int ACT, int FORM, bool BKM>
__global__ __launch_bounds__(NW * 64) void gemm_f32_kslice_kernel(GemmOperands op, EpiParams ep, int tilesN)
{
    kslice_body<NW, CPW, ACT, FORM, BKM>(op, ep, tilesN);
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

template <int NW, int CPW, int ACT, bool BKM>
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
    kslice_body<NW, CPW, ACT, EPI_FORM_F32, BKM>(op, ep, r.tilesN);
}

}  // namespace

bool kudnn_kslice_eligible(const GemmOperands &op)
{
    return op.K > 0 && op.K % kChunk == 0 && op.lda % 4 == 0 && op.ldb % 4 == 0 &&
           reinterpret_cast<uintptr_t>(op.a) % 16 == 0 && reinterpret_cast<uintptr_t>(op.b) % 16 == 0;
}

namespace {

template <int NW, int CPW, bool BKM>
int launch_kslice(const GemmOperands &op, const EpiParams &ep, int64_t batches, int64_t tilesN, dim3 grid,
                  hipStream_t stream)
{
    const bool f32Form = epi_form(ep, false) == EPI_FORM_F32;
    if (f32Form && batches == 1 && (ep.bin == KUDNN_BINARY_NONE || ep.src_sn == 1) && ep.y_sn == 1) {
        decltype(&gemm_f32_kslice_compact_kernel<NW, CPW, 0, BKM>) ck = nullptr;
        switch (ep.act) {
            case KUDNN_ACT_UNIMPLEMENTED: ck = gemm_f32_kslice_compact_kernel<NW, CPW, KUDNN_ACT_UNIMPLEMENTED, BKM>; break;
            case KUDNN_ACT_RELU: ck = gemm_f32_kslice_compact_kernel<NW, CPW, KUDNN_ACT_RELU, BKM>; break;
            case KUDNN_ACT_SWISH: ck = gemm_f32_kslice_compact_kernel<NW, CPW, KUDNN_ACT_SWISH, BKM>; break;
            case KUDNN_ACT_GELU_TANH: ck = gemm_f32_kslice_compact_kernel<NW, CPW, KUDNN_ACT_GELU_TANH, BKM>; break;
            case KUDNN_ACT_GELU_ERF: ck = gemm_f32_kslice_compact_kernel<NW, CPW, KUDNN_ACT_GELU_ERF, BKM>; break;
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
    decltype(&gemm_f32_kslice_kernel<NW, CPW, 0, EPI_FORM_GENERIC, BKM>) kernel = gemm_f32_kslice_kernel<NW, CPW, 0, EPI_FORM_GENERIC, BKM>;
    if (f32Form) {
        switch (ep.act) {
            case KUDNN_ACT_UNIMPLEMENTED:
                kernel = gemm_f32_kslice_kernel<NW, CPW, KUDNN_ACT_UNIMPLEMENTED, EPI_FORM_F32, BKM>;
                break;
            case KUDNN_ACT_RELU: kernel = gemm_f32_kslice_kernel<NW, CPW, KUDNN_ACT_RELU, EPI_FORM_F32, BKM>; break;
            case KUDNN_ACT_SWISH: kernel = gemm_f32_kslice_kernel<NW, CPW, KUDNN_ACT_SWISH, EPI_FORM_F32, BKM>; break;
            case KUDNN_ACT_GELU_TANH: kernel = gemm_f32_kslice_kernel<NW, CPW, KUDNN_ACT_GELU_TANH, EPI_FORM_F32, BKM>; break;
            case KUDNN_ACT_GELU_ERF: kernel = gemm_f32_kslice_kernel<NW, CPW, KUDNN_ACT_GELU_ERF, EPI_FORM_F32, BKM>; break;
            default: break;
        }
    }
    hipLaunchKernelGGL(kernel, grid, dim3(NW * 64), 0, stream, op, ep, static_cast<int>(tilesN));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

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
    const int64_t chunks = op.K / kChunk;
    // whole-line loads through LDS with 8 waves when K is 256 times 1, 2, 3, 4, 6, 8, 12 or 16 (K <= 4096; past
    // 2048, 6 pairs of loads in flight per wave); otherwise 4 waves and the operand layout. A [K][N] weight (the
    // planner gives one only with such a K) is read in place by the whole-line form.
    auto whole = [&](auto bkm) -> int {
        constexpr bool B = decltype(bkm)::value;
        switch (chunks / 16) {
            case 1: return launch_kslice<8, 2, B>(op, ep, batches, tilesN, grid, stream);
            case 2: return launch_kslice<8, 4, B>(op, ep, batches, tilesN, grid, stream);
            case 3: return launch_kslice<8, 6, B>(op, ep, batches, tilesN, grid, stream);
            case 4: return launch_kslice<8, 8, B>(op, ep, batches, tilesN, grid, stream);
            case 6: return launch_kslice<8, 12, B>(op, ep, batches, tilesN, grid, stream);
            case 8: return launch_kslice<8, 16, B>(op, ep, batches, tilesN, grid, stream);
            case 12: return launch_kslice<8, 24, B>(op, ep, batches, tilesN, grid, stream);
            case 16: return launch_kslice<8, 32, B>(op, ep, batches, tilesN, grid, stream);
            default: return -1;
        }
    };
    if (kudnn_kslice_whole_line(op.K)) {
        return op.b_kmajor ? whole(std::true_type{}) : whole(std::false_type{});
    }
    if (op.b_kmajor) {
        return -1;
    }
    return launch_kslice<4, 0, false>(op, ep, batches, tilesN, grid, stream);
}
