// bf16 / f16 / s8 GEMM on gfx950 MFMA, 8-wave ping-pong schedule, 256 x 256 output tile, k-tile of 128 bytes
// (64 bf16 or f16, 128 s8), fused epilogue.
//
// This is the kernel behind cblas_sbgemm / cblas_bgemm, cblas_hgemm / cblas_shgemm and cblas_gemm_s8s8s32 in the
// reference (src/dnn/src/kudnn_gemm.cpp:182-264) for large M: Y = epilogue(A[M][K] x B[N][K]^T), both operands
// contiguous along K. The three element types share the data path byte for byte: each MFMA
// (v_mfma_f32_32x32x16_bf16 / _f16, v_mfma_i32_32x32x32_i8) takes 16 bytes of a row per lane, lane half h holding
// bytes 16h .. 16h+15 of each 32-byte k step for both operands; s8 accumulates in int32 (the same registers, as bit
// patterns) and ends in the exact integer epilogue.
//
// Why this schedule. On gfx950 a wave that issues a global->LDS copy (buffer_load ... lds) stalls until the
// texture-address unit accepts it, about 22 cycles per 1 KB instruction per CU (measured; the cost is per 128-byte
// cache line, so k-tiles of 64 bf16 = full lines are used). A 256x256x64 tile needs 64 such instructions
// (~1400 cycles) against 2048 cycles of MFMA per SIMD, so the copies must never sit in front of the MFMAs.
// Eight waves run as two groups on the four SIMDs (wave w: group g = w/4, SIMD p = w%4) and alternate phases
// separated by s_barrier, group 1 one phase behind group 0:
//   memory phase M(t): read this wave's A fragments of k-tile t from LDS, issue its share of the next copies
//                      (group 0: A(t+1), group 1: B(t+2)), read the B fragments of the first k16 step;
//   compute phase C(t): 32 v_mfma_f32_32x32x16_bf16, B fragments of step s+1 read while step s issues.
// While one wave of a SIMD is in its memory phase the other issues MFMAs. A wave raises its priority (s_setprio 1) for
// its compute phase, so when both waves of a SIMD have an instruction ready the arbiter issues the MFMA wave's first
// instead of the older wave's (measured on C3, alternating runs on one box: 1203-1209 TFLOP/s without, 1222-1225 with).
//
// LDS (160 KB): A tiles double-buffered, B tiles triple-buffered (5 x 32 KB). A(t) is read in phases 2t, 2t+1 and
// rewritten by A(t+2) from phase 2t+2; B(t) is read in phases 2t .. 2t+2 and rewritten by B(t+3) at phase 2t+3.
// Each buffer is its own __shared__ array and the loop is unrolled by 6 so every access names its buffer at compile
// time; the compiler can then tell that the copies and the fragment reads never alias and does not insert a full
// vmcnt(0) wait in front of every LDS read.
//
// Rows are 128 bytes per k-tile with a XOR swizzle (chunk ^ ((row >> 1) & 7)) so the 16 lanes of a ds_read_b128
// quarter-wave hit 16 distinct 16-byte slots of the 64 LDS banks.
//
// Copies are issued from inline asm, so the compiler inserts no waits for them (its alias analysis cannot tell which
// buffer a copy writes and would otherwise wait for every copy of a memory phase before the next LDS read); the
// kernel's own s_waitcnt vmcnt(N) calls order each buffer's copies before its first read: group 1 waits at the end of
// its memory phase for the previous memory phase's copies, group 0 at the end of its compute phase for its A copies.
// A tile that lies wholly inside the matrix copies through one buffer resource over the whole operand, the lane's row
// and chunk in the vector offset and the 8-row block and k-tile in the scalar offset: three scalar instructions per
// 1 KB copy. (Building a resource per copy, as the edge tiles do, took VALU work and SGPR hazards per copy and made the
// memory phase, 32 copies per group, as long as the compute phase: about 1,080 cycles against 580.) A tile that
// crosses the matrix edge builds a resource per copy that starts at the copied 8-row block, so rows past the end of
// the operand fall outside its range and read as zero.
//
// Epilogue: the accumulators pass through LDS one 32-column strip at a time and are read back row-major, 8
// consecutive columns per lane, so bias / activation / residual run on 8 values and the result is one 16-byte store;
// the bias and binary operand are loaded two strips ahead of their use. The activation is a template
// argument of the kernel and the all-bf16 case has its own code, so the epilogue of a full tile is short straight-line
// code (an epilogue that dispatched every option at run time at each of its 16 call sites made the kernel 2.2 MB and
// spent most of its time in instruction-cache misses). Tiles that cross the matrix edge take a rolled per-element loop.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <utility>

#include "device_common.h"
#include "kernels.h"
#include "kmajor_copy.h"

using namespace kudnn_dev;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBM = 256, kBN = 256, kKC = 8, kRowBytes = 128;  // k-tile: 128 bytes of each row
constexpr int kTile = 256 * kKC;        // uint4 per A or B tile buffer (32 KB)
constexpr int kPitch = 36;              // epilogue staging pitch in floats (32 columns + 4)

template <int... I, typename F>
__device__ __forceinline__ void sfor_impl(std::integer_sequence<int, I...>, F &&f)
{
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sfor(F &&f)
{
    sfor_impl(std::make_integer_sequence<int, N>{}, f);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    // s_waitcnt: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14; expcnt (7) and lgkmcnt (15) left unconstrained
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// The split (SK) instances keep compiler-visible copies: the intrinsic below, whose waits the compiler inserts (a
// vmcnt(0) at the end of each memory phase). Their extra live state leaves no registers for the asm copy path.
// One 1 KB copy global -> LDS of an 8-row block through a raw buffer resource that starts at the block's first byte
// (wave-uniform byte offset `off` from `base`) and covers the bytes of the operand after it.
__device__ __forceinline__ void copy_block(const uint8_t *base, uint32_t totalBytes, uint32_t off, uint32_t voff, uint4 *dst)
{
    const uint32_t remain = __builtin_amdgcn_readfirstlane(off < totalBytes ? totalBytes - off : 0u);
    __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)(base + off), (short)0, (int)remain, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)dst, 16, voff, 0, 0, 0);
}

typedef int i32x4_rs_t __attribute__((ext_vector_type(4)));

// Raw buffer resource words: base address, no stride, `bytes` in range, 32-bit data format.
__device__ __forceinline__ i32x4_rs_t make_rsrc(const uint8_t *base, uint32_t bytes)
{
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    i32x4_rs_t rs;
    rs.x = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(p)));
    rs.y = __builtin_amdgcn_readfirstlane(static_cast<int>((p >> 32) & 0xffffu));
    rs.z = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
    rs.w = 0x00020000;
    return rs;
}

// LDS byte address of a __shared__ buffer.
__device__ __forceinline__ uint32_t lds_addr(const uint4 *p)
{
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void *)p));
}

// One 1 KB copy global -> LDS (64 lanes x 16 bytes written to lds .. lds + 1023): lane bytes at voff + soff of the
// resource. The s_nop before the copy covers the wait states a copy needs after VALU writes of the SGPRs it reads
// (the resource words may come from v_readfirstlane) and after the write of M0, which inline asm hides from the
// compiler's hazard tracking.
__device__ __forceinline__ void copy_lds(i32x4_rs_t rs, uint32_t voff, uint32_t soff, uint32_t lds)
{
    soff = __builtin_amdgcn_readfirstlane(soff);
    lds = __builtin_amdgcn_readfirstlane(lds);
    asm volatile("s_nop 4\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %3 offen lds"
                 ::"v"(voff), "s"(rs), "s"(lds), "s"(soff) : "memory");
}

// The same without the leading wait states, for copies whose SGPR operands were written by scalar instructions.
__device__ __forceinline__ void copy_lds_fast(i32x4_rs_t rs, uint32_t voff, uint32_t soff, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %3 offen lds"
                 ::"v"(voff), "s"(rs), "s"(lds), "s"(soff) : "memory");
}

// A copy of an 8-row block of a tile that may cross the matrix edge: the resource starts at the block's first byte
// (`off` from `base`) and covers the bytes of the operand after it, so the hardware range check on the per-lane
// offset `voff` turns rows past the end of the operand into zeros instead of reads outside the allocation.
__device__ __forceinline__ void copy_block_edge(const uint8_t *base, uint32_t totalBytes, uint32_t off, uint32_t voff,
                                                uint32_t lds)
{
    // the clamped difference is a saturating subtract, which only the vector ALU has; readfirstlane makes it scalar
    const uint32_t remain = __builtin_amdgcn_readfirstlane(off < totalBytes ? totalBytes - off : 0u);
    copy_lds(make_rsrc(base + off, remain), voff, 0u, lds);
}

// Writes strip j of a wave's accumulators (64 rows x 32 columns) to its staging area, row pitch kPitch floats.
__device__ __forceinline__ void stage_strip(const f32x16_t (&accj)[2], float *stage, int lrow, int lh)
{
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            float *dst = stage + (i * 32 + lrow) * kPitch + q4 * 8 + lh * 4;
            *reinterpret_cast<float4 *>(dst) =
                make_float4(accj[i][4 * q4 + 0], accj[i][4 * q4 + 1], accj[i][4 * q4 + 2], accj[i][4 * q4 + 3]);
        }
    }
}

// The staging area is private to the wave: ordering its LDS writes and reads needs a wave barrier only.
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Epilogue of a full tile (all rows and columns in bounds) in a fixed form, with no bias or a bias that is one row
// broadcast over m: lane -> row rl + 16 * pass, columns col8 .. +8 of each strip. The bias and binary operand of
// AHEAD strips are in flight at a time (strip j + AHEAD's loads are issued once strip j is stored), and the first
// AHEAD strips' are issued before the barrier that ends the main loop, so one memory latency is exposed per tile
// instead of one per strip. Two strips ahead for the 16-bit forms; the f32 form's operands are twice the registers,
// so it runs one ahead. The bias is the same for the four rows a lane covers in a strip and is loaded once.
template <int ACT, int FORM>
__device__ __forceinline__ void epilogue_full(const EpiParams &ep, const EpiBatch &ob, const f32x16_t (&acc)[4][2],
                                              float *stage, int lane, int64_t mW, int64_t nW)
{
    constexpr int AHEAD = FORM == EPI_FORM_F32 ? 1 : 2;
    const int lrow = lane & 31, lh = lane >> 5;
    const int col8 = (lane & 3) * 8, rl = lane >> 2;
    Raw8 src[AHEAD][4], bias[AHEAD];
    auto fetch = [&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nW + j * 32 + col8;
        bias[j % AHEAD] = epi_prefetch8_bias<FORM>(ep, ob, mW + rl, n);
        sfor<4>([&](auto pc) __attribute__((always_inline)) {
            constexpr int ps = decltype(pc)::value;
            src[j % AHEAD][ps] = epi_prefetch8_src<FORM>(ep, ob, mW + rl + ps * 16, n);
        });
    };
    sfor<AHEAD>([&](auto jc) __attribute__((always_inline)) { fetch(jc); });
    // the output address of this lane's first group (row mW + rl, column nW + col8); pass ps adds 16 ps rows, strip j
    // 32 j columns
    constexpr int64_t ES = FORM == EPI_FORM_F32 ? 4 : 2;
    char *yLane = static_cast<char *>(ep.y) + (ob.y + (mW + rl) * ep.y_sm + nW + col8) * ES;
    const int64_t yPass = 16 * ep.y_sm * ES;
    __syncthreads();  // every wave is done with the tile buffers that the staging area reuses
    sfor<4>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        stage_strip(acc[j], stage, lrow, lh);
        // the strip's bias values (one row of them: the same for the four passes)
        float bv[8];
        epi_bias8<FORM>(ep, bias[j % AHEAD], bv);
        wave_sync();
        sfor<4>([&](auto pc) __attribute__((always_inline)) {
            constexpr int ps = decltype(pc)::value;
            const int r = rl + ps * 16;
            const float *sp = stage + r * kPitch + col8;
            const float4 lo = *reinterpret_cast<const float4 *>(sp);
            const float4 hi = *reinterpret_cast<const float4 *>(sp + 4);
            const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            epi_fast8_core<ACT, FORM>(ep, yLane + ps * yPass + j * 32 * ES, v, src[j % AHEAD][ps], bv);
        });
        if constexpr (j + AHEAD < 4) {
            fetch(std::integral_constant<int, j + AHEAD>{});
        }
        wave_sync();
    });
}

// The same for the 16-bit forms, with every residual load and output store covering 8 rows x 128 bytes (whole cache
// lines) instead of 16 rows x 64 bytes (a 32-column strip of 16-bit values): two strips' 32-row halves are staged at a
// time (32 rows x 64 columns, row pitch 68 floats), and lane -> row rl + 8 * pass, columns col8 .. +8 of the pair.
// The vector memory path serves 64-byte row pieces at half the rate of whole lines. Four units (strip pair jj, row
// half i), the binary operand of two units in flight; the bias of a strip pair is loaded once.
template <int ACT, int FORM>
__device__ __forceinline__ void epilogue_full_rows(const EpiParams &ep, const EpiBatch &ob, const f32x16_t (&acc)[4][2],
                                                   float *stage, int lane, int64_t mW, int64_t nW)
{
    constexpr int P = 68;  // staging pitch in floats (64 columns + 4)
    const int lrow = lane & 31, lh = lane >> 5;
    const int col8 = (lane & 7) * 8, rl = lane >> 3;
    Raw8 src[2][4], bias[2];
    auto fetch = [&](auto uc) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value, jj = u / 2, i = u % 2;
        const int64_t n = nW + jj * 64 + col8;
        if constexpr (i == 0) {
            bias[jj] = epi_prefetch8_bias<FORM>(ep, ob, mW + rl, n);
        }
        sfor<4>([&](auto pc) __attribute__((always_inline)) {
            constexpr int ps = decltype(pc)::value;
            src[u % 2][ps] = epi_prefetch8_src<FORM>(ep, ob, mW + i * 32 + rl + ps * 8, n);
        });
    };
    fetch(std::integral_constant<int, 0>{});
    fetch(std::integral_constant<int, 1>{});
    constexpr int64_t ES = 2;
    char *yLane = static_cast<char *>(ep.y) + (ob.y + (mW + rl) * ep.y_sm + nW + col8) * ES;
    __syncthreads();  // every wave is done with the tile buffers that the staging area reuses
    sfor<4>([&](auto uc) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value, jj = u / 2, i = u % 2;
#pragma unroll
        for (int sh = 0; sh < 2; ++sh) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                float *dst = stage + lrow * P + sh * 32 + q4 * 8 + lh * 4;
                const f32x16_t &a = acc[2 * jj + sh][i];
                *reinterpret_cast<float4 *>(dst) = make_float4(a[4 * q4 + 0], a[4 * q4 + 1], a[4 * q4 + 2], a[4 * q4 + 3]);
            }
        }
        float bv[8];
        epi_bias8<FORM>(ep, bias[jj], bv);
        wave_sync();
        sfor<4>([&](auto pc) __attribute__((always_inline)) {
            constexpr int ps = decltype(pc)::value;
            const float *sp = stage + (rl + ps * 8) * P + col8;
            const float4 lo = *reinterpret_cast<const float4 *>(sp);
            const float4 hi = *reinterpret_cast<const float4 *>(sp + 4);
            const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            epi_fast8_core<ACT, FORM>(ep, yLane + ((i * 32 + ps * 8) * ep.y_sm + jj * 64) * ES, v, src[u % 2][ps], bv);
        });
        if constexpr (u + 2 < 4) {
            fetch(std::integral_constant<int, u + 2>{});
        }
        wave_sync();
    });
}

// Epilogue of a tile that crosses the matrix edge, in a fixed form: whole 8-column groups as in a full tile, the
// last partial group of a row one element at a time; rolled loops keep the code small.
template <int ACT, int FORM>
__device__ __forceinline__ void epilogue_edge(const EpiParams &ep, const EpiBatch &ob, const f32x16_t (&acc)[4][2],
                                              float *stage, int lane, int64_t mW, int64_t nW, int64_t M, int64_t N)
{
    const int lrow = lane & 31, lh = lane >> 5;
    const int col8 = (lane & 3) * 8, rl = lane >> 2;
    __syncthreads();  // every wave is done with the tile buffers that the staging area reuses
    sfor<4>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nW + j * 32 + col8;
        stage_strip(acc[j], stage, lrow, lh);
        wave_sync();
#pragma unroll 1
        for (int ps = 0; ps < 4; ++ps) {
            const int r = rl + ps * 16;
            const int64_t m = mW + r;
            const float *src = stage + r * kPitch + col8;
            if (m < M && n + 7 < N) {
                const float4 lo = *reinterpret_cast<const float4 *>(src);
                const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
                const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                epi_fast8<ACT, FORM>(ep, ob, m, n, v, epi_prefetch8<FORM>(ep, ob, m, n));
            } else if (m < M) {
#pragma unroll 1
                for (int q = 0; q < 8; ++q) {
                    if (n + q < N) {
                        epi_elem<ACT, FORM>(ep, ob, m, n + q, src[q]);
                    }
                }
            }
        }
        wave_sync();
    });
}

// Epilogue of any tile in the generic form: one element at a time through epi_apply (activation read at run time).
__device__ __forceinline__ void epilogue_generic(const EpiParams &ep, const EpiBatch &ob, const f32x16_t (&acc)[4][2],
                                                 float *stage, int lane, int64_t mW, int64_t nW, int64_t M, int64_t N)
{
    const int lrow = lane & 31, lh = lane >> 5;
    const int col8 = (lane & 3) * 8, rl = lane >> 2;
    __syncthreads();  // every wave is done with the tile buffers that the staging area reuses
    sfor<4>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nW + j * 32 + col8;
        stage_strip(acc[j], stage, lrow, lh);
        wave_sync();
#pragma unroll 1
        for (int ps = 0; ps < 4; ++ps) {
            const int r = rl + ps * 16;
            const int64_t m = mW + r;
            if (m < M) {
#pragma unroll 1
                for (int q = 0; q < 8; ++q) {
                    if (n + q < N) {
                        epi_apply(ep, ob, m, n + q, stage[r * kPitch + col8 + q]);
                    }
                }
            }
        }
        wave_sync();
    });
}

// Epilogue of the integer form (s8 x s8 -> s32): the accumulators hold int32 bit patterns; y = acc + bias exactly.
__device__ __forceinline__ void epilogue_int(const EpiParams &ep, const EpiBatch &ob, const f32x16_t (&acc)[4][2],
                                             float *stage, int lane, int64_t mW, int64_t nW, int64_t M, int64_t N)
{
    const int lrow = lane & 31, lh = lane >> 5;
    const int col8 = (lane & 3) * 8, rl = lane >> 2;
    __syncthreads();  // every wave is done with the tile buffers that the staging area reuses
    sfor<4>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nW + j * 32 + col8;
        stage_strip(acc[j], stage, lrow, lh);
        wave_sync();
#pragma unroll 1
        for (int ps = 0; ps < 4; ++ps) {
            const int r = rl + ps * 16;
            const int64_t m = mW + r;
            const float *src = stage + r * kPitch + col8;
            if (ep.fast8 && m < M && n + 7 < N) {
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
        wave_sync();
    });
}

typedef float v4f __attribute__((ext_vector_type(4)));

// A K slice's sums of a tile, stored as f32 rows (pitch ld floats) through the same staging as the epilogues: lane ->
// row rl + 16 * pass, columns col8 .. +8 of each strip, two 16-byte non-temporal stores; an edge tile stores only its
// elements inside the matrix.
__device__ __forceinline__ void epilogue_partial(float *out, int64_t ld, const f32x16_t (&acc)[4][2], float *stage,
                                                 int lane, int64_t mW, int64_t nW, int64_t M, int64_t N)
{
    const int lrow = lane & 31, lh = lane >> 5;
    const int col8 = (lane & 3) * 8, rl = lane >> 2;
    __syncthreads();  // every wave is done with the tile buffers that the staging area reuses
    sfor<4>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        const int64_t n = nW + j * 32 + col8;
        stage_strip(acc[j], stage, lrow, lh);
        wave_sync();
#pragma unroll
        for (int ps = 0; ps < 4; ++ps) {
            const int r = rl + ps * 16;
            const int64_t m = mW + r;
            const float *src = stage + r * kPitch + col8;
            float *dst = out + m * ld + n;
            if (m < M && n + 7 < N) {
                __builtin_nontemporal_store(*reinterpret_cast<const v4f *>(src), reinterpret_cast<v4f *>(dst));
                __builtin_nontemporal_store(*reinterpret_cast<const v4f *>(src + 4), reinterpret_cast<v4f *>(dst + 4));
            } else if (m < M) {
                for (int q = 0; q < 8; ++q) {
                    if (n + q < N) {
                        dst[q] = src[q];
                    }
                }
            }
        }
        wave_sync();
    });
}

// Tail split of the grid. Whole rounds of tiles (one tile per CU) run data-parallel, one workgroup per tile. The
// k-iterations of the remaining tiles are divided evenly between one workgroup per CU (a second launch), so the last
// round ends with every CU busy instead of (tiles mod CUs) of them. A tile whose iterations span several workgroups
// is finished by the last of them to arrive: every contributor stores its accumulators (fp32, or int32 bit patterns)
// in its slot of the workspace and takes a ticket from the tile's counter; the holder of the last ticket sums all the
// slots, its own included, in contributor order (so the result does not depend on which workgroup arrives last) and
// runs the epilogue. No workgroup ever waits for another one.
// The slots are written and read with agent-scope atomic stores and loads, which are coherent across the XCDs' L2
// caches access by access, and every wave waits for its stores to complete before the ticket is taken. A device-scope
// fence would do the same by writing back and invalidating a whole L2, which evicts the operand panels that the
// other workgroups of that XCD are streaming.
struct SkArgs {
    float *part;    // nTail x maxc slots of 256 x 256 accumulators
    uint32_t *cnt;  // nTail arrival counters, zeroed by the data-parallel launch (or by sk_zero_kernel)
    int D;          // tiles of the data-parallel launch (whole rounds; the tail's tiles follow them in tile order)
    int nTail;      // tiles of the tail
    int L;          // k-iterations per tail workgroup (the last one may have fewer)
    int maxc;       // slots per tail tile: the most workgroups any tail tile spans
    // K slices (EPI_FORM_PARTIAL): slice z of every tile sums k-tiles z * sliceKT .. + sliceKT - 1 and stores them to
    // slices + z * sliceFloats, row pitch sliceLd floats
    float *slices;
    int64_t sliceFloats, sliceLd;
    int sliceKT, nSlices;
    // tail slices: the sliced tiles are logical tiles tileBase .. tileBase + nTiles - 1, and slice z of sliced tile i
    // is a 256 x 256 block at slices + (z * nTiles + i) * kSlotFloats (row pitch 256); tileBase = 0: every tile,
    // stored at slices + z * sliceFloats with the matrix's own coordinates
    int tileBase, nTiles;
};

constexpr int kSlotFloats = kBM * kBN;  // one 256 x 256 accumulator tile

// K-major B (BKM). A weight stored [K][N] (N contiguous, the K-major W{K,N} of a transposed nn.Linear) is read in
// place instead of packed: a k-tile of B is 64 k-rows of 512 bytes (256 n), copied two rows per 1 KB copy, and held
// in LDS as [64 k][32 chunks of 16 bytes] with chunk c of row k in slot c ^ (4 * (k % 4)). The MFMA wants 8
// consecutive k of one n per lane, which ds_read_b64_tr_b16 delivers: within each 16-lane group, address lane
// a = 4 jj + q reads 4 consecutive n (n0 + 4q .. +3) of row k0 + jj, and output lane i receives element i % 4 of
// address lane 4 jj + i / 4 for jj = 0..3, that is n0 + i at k0 .. k0 + 3 (measured on gfx950). Two such reads give
// a lane its 8 k. In a half-wave the four rows sit at four distinct 64-byte offsets modulo 256 bytes, so the reads are
// free of bank conflicts. Needs K a multiple of 64 (no edge along k) and N of 8. At an edge along n, a k-row's copy
// runs past column N into the first columns of the next k-row; the last k-row's copy goes through a resource that
// starts at its own first row and ends at the operand's last byte, so the range check blanks the chunks past the end
// (kmajor_copy.h). Those values reach only accumulator columns >= N, which the epilogues never store.
//
// CT: operand type, KUDNN_DT_BF16 / F16 / S8. SK: false for the data-parallel launch (block -> one whole tile),
// true for the tail launch (block -> a range of k-iterations over one or more tiles). BKM: B is K-major (bf16 / f16,
// data-parallel launch only).
template <int CT, int ACT, int FORM, bool SK, bool BKM = false>
__global__ __launch_bounds__(512, 1) void gemm_pingpong_kernel(GemmOperands op, EpiParams ep, int tilesM, int tilesN,
                                                               int group, SkArgs sk)
{
    static_assert(!BKM || (!SK && CT != KUDNN_DT_S8), "K-major B: 16-bit operands, data-parallel launch");
    constexpr uint32_t ES = CT == KUDNN_DT_S8 ? 1u : 2u;  // element size in bytes
    __shared__ uint4 a0[kTile], a1[kTile], b0[kTile], b1[kTile], b2[kTile];
    auto abuf = [&](auto ic) __attribute__((always_inline)) -> uint4 * {
        if constexpr (decltype(ic)::value % 2 == 0) return a0; else return a1;
    };
    auto bbuf = [&](auto ic) __attribute__((always_inline)) -> uint4 * {
        constexpr int I = decltype(ic)::value % 3;
        if constexpr (I == 0) return b0; else if constexpr (I == 1) return b1; else return b2;
    };

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = wave >> 2, p = wave & 3;
    const int M = static_cast<int>(op.M), N = static_cast<int>(op.N), K = static_cast<int>(op.K);

    const int64_t batch = blockIdx.y;
    const int64_t i2 = batch % ep.bdim[2];
    const int64_t i1 = (batch / ep.bdim[2]) % ep.bdim[1];
    const int64_t i0 = batch / (ep.bdim[2] * ep.bdim[1]);
    const uint8_t *A = static_cast<const uint8_t *>(op.a) + (i0 * op.a_bs[0] + i1 * op.a_bs[1] + i2 * op.a_bs[2]) * ES;
    const uint8_t *B = static_cast<const uint8_t *>(op.b) + (i0 * op.b_bs[0] + i1 * op.b_bs[1] + i2 * op.b_bs[2]) * ES;
    const uint32_t lda = static_cast<uint32_t>(op.lda) * ES, ldb = static_cast<uint32_t>(op.ldb) * ES;  // row pitch, bytes
    // bytes of each operand after its base, through the end of its last row (K-major B: K rows of N elements); a row
    // count of one has a pitch of 0 in the descriptors, so the count times the pitch is not the extent
    const uint32_t bytesA = static_cast<uint32_t>(op.M - 1) * lda + static_cast<uint32_t>(op.K) * ES,
                   bytesB = BKM ? static_cast<uint32_t>(op.K - 1) * ldb + static_cast<uint32_t>(op.N) * ES
                                : static_cast<uint32_t>(op.N - 1) * ldb + static_cast<uint32_t>(op.K) * ES;
    const int KT = static_cast<int>(static_cast<uint32_t>(K) * ES / kRowBytes);

    // the data-parallel launch clears the tail launch's arrival counters (the tail runs after it on the stream)
    if constexpr (!SK) {
        if (sk.cnt != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
            for (int i = static_cast<int>(threadIdx.x); i < sk.nTail; i += 512) sk.cnt[i] = 0u;
        }
    }

    // the current segment: tile (m0, n0), k-tiles kb .. kb + nk - 1
    int m0 = 0, n0 = 0, kb = 0, nk = KT;

    // copy addressing: a 1 KB copy covers an 8-row block q (rows 8q .. 8q+7 of the tile); lane -> row lr, LDS slot ls,
    // source chunk ls ^ ((row >> 1) & 7) = ls ^ (4 * (q & 1) + (lr >> 1))
    const int lr = lane >> 3, ls = lane & 7;
    const uint32_t loA0 = lr * lda + static_cast<uint32_t>((ls ^ (lr >> 1)) * 16);
    const uint32_t loA1 = lr * lda + static_cast<uint32_t>((ls ^ (4 + (lr >> 1))) * 16);
    // K-major B: a 1 KB copy covers rows 2q, 2q+1 of the k-tile (kmajor_copy.h); the lane offsets of even and odd q
    const uint32_t loB0 = BKM ? kudnn_km::lane_voff(ldb, static_cast<uint32_t>(lane), 0u)
                              : lr * ldb + static_cast<uint32_t>((ls ^ (lr >> 1)) * 16);
    const uint32_t loB1 = BKM ? kudnn_km::lane_voff(ldb, static_cast<uint32_t>(lane), 1u)
                              : lr * ldb + static_cast<uint32_t>((ls ^ (4 + (lr >> 1))) * 16);
    auto copyA = [&](int q, int t, uint4 *dst) __attribute__((always_inline)) {
        const uint32_t off = static_cast<uint32_t>(m0 + q * 8) * lda + static_cast<uint32_t>((kb + t) * kRowBytes);
        if constexpr (SK) {
            copy_block(A, bytesA, off, (q & 1) ? loA1 : loA0, dst + q * 8 * kKC);
        } else {
            copy_block_edge(A, bytesA, off, (q & 1) ? loA1 : loA0, lds_addr(dst + q * 8 * kKC));
        }
    };
    auto copyB = [&](int q, int t, uint4 *dst) __attribute__((always_inline)) {
        const uint32_t off = BKM ? kudnn_km::block_off(ldb, static_cast<uint32_t>(n0) * ES, static_cast<uint32_t>(kb + t),
                                                       static_cast<uint32_t>(q))
                                 : static_cast<uint32_t>(n0 + q * 8) * ldb + static_cast<uint32_t>((kb + t) * kRowBytes);
        if constexpr (SK) {
            copy_block(B, bytesB, off, (q & 1) ? loB1 : loB0, dst + q * 8 * kKC);
        } else {
            copy_block_edge(B, bytesB, off, (q & 1) ? loB1 : loB0, lds_addr(dst + q * 8 * kKC));
        }
    };
    // the operand this wave streams inside the loop, selected once by value (group 0: A, group 1: B)
    const uint8_t *sX = g == 0 ? A : B;
    const uint32_t sBytes = g == 0 ? bytesA : bytesB;
    const uint32_t sLd = g == 0 ? lda : ldb;
    const uint32_t sLo0 = g == 0 ? loA0 : loB0, sLo1 = g == 0 ? loA1 : loB1;

    bool fullTile = false;  // the segment's tile lies wholly inside the matrix (set per segment)
    bool fullN = false;     // the segment's tile lies wholly inside the matrix along n (set per segment)
    // LDS byte address of the buffer k-tile I goes to: operand 0 = A (double-buffered), 1 = B (triple-buffered)
    auto ldsOf = [&](auto ic, int operand) __attribute__((always_inline)) -> uint32_t {
        constexpr int I = decltype(ic)::value;
        const uint32_t la = lds_addr(I % 2 == 0 ? a0 : a1);
        const uint32_t lb = lds_addr(I % 3 == 0 ? b0 : (I % 3 == 1 ? b1 : b2));
        return operand == 0 ? la : lb;
    };
    // fragment addressing: rows of a 32-row block start at multiples of 32, so the swizzle term depends on lrow only
    const int lrow = lane & 31, lh = lane >> 5;
    const int fsw = (lrow >> 1) & 7;
    const int offA = (p * 64 + lrow) * kKC, offB = (g * 128 + lrow) * kKC;

    f32x16_t acc[4][2];
    uint4 fa[4][2], fb[2][4];

    // K-major B: this lane's byte offset in a B tile for its transposed reads of strip j = 0 (strip j: XOR 64 j):
    // row 8 (lane / 32) + jj, column bytes g * 256 + 64 jj + 16 (2 ((lane / 16) & 1) + (lane & 3) / 2) + 8 (lane & 1)
    // with jj = (lane & 15) / 4; step s and half h add (16 s + 4 h) rows
    const uint32_t kmJJ = static_cast<uint32_t>((lane & 15) >> 2);
    const uint32_t trOff = (8u * static_cast<uint32_t>(lane >> 5) + kmJJ) * 512u + static_cast<uint32_t>(g) * 256u +
                           64u * kmJJ + 16u * (2u * static_cast<uint32_t>((lane >> 4) & 1) + static_cast<uint32_t>((lane & 3) >> 1)) +
                           8u * static_cast<uint32_t>(lane & 1);
    auto readB = [&](const uint4 *bt, auto slotc, auto stepc) __attribute__((always_inline)) {
        constexpr int slot = decltype(slotc)::value, s = decltype(stepc)::value;
        if constexpr (BKM) {
            typedef short v4i16_t __attribute__((ext_vector_type(4)));
            typedef __attribute__((address_space(3))) v4i16_t lds_v4i16;
            typedef __attribute__((address_space(3))) char lds_char;
            lds_char *base = (lds_char *)(const_cast<uint4 *>(bt));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lds_char *pj = base + (trOff ^ static_cast<uint32_t>(64 * j));
                const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(pj + (16 * s) * 512));
                const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(pj + (16 * s + 4) * 512));
                const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
                fb[slot][j] = make_uint4(l2.x, l2.y, h2.x, h2.y);
            }
        } else {
            const int sl = (2 * s + lh) ^ fsw;
#pragma unroll
            for (int j = 0; j < 4; ++j) fb[slot][j] = bt[offB + j * 32 * kKC + sl];
        }
    };
    auto step = [&](auto ic, int t, int sR0) __attribute__((always_inline)) {
        constexpr int I = decltype(ic)::value;
        const uint4 *at = abuf(ic);
        const uint4 *bt = bbuf(ic);
        // ---- memory phase
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int sl = (2 * s + lh) ^ fsw;
#pragma unroll
            for (int i = 0; i < 2; ++i) fa[s][i] = at[offA + i * 32 * kKC + sl];
        }
        if constexpr (SK) {
            const int tt = t + 1 + g;  // group 0 copies A(t+1), group 1 copies B(t+2)
            uint4 *dst = g == 0 ? abuf(std::integral_constant<int, I + 1>{}) : bbuf(std::integral_constant<int, I + 2>{});
            if (tt < nk) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int q = p * 8 + j;
                    copy_block(sX, sBytes, static_cast<uint32_t>(sR0 + q * 8) * sLd + static_cast<uint32_t>((kb + tt) * kRowBytes),
                               (q & 1) ? sLo1 : sLo0, dst + q * 8 * kKC);
                }
            }
        } else {
            const int tt = t + 1 + g;  // group 0 copies A(t+1), group 1 copies B(t+2)
            const uint32_t dl = __builtin_amdgcn_readfirstlane(g == 0 ? ldsOf(std::integral_constant<int, I + 1>{}, 0)
                                                                      : ldsOf(std::integral_constant<int, I + 2>{}, 1));
            if (tt < nk) {
                const uint32_t kofs = static_cast<uint32_t>((kb + tt) * kRowBytes);
                if (BKM && g == 1 && fullN) {
                    // K-major B, a tile inside the matrix along n: the k-tile's 64 rows through one resource from its
                    // first byte at column n0, two rows per copy, the row pair in the scalar offset (which the range
                    // check does not cover, so this form is kept to tiles whose columns all lie inside every k-row)
                    const uint32_t tileOff = kudnn_km::tile_off(
                        sLd, static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(n0)) * ES, static_cast<uint32_t>(kb + tt));
                    const i32x4_rs_t rs = make_rsrc(sX + tileOff, sBytes - tileOff);
                    asm volatile("s_nop 4" ::: "memory");  // wait states after VALU writes of the SGPRs the copies read
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int q = p * 8 + j;
                        copy_lds_fast(rs, (q & 1) ? sLo1 : sLo0, kudnn_km::tile_soff(sLd, static_cast<uint32_t>(q)),
                                      dl + static_cast<uint32_t>(q * 8 * kKC * 16));
                    }
                } else if (BKM && g == 1) {
                    // K-major B, a tile that crosses column N: a resource per copy from the copy's first row, so the
                    // range check blanks the chunks of the last k-row that lie past the operand's end
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int q = p * 8 + j;
                        copy_block_edge(sX, sBytes,
                                        kudnn_km::block_off(sLd, static_cast<uint32_t>(n0) * ES, static_cast<uint32_t>(kb + tt),
                                                            static_cast<uint32_t>(q)),
                                        (q & 1) ? sLo1 : sLo0, dl + static_cast<uint32_t>(q * 8 * kKC * 16));
                    }
                } else if (fullTile) {
                    // one resource from the k-tile's first byte: the lane's row and chunk in the vector offset, the
                    // 8-row block in the scalar offset; every word is scalar arithmetic
                    const uint32_t tileOff = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(sR0)) * sLd + kofs;
                    const i32x4_rs_t rs = make_rsrc(sX + tileOff, sBytes - tileOff);
                    asm volatile("s_nop 4" ::: "memory");  // wait states after VALU writes of the SGPRs the copies read
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int q = p * 8 + j;
                        copy_lds_fast(rs, (q & 1) ? sLo1 : sLo0, static_cast<uint32_t>(q * 8) * sLd,
                                      dl + static_cast<uint32_t>(q * 8 * kKC * 16));
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int q = p * 8 + j;
                        copy_block_edge(sX, sBytes, static_cast<uint32_t>(sR0 + q * 8) * sLd + kofs, (q & 1) ? sLo1 : sLo0,
                                        dl + static_cast<uint32_t>(q * 8 * kKC * 16));
                    }
                }
            }
        }
        // group 1 lets this phase's copies (B(t+2)) fly and waits for the previous phase's (B(t+1)), which group 0
        // reads in the next phase
        if (!SK && g == 1) {
            if (t + 2 < nk) {
                wait_vmcnt<8>();
            } else {
                wait_vmcnt<0>();
            }
        }
        readB(bt, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
        wait_lgkmcnt0();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // ---- compute phase, at raised wave priority
        __builtin_amdgcn_s_setprio(1);
        sfor<4>([&](auto sc) __attribute__((always_inline)) {
            constexpr int s = decltype(sc)::value;
            if constexpr (s + 1 < 4) {
                readB(bt, std::integral_constant<int, (s + 1) & 1>{}, std::integral_constant<int, s + 1>{});
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    if constexpr (CT == KUDNN_DT_BF16) {
                        acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, fb[s & 1][j]),
                                                                            __builtin_bit_cast(bf16x8_t, fa[s][i]), acc[j][i], 0, 0, 0);
                    } else if constexpr (CT == KUDNN_DT_F16) {
                        acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, fb[s & 1][j]),
                                                                           __builtin_bit_cast(f16x8_t, fa[s][i]), acc[j][i], 0, 0, 0);
                    } else {
                        acc[j][i] = __builtin_bit_cast(
                            f32x16_t, __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, fb[s & 1][j]),
                                                                           __builtin_bit_cast(i32x4_t, fa[s][i]),
                                                                           __builtin_bit_cast(i32x16_t, acc[j][i]), 0, 0, 0));
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        });
        __builtin_amdgcn_s_setprio(0);
        // group 0's A(t+1) (its only copies in flight), which it reads in the next phase; (SK) group 1's B(t+1)
        if (g == 0) {
            wait_vmcnt<0>();
        } else if (SK) {
            if (t + 2 < nk) {
                wait_vmcnt<8>();
            } else {
                wait_vmcnt<0>();
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    // Accumulates k-tiles kb .. kb + nk - 1 of tile (m0, n0) into acc (from zero) and leaves every copy landed.
    auto mainloop = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.0f;
            }
        }
        const int sR0 = g == 0 ? m0 : n0;
        fullTile = m0 + kBM <= M && n0 + kBN <= N;
        fullN = kudnn_km::whole_tile(static_cast<uint32_t>(n0), static_cast<uint32_t>(N));
        // prologue: A(0), B(0), B(1); wave w copies 8-row blocks 4w .. 4w+3 of each
#pragma unroll
        for (int j = 0; j < 4; ++j) copyA(wave * 4 + j, 0, a0);
#pragma unroll
        for (int j = 0; j < 4; ++j) copyB(wave * 4 + j, 0, b0);
        if (nk > 1) {
#pragma unroll
            for (int j = 0; j < 4; ++j) copyB(wave * 4 + j, 1, b1);
            wait_vmcnt<4>();
        } else {
            wait_vmcnt<0>();
        }
        __builtin_amdgcn_s_barrier();
        if (g == 1) {
            __builtin_amdgcn_s_barrier();  // group 1 runs one phase behind
        }
        for (int t = 0; t < nk; t += 6) {
            sfor<6>([&](auto ic) __attribute__((always_inline)) {
                if (t + decltype(ic)::value < nk) step(ic, t + decltype(ic)::value, sR0);
            });
        }
        if (g == 0) {
            __builtin_amdgcn_s_barrier();  // matches group 1's extra barrier at the start
        }
        wait_vmcnt<0>();
    };

    // ---- epilogue: wave (p, g) owns rows p*64 .. +64, columns g*128 .. +128; 4 strips of 32 columns
    // 64 x 36 floats (9 KB) per wave: waves 0-2 stage in a0, 3-5 in a1, 6-7 in b0
    float *stage = reinterpret_cast<float *>(wave < 3 ? a0 : (wave < 6 ? a1 : b0)) + (wave % 3) * (64 * kPitch);
    const EpiBatch ob = epi_batch_offsets(ep, batch);
    auto epilogue = [&]() __attribute__((always_inline)) {
        // each epilogue starts with a barrier: every wave is done with the tile buffers that the staging area reuses
        const int64_t mW = m0 + p * 64, nW = n0 + g * 128;
        if constexpr (FORM == EPI_FORM_I32) {
            epilogue_int(ep, ob, acc, stage, lane, mW, nW, M, N);
        } else if constexpr (FORM == EPI_FORM_GENERIC) {
            epilogue_generic(ep, ob, acc, stage, lane, mW, nW, M, N);
        } else if constexpr (FORM != EPI_FORM_PARTIAL) {
            if (m0 + kBM <= M && n0 + kBN <= N && (ep.bias == nullptr || ep.bias_sm == 0)) {
                if constexpr (FORM == EPI_FORM_F32) {
                    epilogue_full<ACT, FORM>(ep, ob, acc, stage, lane, mW, nW);  // 32 f32 columns: whole lines already
                } else {
                    epilogue_full_rows<ACT, FORM>(ep, ob, acc, stage, lane, mW, nW);
                }
            } else {
                epilogue_edge<ACT, FORM>(ep, ob, acc, stage, lane, mW, nW, M, N);
            }
        }
    };

    if constexpr (!SK && FORM == EPI_FORM_PARTIAL) {
        // K slices: logical block z * tiles + t (consecutive logical blocks share an XCD, so one XCD's workgroups work
        // on neighbouring tiles of one slice and share its A and B panels in L2)
        const int tiles = sk.nTiles;
        const int lid = xcd_remap(blockIdx.x, gridDim.x);
        const int z = lid / tiles, ti = lid - z * tiles;
        int tm, tn;
        grouped_tile(sk.tileBase + ti, tilesM, tilesN, group, tm, tn);
        m0 = tm * kBM;
        n0 = tn * kBN;
        kb = z * sk.sliceKT;
        nk = min(sk.sliceKT, KT - kb);
        mainloop();
        if (sk.tileBase == 0) {
            epilogue_partial(sk.slices + z * sk.sliceFloats, sk.sliceLd, acc, stage, lane, m0 + p * 64, n0 + g * 128, M, N);
        } else {
            epilogue_partial(sk.slices + static_cast<int64_t>(z * tiles + ti) * kSlotFloats, kBN, acc, stage, lane, p * 64,
                             g * 128, M - m0, N - n0);
        }
    } else if constexpr (!SK) {
        int tm, tn;
        grouped_tile(xcd_remap(blockIdx.x, gridDim.x), tilesM, tilesN, group, tm, tn);
        m0 = tm * kBM;
        n0 = tn * kBN;
        mainloop();
        epilogue();
    } else {
        // this workgroup's k-iterations of the tail: [c * L, c * L + L), XCD-remapped so that the workgroups of one
        // XCD work on neighbouring tiles
        const int c = xcd_remap(blockIdx.x, gridDim.x);
        const int total = sk.nTail * KT;
        int it = c * sk.L;
        const int end = min(it + sk.L, total);
        // slot layout: per wave, 32 quads of 4 accumulators, 64 lanes each (1 KB per quad and wave, coalesced); a
        // quad is two 64-bit atomic accesses
        auto slot_at = [&](int T, int ci) __attribute__((always_inline)) {
            return reinterpret_cast<uint64_t *>(sk.part + (static_cast<int64_t>(T) * sk.maxc + ci) * kSlotFloats) +
                   2 * (wave * 32 * 64 + lane);
        };
        auto pack2 = [](float lo, float hi) __attribute__((always_inline)) {
            return static_cast<uint64_t>(__builtin_bit_cast(uint32_t, lo)) |
                   (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, hi)) << 32);
        };
        uint32_t *ticket = reinterpret_cast<uint32_t *>(b1);  // broadcast slot: b1 holds no staging area
        while (it < end) {
            const int T = it / KT;
            kb = it - T * KT;
            nk = min(KT - kb, end - it);
            int tm, tn;
            grouped_tile(sk.D + T, tilesM, tilesN, group, tm, tn);
            m0 = tm * kBM;
            n0 = tn * kBN;
            mainloop();
            const int cf = (T * KT) / sk.L, cl = ((T + 1) * KT - 1) / sk.L;
            bool last = true;
            if (cl > cf) {
                // a shared tile: publish this workgroup's part, then take a ticket
                uint64_t *mine = slot_at(T, c - cf);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            uint64_t *d = mine + 2 * ((j * 2 + i) * 4 + q) * 64;
                            __hip_atomic_store(d, pack2(acc[j][i][4 * q], acc[j][i][4 * q + 1]), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                            __hip_atomic_store(d + 1, pack2(acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        }
                    }
                }
                wait_vmcnt<0>();  // this wave's part has reached the coherence point
                __syncthreads();
                if (threadIdx.x == 0) {
                    // system scope: the add is performed past the XCDs' private L2 caches
                    ticket[0] = __hip_atomic_fetch_add(&sk.cnt[T], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                }
                __syncthreads();
                last = ticket[0] == static_cast<uint32_t>(cl - cf);
                if (last) {
                    // acc = slot 0 + slot 1 + ... in contributor order, whoever arrived last
                    for (int ci = 0; ci <= cl - cf; ++ci) {
                        uint64_t *part = slot_at(T, ci);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
#pragma unroll
                            for (int i = 0; i < 2; ++i) {
#pragma unroll
                                for (int q = 0; q < 4; ++q) {
                                    uint64_t *src = part + 2 * ((j * 2 + i) * 4 + q) * 64;
                                    const uint64_t v0 = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                    const uint64_t v1 = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                    const uint32_t o[4] = {static_cast<uint32_t>(v0), static_cast<uint32_t>(v0 >> 32),
                                                           static_cast<uint32_t>(v1), static_cast<uint32_t>(v1 >> 32)};
#pragma unroll
                                    for (int e = 0; e < 4; ++e) {
                                        const float x = acc[j][i][4 * q + e];
                                        float r;
                                        if constexpr (CT == KUDNN_DT_S8) {
                                            r = __builtin_bit_cast(float, __builtin_bit_cast(int, x) + __builtin_bit_cast(int, o[e]));
                                        } else {
                                            r = x + __builtin_bit_cast(float, o[e]);
                                        }
                                        acc[j][i][4 * q + e] = ci == 0 ? __builtin_bit_cast(float, o[e]) : r;
                                    }
                                }
                            }
                        }
                    }
                    if (threadIdx.x == 0) {
                        __hip_atomic_store(&sk.cnt[T], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);  // next launch
                    }
                }
            }
            if (last) {
                epilogue();
            }
            it += nk;
            __syncthreads();  // the staging area and the ticket are tile buffers the next segment's copies overwrite
        }
    }
}

// Clears the tail's arrival counters when there is no data-parallel launch ahead of it.
__global__ void sk_zero_kernel(uint32_t *cnt, int n)
{
    for (int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x); i < n; i += static_cast<int>(gridDim.x * blockDim.x)) {
        cnt[i] = 0u;
    }
}

}  // namespace

bool kudnn_pingpong_eligible(const GemmOperands &op, int ct)
{
    // whole k-tiles, 16-byte aligned rows, 32-bit buffer offsets (the offset of the first byte past each operand's
    // last row, and that of the row after it, which an edge tile's copies compute); a K-major B also whole 64-deep
    // k-tiles and whole 16-byte chunks of columns, so that its copies are wholly inside the operand or wholly past it
    const int64_t es = ct == KUDNN_DT_S8 ? 1 : 2;
    const int64_t lim = int64_t(1) << 31;
    const bool aFits = op.M * op.lda * es < lim && ((op.M - 1) * op.lda + op.K) * es < lim;
    if (op.b_kmajor) {
        return (ct == KUDNN_DT_BF16 || ct == KUDNN_DT_F16) && op.K > 0 && op.K % 64 == 0 && op.N % 8 == 0 &&
               (op.lda * es) % 16 == 0 && (op.ldb * es) % 16 == 0 && op.ldb >= op.N && aFits &&
               op.K * op.ldb * es < lim && reinterpret_cast<uintptr_t>(op.b) % 16 == 0;
    }
    return (ct == KUDNN_DT_BF16 || ct == KUDNN_DT_F16 || ct == KUDNN_DT_S8) && (op.K * es) % kRowBytes == 0 &&
           (op.lda * es) % 16 == 0 && (op.ldb * es) % 16 == 0 && aFits && op.N * op.ldb * es < lim &&
           ((op.N - 1) * op.ldb + op.K) * es < lim && op.K > 0;
}

namespace {

// How a launch splits into the data-parallel rounds and the tail (all zero: one data-parallel launch).
struct SkPlan {
    int D = 0, nTail = 0, L = 0, maxc = 0, nWG = 0;
    size_t slotBytes = 0, bytes = 0;
};

size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// CUs of the current device, queried once per device (0 when there is none).
int cu_count()
{
    static std::atomic<int> cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 0;
    }
    int cus = cache[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
            (void)hipGetLastError();
            return 0;
        }
        cache[dev].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

// The tail split pays only for grids of at most a quarter of the CUs with long K (at least 128 k-tiles, 24 or more
// per workgroup), measured on MI355X: at 128 tiles it lost to the unsplit launch (1024 x 8192 x 8192: 158 against
// 141 us), and for 16-bit operands the K slices beat it below (512 x 4096 x 14336: 83 against 156 us). Behind whole rounds of tiles it loses: the tail's workgroups start at k offsets
// spread over the whole K range, so they no longer read the same A and B panels at the same time as their XCD's
// other workgroups, and the copies that then miss the L2 cost more than the idle CUs did (C3: 441 us split against
// 324 us unsplit). KUDNN_HIP_FORCE_STREAMK=1 forces it for any tail (tests), =0 turns it off.
SkPlan sk_plan(const GemmOperands &op, int64_t batches, int ct)
{
    SkPlan s;
    const int64_t es = ct == KUDNN_DT_S8 ? 1 : 2;
    if (batches != 1 || op.K <= 0 || (op.K * es) % kRowBytes != 0 || op.b_kmajor) {
        return s;
    }
    const char *f = std::getenv("KUDNN_HIP_FORCE_STREAMK");
    const int force = f != nullptr ? std::atoi(f) : -1;
    if (force == 0) {
        return s;
    }
    const int cus = cu_count();
    if (cus <= 0) {
        return s;
    }
    const int64_t tiles = ((op.M + kBM - 1) / kBM) * ((op.N + kBN - 1) / kBN);
    const int KT = static_cast<int>(op.K * es / kRowBytes);
    const int rem = static_cast<int>(tiles % cus);
    if (rem == 0 || (force != 1 && (tiles != rem || rem * 4 > cus || KT < 128))) {
        return s;
    }
    const int64_t total = static_cast<int64_t>(rem) * KT;
    const int L = static_cast<int>((total + cus - 1) / cus);
    if (force != 1 && L < 24) {
        return s;
    }
    int maxc = 1;
    for (int t = 0; t < rem; ++t) {
        maxc = std::max(maxc, ((t + 1) * KT - 1) / L - (t * KT) / L + 1);
    }
    s.D = static_cast<int>(tiles - rem);
    s.nTail = rem;
    s.L = L;
    s.maxc = maxc;
    s.nWG = static_cast<int>((total + L - 1) / L);
    s.slotBytes = align256(static_cast<size_t>(rem) * maxc * kSlotFloats * sizeof(float));
    s.bytes = s.slotBytes + align256(static_cast<size_t>(rem) * sizeof(uint32_t));
    return s;
}

// K slices of a small grid: every tile's k-tiles are divided into S slices of sliceKT, one workgroup per (tile, slice),
// all run by the data-parallel kernel's own loop; each stores its f32 sums, and slice_reduce_kernel adds the S slices
// of every output element in slice order and runs the epilogue. Unlike the tail split, no workgroup waits on or reads
// another's results inside the launch, and the slices' workgroups keep the data-parallel copy path and L2 sharing.
// S from kudnn_kslice_rule; KUDNN_HIP_FORCE_KSLICES=S forces S slices (0: none). Where that gives none, a grid of
// more tiles than CUs may slice only its last partial round (kudnn_tail_slice_rule; KUDNN_HIP_FORCE_TAILSLICES=S):
// the full rounds run first as one data-parallel launch of whole tiles.
struct SlicePlan {
    int S = 0, sliceKT = 0;
    int64_t ld = 0;
    size_t bytes = 0;
    int tileBase = 0, tail = 0;  // tail slices: tiles tileBase .. tileBase + tail - 1 sliced, the others whole
};

SlicePlan slice_plan(const GemmOperands &op, int64_t batches, int ct)
{
    SlicePlan s;
    if (batches != 1 || ct == KUDNN_DT_S8 || op.K <= 0 || (op.K * 2) % kRowBytes != 0) {
        return s;
    }
    const int KT = static_cast<int>(op.K * 2 / kRowBytes);
    const char *f = std::getenv("KUDNN_HIP_FORCE_KSLICES");
    int S = f != nullptr ? std::atoi(f) : kudnn_kslice_rule(op.M, op.N, KT, batches, ct);
    if (S < 2) {
        // the last partial round of a grid larger than the CUs: its tiles split into slices, the full rounds run whole
        const char *ft = std::getenv("KUDNN_HIP_FORCE_TAILSLICES");
        const int cus = cu_count();
        if (cus <= 0 || (ft == nullptr && (f != nullptr || std::getenv("KUDNN_HIP_FORCE_STREAMK") != nullptr))) {
            return s;
        }
        const int64_t tiles = ((op.M + kBM - 1) / kBM) * ((op.N + kBN - 1) / kBN);
        const int rem = static_cast<int>(tiles % cus);
        const int St = ft != nullptr ? std::atoi(ft) : kudnn_tail_slice_rule(op.M, op.N, KT, batches, ct, cus);
        if (tiles <= cus || rem == 0 || St < 2) {
            return s;
        }
        s.sliceKT = (KT + std::min(St, KT) - 1) / std::min(St, KT);
        s.S = (KT + s.sliceKT - 1) / s.sliceKT;
        if (s.S < 2) {
            return SlicePlan{};
        }
        s.tail = rem;
        s.tileBase = static_cast<int>(tiles - rem);
        s.ld = kBN;
        s.bytes = align256(static_cast<size_t>(s.S) * static_cast<size_t>(rem) * kSlotFloats * sizeof(float));
        return s;
    }
    S = std::min(S, KT);
    s.sliceKT = (KT + S - 1) / S;
    s.S = (KT + s.sliceKT - 1) / s.sliceKT;  // no empty slice
    if (s.S < 2) {
        return SlicePlan{};
    }
    s.ld = (op.N + 7) / 8 * 8;
    s.bytes = align256(static_cast<size_t>(s.S) * static_cast<size_t>(op.M) * static_cast<size_t>(s.ld) * sizeof(float));
    return s;
}

// Tail slices as the reduction sees them: sliced tiles tileBase .. tileBase + nTiles - 1 of the grouped tile order
// (nTiles = 0: the whole matrix is sliced).
struct SliceTiles {
    int tileBase, nTiles, tilesM, tilesN, group;
};

// One thread per run of 8 columns (m, n .. n + 7): the sum of the S slices in slice order, then the epilogue of FORM.
// Whole-matrix slices: threads in row-major order over the matrix. Tail slices: 32 workgroups per sliced tile, each
// 8 rows of it (32 threads per row).
template <int ACT, int FORM>
__global__ __launch_bounds__(256) void slice_reduce_kernel(const float *slices, int64_t sliceFloats, int64_t ld, int S,
                                                           int64_t M, int64_t N, EpiParams ep, SliceTiles st)
{
    int64_t m, n;
    const float *src;
    if (st.nTiles == 0) {
        const int64_t groupsN = (N + 7) / 8;
        const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
        if (idx >= M * groupsN) {
            return;
        }
        m = idx / groupsN;
        n = (idx - m * groupsN) * 8;
        src = slices + m * ld + n;
    } else {
        const int ti = static_cast<int>(blockIdx.x / 32);
        const int r = static_cast<int>(blockIdx.x % 32) * 8 + static_cast<int>(threadIdx.x / 32);
        const int c = static_cast<int>(threadIdx.x % 32) * 8;
        int tm, tn;
        grouped_tile(st.tileBase + ti, st.tilesM, st.tilesN, st.group, tm, tn);
        m = static_cast<int64_t>(tm) * kBM + r;
        n = static_cast<int64_t>(tn) * kBN + c;
        if (m >= M || n >= N) {
            return;
        }
        src = slices + static_cast<int64_t>(ti) * kSlotFloats + r * kBN + c;
    }
    const EpiBatch ob{0, 0, 0, 0, 0, 0};
    float v[8];
    if (n + 7 < N) {
        v4f lo = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(src));
        v4f hi = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(src + 4));
        for (int z = 1; z < S; ++z) {
            lo += __builtin_nontemporal_load(reinterpret_cast<const v4f *>(src + z * sliceFloats));
            hi += __builtin_nontemporal_load(reinterpret_cast<const v4f *>(src + z * sliceFloats + 4));
        }
        v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
        v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
        if constexpr (FORM == EPI_FORM_GENERIC) {
#pragma unroll
            for (int q = 0; q < 8; ++q) epi_apply(ep, ob, m, n + q, v[q]);
        } else {
            epi_fast8<ACT, FORM>(ep, ob, m, n, v, epi_prefetch8<FORM>(ep, ob, m, n));
        }
        return;
    }
    for (int q = 0; n + q < N; ++q) {
        float x = src[q];
        for (int z = 1; z < S; ++z) x += src[z * sliceFloats + q];
        if constexpr (FORM == EPI_FORM_GENERIC) {
            epi_apply(ep, ob, m, n + q, x);
        } else {
            epi_elem<ACT, FORM>(ep, ob, m, n + q, x);
        }
    }
}

using SliceReduceKernel = decltype(&slice_reduce_kernel<0, EPI_FORM_GENERIC>);

// The reduce instance of the epilogue's activation and tensor types (the generic one for the others).
template <int CT>
SliceReduceKernel select_slice_reduce(const EpiParams &ep)
{
    SliceReduceKernel kernel = nullptr;
    const int form = epi_form(ep);
    auto pick = [&](auto formc) {
        constexpr int F = decltype(formc)::value;
        switch (ep.act) {
            case KUDNN_ACT_UNIMPLEMENTED: kernel = slice_reduce_kernel<KUDNN_ACT_UNIMPLEMENTED, F>; break;
            case KUDNN_ACT_RELU: kernel = slice_reduce_kernel<KUDNN_ACT_RELU, F>; break;
            case KUDNN_ACT_SWISH: kernel = slice_reduce_kernel<KUDNN_ACT_SWISH, F>; break;
            case KUDNN_ACT_GELU_TANH: kernel = slice_reduce_kernel<KUDNN_ACT_GELU_TANH, F>; break;
            case KUDNN_ACT_GELU_ERF: kernel = slice_reduce_kernel<KUDNN_ACT_GELU_ERF, F>; break;
            default: break;
        }
    };
    if constexpr (CT == KUDNN_DT_BF16) {
        if (form == EPI_FORM_BF16) {
            pick(std::integral_constant<int, EPI_FORM_BF16>{});
        } else if (form == EPI_FORM_F32) {
            pick(std::integral_constant<int, EPI_FORM_F32>{});
        }
    } else if (form == EPI_FORM_F16) {
        pick(std::integral_constant<int, EPI_FORM_F16>{});
    }
    return kernel != nullptr ? kernel : slice_reduce_kernel<0, EPI_FORM_GENERIC>;
}

using PingpongKernel = decltype(&gemm_pingpong_kernel<KUDNN_DT_BF16, 0, EPI_FORM_GENERIC, false>);

// The activation and the tensor types of the epilogue select one of the compiled variants.
template <int CT, bool SK, bool BKM = false>
PingpongKernel select_pingpong(const EpiParams &ep)
{
    PingpongKernel kernel = nullptr;
    const int form = epi_form(ep);
    if constexpr (CT == KUDNN_DT_S8) {
        if (form == EPI_FORM_I32) {
            kernel = gemm_pingpong_kernel<CT, 0, EPI_FORM_I32, SK>;
        }
    } else {
        auto pick = [&](auto formc) {
            constexpr int F = decltype(formc)::value;
            switch (ep.act) {
                case KUDNN_ACT_UNIMPLEMENTED: kernel = gemm_pingpong_kernel<CT, KUDNN_ACT_UNIMPLEMENTED, F, SK, BKM>; break;
                case KUDNN_ACT_RELU: kernel = gemm_pingpong_kernel<CT, KUDNN_ACT_RELU, F, SK, BKM>; break;
                case KUDNN_ACT_SWISH: kernel = gemm_pingpong_kernel<CT, KUDNN_ACT_SWISH, F, SK, BKM>; break;
                case KUDNN_ACT_GELU_TANH: kernel = gemm_pingpong_kernel<CT, KUDNN_ACT_GELU_TANH, F, SK, BKM>; break;
                case KUDNN_ACT_GELU_ERF: kernel = gemm_pingpong_kernel<CT, KUDNN_ACT_GELU_ERF, F, SK, BKM>; break;
                default: break;
            }
        };
        // bf16 operands compile the bf16 and f32 output forms, f16 operands the f16 form; the rest is generic
        if constexpr (CT == KUDNN_DT_BF16) {
            if (form == EPI_FORM_BF16) {
                pick(std::integral_constant<int, EPI_FORM_BF16>{});
            } else if (form == EPI_FORM_F32) {
                pick(std::integral_constant<int, EPI_FORM_F32>{});
            }
        } else {
            if (form == EPI_FORM_F16) {
                pick(std::integral_constant<int, EPI_FORM_F16>{});
            }
        }
        if (kernel == nullptr && form != EPI_FORM_I32) {
            // the other activation kinds, and the other tensor types, read everything at run time
            kernel = gemm_pingpong_kernel<CT, 0, EPI_FORM_GENERIC, SK, BKM>;
        }
    }
    return kernel;
}

template <int CT>
int launch_pingpong(const GemmOperands &op, const EpiParams &ep, int64_t batches, void *ws, bool slicesOk,
                    hipStream_t stream)
{
    const int tilesM = static_cast<int>((op.M + kBM - 1) / kBM);
    const int tilesN = static_cast<int>((op.N + kBN - 1) / kBN);
    if constexpr (CT != KUDNN_DT_S8) {
        const SlicePlan sl = ws != nullptr && slicesOk ? slice_plan(op, batches, CT) : SlicePlan{};
        if (sl.S >= 2) {
            SkArgs args{};
            args.slices = static_cast<float *>(ws);
            args.sliceFloats = op.M * sl.ld;
            args.sliceLd = sl.ld;
            args.sliceKT = sl.sliceKT;
            args.nSlices = sl.S;
            const PingpongKernel part = op.b_kmajor ? gemm_pingpong_kernel<CT, 0, EPI_FORM_PARTIAL, false, true>
                                                    : gemm_pingpong_kernel<CT, 0, EPI_FORM_PARTIAL, false, false>;
            SliceTiles st{0, 0, tilesM, tilesN, 8};
            if (sl.tail > 0) {
                // the full rounds as whole tiles, then the last round's tiles in slices
                const PingpongKernel dp = op.b_kmajor ? select_pingpong<CT, false, true>(ep) : select_pingpong<CT, false>(ep);
                if (dp == nullptr) {
                    return -1;
                }
                hipLaunchKernelGGL(dp, dim3(static_cast<unsigned>(sl.tileBase)), dim3(512), 0, stream, op, ep, tilesM,
                                   tilesN, 8, args);
                args.tileBase = sl.tileBase;
                args.nTiles = sl.tail;
                args.sliceFloats = static_cast<int64_t>(sl.tail) * kSlotFloats;
                st.tileBase = sl.tileBase;
                st.nTiles = sl.tail;
            } else {
                args.nTiles = tilesM * tilesN;
            }
            hipLaunchKernelGGL(part, dim3(static_cast<unsigned>(args.nTiles * sl.S)), dim3(512), 0, stream, op, ep,
                               tilesM, tilesN, 8, args);
            const int64_t blocks = sl.tail > 0 ? static_cast<int64_t>(sl.tail) * 32 : (op.M * ((op.N + 7) / 8) + 255) / 256;
            hipLaunchKernelGGL(select_slice_reduce<CT>(ep), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                               static_cast<const float *>(ws), args.sliceFloats, sl.ld, sl.S, op.M, op.N, ep, st);
            return hipGetLastError() == hipSuccess ? 0 : -1;
        }
    }
    const SkPlan s = ws != nullptr ? sk_plan(op, batches, CT) : SkPlan{};
    SkArgs args{};
    if (s.nTail > 0) {
        args.part = static_cast<float *>(ws);
        args.cnt = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + s.slotBytes);
        args.D = s.D;
        args.nTail = s.nTail;
        args.L = s.L;
        args.maxc = s.maxc;
    }
    PingpongKernel dp = nullptr;
    if constexpr (CT != KUDNN_DT_S8) {
        dp = op.b_kmajor ? select_pingpong<CT, false, true>(ep) : select_pingpong<CT, false>(ep);
    } else {
        dp = select_pingpong<CT, false>(ep);
    }
    PingpongKernel tail = s.nTail > 0 ? select_pingpong<CT, true>(ep) : nullptr;
    if (dp == nullptr || (s.nTail > 0 && tail == nullptr)) {
        return -1;
    }
    const int dpTiles = s.nTail > 0 ? s.D : tilesM * tilesN;
    if (dpTiles > 0) {
        dim3 grid(static_cast<unsigned>(dpTiles), static_cast<unsigned>(batches));
        hipLaunchKernelGGL(dp, grid, dim3(512), 0, stream, op, ep, tilesM, tilesN, 8, args);
    } else {
        hipLaunchKernelGGL(sk_zero_kernel, dim3(1), dim3(256), 0, stream, args.cnt, args.nTail);
    }
    if (s.nTail > 0) {
        hipLaunchKernelGGL(tail, dim3(static_cast<unsigned>(s.nWG)), dim3(512), 0, stream, op, ep, tilesM, tilesN, 8, args);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

size_t kudnn_pingpong_workspace_bytes(const GemmOperands &op, int64_t batches, int ct, bool slicesOk)
{
    const SlicePlan sl = slicesOk ? slice_plan(op, batches, ct) : SlicePlan{};
    return sl.S >= 2 ? sl.bytes : sk_plan(op, batches, ct).bytes;
}

int kudnn_pingpong_slices(const GemmOperands &op, int64_t batches, int ct)
{
    return slice_plan(op, batches, ct).S;
}

int kudnn_pingpong_slice_tail(const GemmOperands &op, int64_t batches, int ct)
{
    return slice_plan(op, batches, ct).tail;
}

void kudnn_pingpong_split(const GemmOperands &op, int64_t batches, int ct, int *dpTiles, int *tailTiles, int *iters)
{
    const SkPlan s = sk_plan(op, batches, ct);
    *dpTiles = s.D;
    *tailTiles = s.nTail;
    *iters = s.L;
}

// The build passes the digest of this file and the headers it compiles from (kudnn_amd/build.py).
#ifndef KUDNN_PINGPONG_DIGEST
#define KUDNN_PINGPONG_DIGEST "unknown"
#endif
extern "C" __attribute__((visibility("default"))) const char *kudnn_pingpong_source_digest(void)
{
    return KUDNN_PINGPONG_DIGEST;
}

int kudnn_launch_gemm_pingpong(const GemmOperands &op, const EpiParams &ep, int64_t batches, int ct, void *ws,
                               bool slicesOk, hipStream_t stream)
{
    if (!kudnn_pingpong_eligible(op, ct)) {
        return -1;
    }
    switch (ct) {
        case KUDNN_DT_BF16: return launch_pingpong<KUDNN_DT_BF16>(op, ep, batches, ws, slicesOk, stream);
        case KUDNN_DT_F16: return launch_pingpong<KUDNN_DT_F16>(op, ep, batches, ws, slicesOk, stream);
        case KUDNN_DT_S8: return launch_pingpong<KUDNN_DT_S8>(op, ep, batches, ws, slicesOk, stream);
        default: return -1;
    }
}
