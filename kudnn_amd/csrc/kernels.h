// Host-side launchers of the HIP kernels (one translation unit per kernel family).
#ifndef KUDNN_KERNELS_H
#define KUDNN_KERNELS_H

#include <hip/hip_runtime.h>

#include "plan_types.h"

// Tile configurations of the dispatcher (values are stable: they appear in plan descriptions).
enum {
    KUDNN_CFG_BF16_256x256 = 1,
    KUDNN_CFG_BF16_256x128 = 2,
    KUDNN_CFG_BF16_128x128 = 3,
    KUDNN_CFG_BF16_PINGPONG_256x256 = 4,
    KUDNN_CFG_F32_128x128 = 10,
    KUDNN_CFG_F32_64x64 = 11,
    KUDNN_CFG_F32_KSLICE_16x32 = 12,  // small f32 grids: 16 x 32 tiles, K split over the waves of the workgroup
    KUDNN_CFG_SKINNY_BF16 = 20,
    KUDNN_CFG_GEMV_BF16 = 21,  // M == 1: one wave per weight row, X staged in LDS (skinny engine)
    KUDNN_CFG_GEMV_MULTI_BF16 = 22,  // 2 <= M <= 5 (M <= 8 forced): one wave per weight row, X staged in LDS
    KUDNN_CFG_GEMV_KSPLIT_BF16 = 23,  // 2 <= M <= 16, K <= 4096, one batch: K split over 8 waves, X in registers
};

// Returns 0 on success, -1 if the launch failed or cfg is unknown. `ct` is the operand (compute) type of the 16- and
// 8-bit kernels: KUDNN_DT_BF16, KUDNN_DT_F16 (f32 accumulation) or KUDNN_DT_S8 (int32 accumulation, integer
// epilogue only). Their tile configurations keep the bf16 names; an s8 k-tile is 128 elements instead of 64.
// 4-wave MFMA kernels (gemm_mfma.hip). A grid too small for the chip is split along K, in the same launch, when `ws`
// (device memory of at least kudnn_gemm_workspace_bytes bytes, 256-byte aligned) and `counters` (at least
// KUDNN_SPLIT_MAX_TILES uint32, zero; a split launch leaves them zero) are given; with nullptr it runs unsplit. s8
// launches are never split.
constexpr int KUDNN_SPLIT_MAX_TILES = 128;
size_t kudnn_gemm_workspace_bytes(const GemmOperands &op, int64_t batches, int cfg, int ct);
int kudnn_launch_gemm_mfma(const GemmOperands &op, const EpiParams &ep, int64_t batches, int cfg, int ct, void *ws,
                           uint32_t *counters, hipStream_t stream);
// 8-wave ping-pong schedule, 256x256 tile (gemm_pingpong.hip). Needs K a whole number of 128-byte k-tiles, 16-byte
// aligned rows and 32-bit operand offsets; kudnn_pingpong_eligible says whether `op` qualifies.
bool kudnn_pingpong_eligible(const GemmOperands &op, int ct);
// Bytes of workspace the launch wants for its K slices (slicesOk) or its tail split (0: one data-parallel launch);
// `ws` of at least that many bytes, or nullptr to run without either. The launch takes the same slicesOk.
size_t kudnn_pingpong_workspace_bytes(const GemmOperands &op, int64_t batches, int ct, bool slicesOk);
// The split the launch would make: tiles of the data-parallel launch, tail tiles, k-iterations per tail workgroup
// (all 0 when it makes none).
void kudnn_pingpong_split(const GemmOperands &op, int64_t batches, int ct, int *dpTiles, int *tailTiles, int *iters);
// The K slices the launch would make when allowed (0: none).
int kudnn_pingpong_slices(const GemmOperands &op, int64_t batches, int ct);
// Tiles in slices when only the last partial round is sliced (0: none, or every tile).
int kudnn_pingpong_slice_tail(const GemmOperands &op, int64_t batches, int ct);
// The planner's K-slice count for the ping-pong kernel (0: none) of an M x N grid with KT k-tiles of 128 bytes.
// Measured on MI355X over 26 shapes (M 256..4096, N 1152..14336, K 2048..14336, against the unsliced ping-pong, its
// tail split and the 4-wave kernel): up to 64 tiles of 256 x 256, as many slices as keep tiles x slices <= 128 (at
// most 8), each of at least 16 k-tiles, were 1.07-2.4x faster than the best of those, except at 64 tiles with fewer
// than 64 k-tiles, where the 4-wave kernel's 128 x 128 tiles fill the CUs (2048 x 2048 x 2048: 49 against 38 us);
// 80-96 tiles with M >= 1024 and at least 48 k-tiles: two slices, 7-23 % faster (M = 512 lost 3 %, 112-128 tiles up
// to 47 %).
inline int kudnn_kslice_rule(int64_t M, int64_t N, int64_t KT, int64_t batches, int ct)
{
    if (batches != 1 || ct == KUDNN_DT_S8 || M <= 0 || N <= 0) {
        return 0;
    }
    const int64_t tiles = (M + 255) / 256 * ((N + 255) / 256);
    int64_t S = 0;
    if (tiles <= 64) {
        S = 128 / tiles;
        S = S < 8 ? S : 8;
        S = S < KT / 16 ? S : KT / 16;
        if (tiles * 4 >= 256 && KT < 64) {
            S = 0;
        }
    } else if (tiles <= 96 && M >= 1024 && KT >= 48) {
        S = 2;
    }
    return S >= 2 ? static_cast<int>(S) : 0;
}

// Slices of the last partial round of a 16-bit grid of more tiles than CUs, whose full rounds run whole tiles (0:
// none). With R tiles in that round (R = tiles mod CUs): R at most an eighth of the CUs, S = min(CUs / 2 / R, 8,
// KT / 16) when that is at least 2. Measured on MI355X against the unsliced grid (bf16, bias): 3072 x 11008 x 4096
// (R = 4) 265 -> 231 us, 4352 x 4096 x 4096 (R = 16) 168 -> 136 us, 4096 x 4608 x 4096 and 2304 x 8192 x 4096
// (R = 32) 168 -> 148-149 us; R = 64 with 48 k-tiles even, with 24 k-tiles 15 % slower; R = 88, 128 and 176 (C3)
// slower at every S; 18 k-tiles slower at every S.
inline int kudnn_tail_slice_rule(int64_t M, int64_t N, int64_t KT, int64_t batches, int ct, int cus)
{
    if (batches != 1 || ct == KUDNN_DT_S8 || M <= 0 || N <= 0 || cus <= 0) {
        return 0;
    }
    const int64_t tiles = (M + 255) / 256 * ((N + 255) / 256);
    const int64_t rem = tiles % cus;
    if (tiles <= cus || rem == 0 || rem * 8 > cus) {
        return 0;
    }
    int64_t S = cus / 2 / rem;
    S = S < 8 ? S : 8;
    S = S < KT / 16 ? S : KT / 16;
    return S >= 2 ? static_cast<int>(S) : 0;
}

int kudnn_launch_gemm_pingpong(const GemmOperands &op, const EpiParams &ep, int64_t batches, int ct, void *ws,
                               bool slicesOk, hipStream_t stream);
int kudnn_launch_gemm_f32(const GemmOperands &op, const EpiParams &ep, int64_t batches, int cfg, void *ws,
                          uint32_t *counters, hipStream_t stream);
// f32, one 16 x 32 tile per workgroup with K split over its waves (gemm_kslice.hip): no workspace. Needs K a multiple
// of 16, 16-byte aligned operands and row strides; kudnn_kslice_eligible says whether `op` qualifies.
bool kudnn_kslice_eligible(const GemmOperands &op);
int kudnn_launch_gemm_f32_kslice(const GemmOperands &op, const EpiParams &ep, int64_t batches, hipStream_t stream);
// M <= 16, bf16 or f16 operands (`ct`), B contiguous along K (M == 1, and M <= 8 under cfg KUDNN_CFG_GEMV_MULTI_BF16:
// row-per-wave GEMV with X staged in LDS; otherwise 16-row MFMA tiles; 64-bit addressed forms for operands of 2 GiB or
// more).
int kudnn_launch_skinny(const GemmOperands &op, const EpiParams &ep, int64_t batches, int ct, int cfg, hipStream_t stream);

// Pack: dst[b][r][k] (row pitch kp, zero for k >= cols) = convert(src element (b, r, k)) where the source
// element sits at src + b-offset + r*s_r + k*s_k. dst dtype is the compute type: F32, BF16, F16 or S8 (conversions are
// exact: widening, 8-bit integers to f16 or f32, or a copy).
struct PackArgs {
    const void *src;
    int src_dt;
    int64_t rows, cols;      // logical rows (M or N) and K
    int64_t s_r, s_k;        // source strides (elements)
    int64_t bdim[3];
    int64_t bs[3];           // source batch strides
    void *dst;
    int dst_dt;
    int64_t kp;              // destination row pitch (elements), >= cols
    int64_t dst_bstride;     // destination batch stride (elements)
    int shift;               // subtracted from every element (128: u8 -> s8 for the integer MFMA); padding stays 0
};
int kudnn_launch_pack(const PackArgs &p, int64_t batches, hipStream_t stream);
// out[c * rows + r] = scale * (sum over the kp int8 of row r of copy c of a packed operand), in wrapping 32-bit
// arithmetic: the correction terms of an integer GEMM whose other operand was a shifted u8.
int kudnn_launch_rowsum_s8(const int8_t *p, int64_t rows, int64_t kp, int64_t copies, int64_t bstride, uint32_t scale,
                           int32_t *out, hipStream_t stream);

#endif  // KUDNN_KERNELS_H
