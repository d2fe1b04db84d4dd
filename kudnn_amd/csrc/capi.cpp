// C ABI of the MI355X Linear/GEMM path: descriptor validation (restating the reference's rules),
// the tile/shape dispatcher, and the launch sequence (pack, GEMM with fused epilogue).
//
// The dispatcher replaces both the reference's dtype registry (g_gemmImpls + ChooseImpl,
// src/dnn/src/kudnn_gemm.cpp:590-708) and its JIT solution cache (SolutionHandler, src/dnn/src/kudnn_jit.hpp:110-152):
// everything that depends only on descriptors is decided once in *_create and stored in the plan;
// *_run only checks pointer kinds/alignment and launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <unistd.h>

#include "../../include/kudnn_hip.h"
#include "kernels.h"
#include "kslice.h"
#include "layout_table.h"
#include "plan_types.h"

namespace {

// ---------------------------------------------------------------------------------------------------
// errors

thread_local std::string g_lastError;

int Fail(int status, const std::string &msg)
{
    g_lastError = msg;
    return status;
}

int FailStatus(int status, const char *op)
{
    if (status == KUDNN_STATUS_BAD_ARGUMENTS) {
        return Fail(status, std::string(op) + ": bad arguments' Shapes");
    }
    if (status == KUDNN_STATUS_UNSUPPORTED) {
        return Fail(status, std::string(op) + ": unsupported configuration of parameters");
    }
    return status;
}

int HipFail(hipError_t e, const char *what)
{
    return Fail(KUDNN_STATUS_HIP_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

// ---------------------------------------------------------------------------------------------------
// threading state (semantics of src/dnn/src/threading_impl.cpp:44-141; no host threads are used)

struct Threading {
    int available = 1;
    int maxThreads = 1;
    int fixedThreads = 0;
    bool fixed = false;
    int envMode = 0;   // 0 = KUDNN_THREAD_USE_ENV, 1 = KUDNN_THREAD_IGNORE_ENV
    int control = 0;   // 0 = KUDNN_DEFAULT, 1 = KUDNN_MANUAL
    Threading()
    {
        long n = sysconf(_SC_NPROCESSORS_ONLN);
        available = n > 0 ? static_cast<int>(n) : 1;
        maxThreads = available;
        if (const char *f = std::getenv("KUDNN_FIXED_NUM_THREADS")) {
            int v = std::atoi(f);
            if (v > 0) {
                fixed = true;
                fixedThreads = std::min(v, available);
                control = 1;
                return;
            }
        }
        if (const char *m = std::getenv("KUDNN_MAX_NUM_THREADS")) {
            int v = std::atoi(m);
            if (v > 0) {
                maxThreads = std::min(v, available);
                control = 1;
            }
        }
    }
};

Threading &Thr()
{
    static Threading t;
    return t;
}
thread_local int g_localThreads = 0;

int MaxThreads()
{
    if (g_localThreads > 0) {
        return g_localThreads;
    }
    return Thr().fixed ? Thr().fixedThreads : Thr().maxThreads;
}

// ---------------------------------------------------------------------------------------------------
// descriptor helpers

bool IsNone(const kudnn_tensor_desc *d) { return d == nullptr || d->ndims == 0; }

int64_t TotalSize(const kudnn_tensor_desc &d)
{
    if (d.ndims == 0) {
        return 0;
    }
    int64_t t = 1;
    for (int i = 0; i < d.ndims; ++i) {
        t *= d.dims[i];
    }
    return t;
}

int64_t TotalSizeOpt(const kudnn_tensor_desc *d) { return IsNone(d) ? 0 : TotalSize(*d); }

int DtSize(int dt)
{
    switch (dt) {
        case KUDNN_DT_F32: case KUDNN_DT_S32: return 4;
        case KUDNN_DT_F16: case KUDNN_DT_BF16: return 2;
        case KUDNN_DT_S8: case KUDNN_DT_U8: return 1;
        default: return 0;
    }
}

bool IsFp(int dt) { return dt == KUDNN_DT_F32 || dt == KUDNN_DT_F16 || dt == KUDNN_DT_BF16; }

bool DescIsDense(const kudnn_tensor_desc &d)
{
    int64_t mins[KUDNN_HIP_MAX_DIMS];
    if (!kudnn_layout::MinStrides(d.layout, d.ndims, d.dims, mins)) {
        return false;
    }
    for (int i = 0; i < d.ndims; ++i) {
        if (mins[i] != d.strides[i]) {
            return false;
        }
    }
    return true;
}

// Stride of the fastest physical dimension (TensorInfo::HasStrideOverFastestDim, kudnn_tensor_info.hpp:189-192).
int64_t FastestStride(const kudnn_tensor_desc &d)
{
    int l = kudnn_layout::LogicalAt(d.layout, d.ndims - 1);
    return l < 0 ? 0 : d.strides[l];
}

// Extent in elements of the memory a descriptor addresses (max offset + 1).
int64_t Extent(const kudnn_tensor_desc &d)
{
    if (TotalSize(d) == 0) {
        return 0;
    }
    int64_t off = 0;
    for (int i = 0; i < d.ndims; ++i) {
        off += (d.dims[i] - 1) * d.strides[i];
    }
    return off + 1;
}

// ---------------------------------------------------------------------------------------------------
// validation, restated from the reference

// ValidateGemmParams (src/dnn/src/kudnn_gemm.cpp:384-476).
int ValidateGemm(const kudnn_tensor_desc &src, const kudnn_tensor_desc &wei, const kudnn_tensor_desc &dst,
                 const kudnn_tensor_desc *bia, int numThreads)
{
    if (!DescIsDense(dst)) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    if (src.dtype == KUDNN_DT_S32 || wei.dtype == KUDNN_DT_S32) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    if (numThreads < 0 || numThreads > MaxThreads()) {
        return KUDNN_STATUS_BAD_ARGUMENTS;
    }
    const bool biasNull = TotalSizeOpt(bia) == 0;
    bool bad = src.ndims != wei.ndims || src.ndims != dst.ndims;
    if (!biasNull) {
        bad = bad || src.ndims != bia->ndims;
    }
    bad = bad || src.ndims < 2;
    if (bad) {
        return KUDNN_STATUS_BAD_ARGUMENTS;
    }
    const int nd = src.ndims;
    bad = src.dims[nd - 2] != dst.dims[nd - 2] || src.dims[nd - 1] != wei.dims[nd - 2] ||
          wei.dims[nd - 1] != dst.dims[nd - 1];
    if (bad) {
        return KUDNN_STATUS_BAD_ARGUMENTS;
    }
    for (int d = 0; d < nd - 2; ++d) {
        bool badDims = false;
        if (src.dims[d] != 1) {
            badDims = badDims || src.dims[d] != dst.dims[d];
        }
        if (wei.dims[d] != 1 && src.dims[d] != 1) {
            badDims = badDims || src.dims[d] != wei.dims[d];
        }
        if (!biasNull && bia->dims[d] != 1) {
            badDims = badDims || bia->dims[d] != dst.dims[d];
        }
        if (badDims) {
            return KUDNN_STATUS_BAD_ARGUMENTS;
        }
    }
    if (!biasNull) {
        const int64_t bn = bia->dims[nd - 1], bm = bia->dims[nd - 2];
        if ((bn != 1 && bn != dst.dims[nd - 1]) || (bm != 1 && bm != dst.dims[nd - 2])) {
            return KUDNN_STATUS_BAD_ARGUMENTS;
        }
    }
    auto strided = [](const kudnn_tensor_desc &d) {
        int64_t s = FastestStride(d);
        return s != 1 && s != 0;
    };
    // As in the reference, this only triggers when a bias is present and every tensor is strided.
    if (strided(src) && strided(wei) && strided(dst) && (!biasNull && strided(*bia))) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    if (TotalSize(src) == 0 || TotalSize(wei) == 0 || TotalSize(dst) == 0) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    return KUDNN_STATUS_SUCCESS;
}

// ActivationLayerFWD::ValidateInput for src == dst == C (src/dnn/src/kudnn_eltwise.cpp:1479-1515).
int ValidateActivation(const kudnn_tensor_desc &c, int kind, float alpha, float beta)
{
    const bool fp = IsFp(c.dtype);
    const bool intOk = (c.dtype == KUDNN_DT_S32 || c.dtype == KUDNN_DT_S8 || c.dtype == KUDNN_DT_U8) &&
                       (kind == KUDNN_ACT_RELU || kind == KUDNN_ACT_LINEAR);
    if (!(fp || intOk)) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    static const int kSupported[] = {
        KUDNN_ACT_ABS, KUDNN_ACT_CLIP, KUDNN_ACT_CLIP_V2, KUDNN_ACT_ELU, KUDNN_ACT_ELU_DST, KUDNN_ACT_EXP,
        KUDNN_ACT_GELU_ERF, KUDNN_ACT_GELU_TANH, KUDNN_ACT_HARDSIGMOID, KUDNN_ACT_HARDSWISH, KUDNN_ACT_LINEAR,
        KUDNN_ACT_LOG, KUDNN_ACT_SIGMOID, KUDNN_ACT_MISH, KUDNN_ACT_POW, KUDNN_ACT_RELU, KUDNN_ACT_ROUND,
        KUDNN_ACT_SRELU, KUDNN_ACT_SQRT, KUDNN_ACT_SQUARE, KUDNN_ACT_SWISH, KUDNN_ACT_TANH};
    bool known = false;
    for (int k : kSupported) {
        known = known || (k == kind);
    }
    if (!known) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    if (((kind == KUDNN_ACT_CLIP || kind == KUDNN_ACT_CLIP_V2) && alpha > beta) ||
        (kind == KUDNN_ACT_SRELU && alpha == 0.0f)) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    if (!DescIsDense(c)) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    if (TotalSize(c) == 0) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    return KUDNN_STATUS_SUCCESS;
}

// ValidateResParams (src/dnn/src/kudnn_linear_res.cpp:136-166).
int ValidateRes(const kudnn_tensor_desc &a, const kudnn_tensor_desc &b, const kudnn_tensor_desc &c,
                const kudnn_tensor_desc *bias, const kudnn_tensor_desc &res, const kudnn_tensor_desc &lr, int kind,
                int numThreads)
{
    int s = ValidateGemm(a, b, c, bias, numThreads);
    if (s != KUDNN_STATUS_SUCCESS) {
        return s;
    }
    if (kind != KUDNN_RES_EXT && kind != KUDNN_RES_MUL && kind != KUDNN_RES_IDENTIAL) {
        return KUDNN_STATUS_UNSUPPORTED;
    }
    if (kind == KUDNN_RES_MUL) {
        return ValidateGemm(c, res, lr, nullptr, numThreads);
    }
    if (c.ndims != res.ndims || c.ndims != lr.ndims) {
        return KUDNN_STATUS_BAD_ARGUMENTS;
    }
    for (int d = 0; d < c.ndims - 1; ++d) {
        if (c.dims[d] != res.dims[d] || c.dims[d] != lr.dims[d]) {
            return KUDNN_STATUS_BAD_ARGUMENTS;
        }
    }
    return KUDNN_STATUS_SUCCESS;
}

// Every kind of the reference's forward activation table (kudnn_eltwise.cpp:333-400) runs as a fused epilogue;
// RELU, SWISH, GELU_TANH and GELU_ERF have kernels of their own, the rest run in the epilogue's generic form.
bool ActImplemented(int kind)
{
    switch (kind) {
        case KUDNN_ACT_ABS: case KUDNN_ACT_EXP: case KUDNN_ACT_LINEAR: case KUDNN_ACT_LOG: case KUDNN_ACT_RELU:
        case KUDNN_ACT_ROUND: case KUDNN_ACT_SQRT: case KUDNN_ACT_SQUARE: case KUDNN_ACT_TANH: case KUDNN_ACT_SIGMOID:
        case KUDNN_ACT_POW: case KUDNN_ACT_CLIP: case KUDNN_ACT_CLIP_V2: case KUDNN_ACT_HARDSIGMOID:
        case KUDNN_ACT_HARDSWISH: case KUDNN_ACT_ELU: case KUDNN_ACT_GELU_TANH: case KUDNN_ACT_ELU_DST:
        case KUDNN_ACT_SWISH: case KUDNN_ACT_SRELU: case KUDNN_ACT_GELU_ERF: case KUDNN_ACT_MISH:
            return true;
        default:
            return false;
    }
}

// ---------------------------------------------------------------------------------------------------
// host bf16 helper (RNE), used for cblas_bgemm's bf16 alpha/beta (kudnn_gemm.cpp:222-224)

float RoundBf16(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        u = (u | 0x00400000u) & 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    std::memcpy(&f, &u, 4);
    return f;
}

// ---------------------------------------------------------------------------------------------------
// the GEMM core plan: one (possibly batched) GEMM launch plus its operand packs

// ENGINE_MFMA_BF16 and ENGINE_SKINNY_BF16 run the 16- and 8-bit operand types (bf16, f16; s8 on the MFMA engine only).
enum Engine { ENGINE_MFMA_BF16 = 1, ENGINE_MFMA_F32 = 2, ENGINE_SKINNY_BF16 = 3 };

struct OperandSpec {
    int dt = 0;
    int64_t rows = 0;      // M for A, N for B
    int64_t s_r = 0;       // stride along rows (m for A, n for B)
    int64_t s_k = 0;       // stride along k
    int64_t bs[3] = {0, 0, 0};
    bool staticPack = false;  // must be packed whatever the pointer alignment
    bool kmajor = false;      // B read in place as [K][N] (N contiguous): ping-pong (16-bit) or 4-wave fp32 kernels
};

struct TensorSpec {
    int dt = 0;
    int64_t sm = 0, sn = 0;
    int64_t bs[3] = {0, 0, 0};
    int64_t extent = 0;  // elements addressed, for host staging
};

struct GemmCore {
    int engine = 0;
    int cfg = 0;
    int computeDt = 0;
    int64_t M = 0, N = 0, K = 0;
    int64_t bdim[3] = {1, 1, 1};
    bool serial = false;  // C is broadcast over a looped batch dim: run batches in order
    OperandSpec A, B;
    TensorSpec C;
    bool hasBias = false;
    bool bf16Scalars = false;  // cblas_bgemm's bf16 alpha / beta apply (a bf16 GEMM into bf16 without bias)
    TensorSpec Bias;
    int64_t kp = 0;  // packed row pitch (elements)
    int64_t Batches() const { return bdim[0] * bdim[1] * bdim[2]; }
};

void BatchStrides(const kudnn_tensor_desc &t, int64_t bs[3], int64_t dims[3]);
TensorSpec SpecOf(const kudnn_tensor_desc &d);

// Fills slot-indexed batch info: logical dim d of an nd-dim tensor maps to slot d - (nd - 2) + 3.
void BatchStrides(const kudnn_tensor_desc &t, int64_t bs[3], int64_t dims[3])
{
    for (int s = 0; s < 3; ++s) {
        bs[s] = 0;
        dims[s] = 1;
    }
    const int nb = t.ndims - 2;
    for (int d = 0; d < nb; ++d) {
        int s = 3 - nb + d;
        bs[s] = t.strides[d];
        dims[s] = t.dims[d];
    }
}

int ElemsPerChunk(int computeDt) { return 16 / DtSize(computeDt); }

// The dtype ChooseImpl sees for a tensor: BatchedExtendedGemm (kudnn_gemm.cpp:722-765) first reorders every tensor of
// more than two dims whose layout is not the standard ABC.. order into an f32 copy (and a reordered dst back from f32
// afterwards, with the same saturating round-half-even conversion for integer types, vector_convert.hpp:153-179).
int DispatchDt(const kudnn_tensor_desc &d, int nd)
{
    const int standard = nd == 3 ? KUDNN_LAYOUT_ABC : (nd == 4 ? KUDNN_LAYOUT_ABCD : KUDNN_LAYOUT_ABCDE);
    return (nd > 2 && d.layout != standard) ? KUDNN_DT_F32 : d.dtype;
}

// Builds the core plan of C = A x B (+ bias) from validated descriptors. Returns a status.
// `extra` lists further m-indexed epilogue tensors (linearRes, the binary operand) that must allow a batch
// fold too; their batch strides are updated with the core's.
int BuildCore(const kudnn_tensor_desc &a, const kudnn_tensor_desc &b, const kudnn_tensor_desc &c,
              const kudnn_tensor_desc *bias, GemmCore &core, const char *op, TensorSpec *extra0 = nullptr,
              TensorSpec *extra1 = nullptr)
{
    TensorSpec *extras[2] = {extra0, extra1};
    const int nd = a.ndims;
    core.M = a.dims[nd - 2];
    core.K = a.dims[nd - 1];
    core.N = b.dims[nd - 1];

    // dtype combination -> compute type (the registry of kudnn_gemm.cpp:590-601 and the widening / all-f32
    // fallback of ChooseImpl, :628-708):
    //  - s8 / u8 x s8 / u8 -> s32 with an s32 or s8 bias or none: int8 MFMA into exact int32 (cblas_gemm_s8s8s32,
    //    s8u8s32, u8s8s32, u8u8s32 with zero operand offsets, :243-324; an s8 bias is the wider-type match, widened
    //    exactly, :655-671); a u8 operand is packed shifted by -128 and the epilogue adds back the shifted-out terms;
    //  - bf16 x bf16: bf16 MFMA (cblas_sbgemm / cblas_bgemm);
    //  - f16 x f16, f16 x s8, f16 x u8: f16 MFMA (cblas_hgemm / cblas_shgemm; an 8-bit weight is converted to f16
    //    exactly, as the reference's MatrixConverter does before hgemm, :341-372);
    //  - everything else computes in f32, with 8-bit integer operands converted exactly.
    // Every combination but the first forms alpha * sum + beta * C + bias in f32, which is the all-f32 fallback's
    // arithmetic (:673-679): the MFMA products of bf16 / f16 / 8-bit values are exact and accumulate in f32. Integer
    // C and bias elements are read as f32 (s32 rounds to nearest even beyond 2^24, as MatrixConverter's cast does) and
    // an integer output takes ConvertFp32ToS32 / ToS8 / ToU8 (saturate, then round half to even; :690-700,
    // service.cpp:77-115). Summing in f32 in a different order than KML changes nothing while every partial sum is
    // exact in f32 (integer-valued terms below 2^24), so integer outputs match bit for bit there; elsewhere they can
    // differ where the f32 value lies within rounding of a .5 boundary.
    // The choice between the exact integer GEMM and f32 arithmetic, and cblas_bgemm's bf16 scalars, follow the dtypes
    // ChooseImpl sees (DispatchDt; without a bias it sees dst's dtype for the bias, :628-634 with the bias-less
    // TensorInfo of kudnn_gemm.hpp). Among the float compute types the operands' own dtypes choose: bf16 / f16 products
    // are exact in f32 either way.
    const int ea = DispatchDt(a, nd), eb = DispatchDt(b, nd), ec = DispatchDt(c, nd);
    const bool noBias = TotalSizeOpt(bias) == 0;
    const int biasDt = noBias ? c.dtype : DispatchDt(*bias, nd);
    const bool int8a = ea == KUDNN_DT_S8 || ea == KUDNN_DT_U8;
    const bool int8b = eb == KUDNN_DT_S8 || eb == KUDNN_DT_U8;
    core.bf16Scalars = noBias && ea == KUDNN_DT_BF16 && eb == KUDNN_DT_BF16 && ec == KUDNN_DT_BF16;
    if (int8a && int8b && ec == KUDNN_DT_S32 && (biasDt == KUDNN_DT_S32 || biasDt == KUDNN_DT_S8)) {
        core.computeDt = KUDNN_DT_S8;
    } else if (a.dtype == KUDNN_DT_BF16 && b.dtype == KUDNN_DT_BF16) {
        core.computeDt = KUDNN_DT_BF16;
    } else if (a.dtype == KUDNN_DT_F16 &&
               (b.dtype == KUDNN_DT_F16 || b.dtype == KUDNN_DT_S8 || b.dtype == KUDNN_DT_U8)) {
        core.computeDt = KUDNN_DT_F16;
    } else {
        core.computeDt = KUDNN_DT_F32;
    }

    // batch dims
    int64_t aDims[3], bDims[3], cDims[3], tmp[3];
    BatchStrides(a, core.A.bs, aDims);
    BatchStrides(b, core.B.bs, bDims);
    BatchStrides(c, core.C.bs, cDims);
    for (int s = 0; s < 3; ++s) {
        core.bdim[s] = std::max(aDims[s], bDims[s]);
        // The reference's validation (kudnn_gemm.cpp:420-432) checks a weight batch dim against src only when src's
        // dim is not 1, so src [1,M,K] x wei [4,K,N] -> dst [2,M,N] passes it; its CPU loop then walks dst and a
        // dst-shaped bias past their ends. On the GPU that would be an out-of-bounds write, so a C batch dim must be
        // 1 (C broadcast: the serial loop) or the batch count itself. Bias dims are 1 or dst's (validated).
        if (cDims[s] != 1 && cDims[s] != core.bdim[s]) {
            return Fail(KUDNN_STATUS_BAD_ARGUMENTS,
                        std::string(op) + ": a batch dim of the output is neither 1 nor the operands' batch count");
        }
        if (core.bdim[s] > 1 && cDims[s] == 1) {
            core.serial = true;
        }
    }
    core.A.dt = a.dtype;
    core.A.rows = core.M;
    core.A.s_r = a.strides[nd - 2];
    core.A.s_k = a.strides[nd - 1];
    core.B.dt = b.dtype;
    core.B.rows = core.N;
    core.B.s_r = b.strides[nd - 1];
    core.B.s_k = b.strides[nd - 2];
    core.C.dt = c.dtype;
    core.C.sm = c.strides[nd - 2];
    core.C.sn = c.strides[nd - 1];
    core.C.extent = Extent(c);
    core.hasBias = TotalSizeOpt(bias) != 0;
    if (core.hasBias) {
        core.Bias.dt = bias->dtype;
        core.Bias.sm = bias->strides[nd - 2];
        core.Bias.sn = bias->strides[nd - 1];
        core.Bias.extent = Extent(*bias);
        BatchStrides(*bias, core.Bias.bs, tmp);
    }

    // Fold dense batch dims into M (e.g. X[8][2048][K] x W[1][K][N] -> M = 16384): allowed when the weight
    // is broadcast over the dim and every m-indexed tensor continues row by row across it.
    if (!core.serial) {
        for (int s = 2; s >= 0; --s) {
            const int64_t D = core.bdim[s];
            if (D == 1) {
                continue;
            }
            bool ok = core.B.bs[s] == 0 && core.A.bs[s] == core.M * core.A.s_r && core.C.bs[s] == core.M * core.C.sm &&
                      (!core.hasBias || core.Bias.bs[s] == core.M * core.Bias.sm);
            // every slot inside s must already be folded
            for (int t = s + 1; t < 3; ++t) {
                ok = ok && core.bdim[t] == 1;
            }
            for (TensorSpec *t : extras) {
                ok = ok && (t == nullptr || t->bs[s] == core.M * t->sm);
            }
            if (core.M == 1) {
                ok = false;  // flushed (zero) row strides cannot express the fold
            }
            if (!ok) {
                break;
            }
            core.M *= D;
            core.bdim[s] = 1;
            core.A.bs[s] = core.B.bs[s] = core.C.bs[s] = 0;
            if (core.hasBias) {
                core.Bias.bs[s] = 0;
            }
            for (TensorSpec *t : extras) {
                if (t != nullptr) t->bs[s] = 0;
            }
            core.A.rows = core.M;
        }
    }

    // Operands the MFMA kernels cannot read in place: wrong dtype, not contiguous along K, or rows /
    // batches not aligned to 16-byte chunks.
    const int epc = ElemsPerChunk(core.computeDt);
    const int64_t bk = 128 / DtSize(core.computeDt);  // k-tile: 128 bytes of each row
    const bool lowp16 = core.computeDt == KUDNN_DT_BF16 || core.computeDt == KUDNN_DT_F16;
    // The MFMA kernels need K to be a whole number of k-tiles (a padded pack provides it); the skinny
    // kernel masks its K tail itself.
    const bool kTiles = core.M <= 16 && lowp16 ? true : (core.K % bk == 0);
    auto needsPack = [&](const OperandSpec &o) {
        bool direct = o.dt == core.computeDt && (o.s_k == 1) && (core.K % epc == 0) && (o.s_r % epc == 0) && kTiles;
        for (int s = 0; s < 3; ++s) {
            direct = direct && (o.bs[s] % epc == 0);
        }
        return !direct;
    };
    core.A.staticPack = needsPack(core.A);
    core.B.staticPack = needsPack(core.B);
    if (core.computeDt == KUDNN_DT_S8 && (core.A.dt == KUDNN_DT_U8 || core.B.dt == KUDNN_DT_U8)) {
        // the correction terms are row sums over the packed layout: both operands are packed
        core.A.staticPack = core.B.staticPack = true;
    }
    core.kp = (core.K + bk - 1) / bk * bk;

    // engine and tile configuration
    const int64_t batches = core.Batches();
    if (core.computeDt != KUDNN_DT_F32) {
        if (core.M <= 16 && lowp16) {
            core.engine = ENGINE_SKINNY_BF16;
            // Measured on MI355X at K = 4096 over M = 2..16 and N = 4096..28672 (bench.py --only decode-sweep):
            // - M <= 5: the GEMV with X staged in LDS, ahead of the 16-row MFMA kernel by 1-17 % (M = 4, N = 14336:
            //   20.0 against 22.1 us) and of the K-split GEMV;
            // - M >= 6, one batch, K <= 4096: the K-split GEMV with X in registers (M = 16, N = 14336: 21.7 against
            //   23.8 us; N = 4096: 8.9 against 9.5 us);
            // - otherwise 16-row MFMA tiles.
            // (its operands addressed with 32-bit offsets: the row pitch is the packed one when an operand is packed)
            const int64_t chunks = (core.K + 7) / 8;
            const int64_t lda = core.A.staticPack ? core.kp : core.A.s_r, ldb = core.B.staticPack ? core.kp : core.B.s_r;
            const bool kgemv = batches == 1 && (chunks + 3) / 4 <= 128 &&
                               ((core.N - 1) * ldb + chunks * 8) * 2 < (int64_t(1) << 31) &&
                               ((core.M - 1) * lda + chunks * 8) * 2 < (int64_t(1) << 31);
            core.cfg = core.M == 1 ? KUDNN_CFG_GEMV_BF16
                                   : (core.M <= 5 ? KUDNN_CFG_GEMV_MULTI_BF16
                                                  : (kgemv ? KUDNN_CFG_GEMV_KSPLIT_BF16 : KUDNN_CFG_SKINNY_BF16));
        } else {
            core.engine = ENGINE_MFMA_BF16;
            // Measured on MI355X over prefill-like shapes (M 256..3072, N and K 2048..14336): the ping-pong kernel
            // wins from about 80 tiles of 256 x 256 on, even when they fill only part of the 256 CUs (a partly busy
            // chip runs each CU faster); with fewer tiles it still wins when K is long enough for its tail split
            // (every tile divided over the CUs along K: at most a quarter of the CUs would be busy, at least 128
            // k-tiles, 24 or more per CU; s8 only now, the 16-bit types take K slices there); otherwise the 4-wave
            // 128 x 128 kernel, whose smaller tiles and split-K spread a small grid.
            // Small grids of 16-bit operands split K into slices instead (kudnn_kslice_rule): the ping-pong kernel
            // then runs one workgroup per tile and slice and a second launch adds the slices.
            const int64_t t256 = (core.M + 255) / 256 * ((core.N + 255) / 256) * batches;
            const int64_t kt = core.kp * DtSize(core.computeDt) / 128;
            const bool tailSplit = batches == 1 && t256 <= 64 && kt >= 128 && (t256 * kt + 255) / 256 >= 24;
            const bool slices = kudnn_kslice_rule(core.M, core.N, kt, batches, core.computeDt) >= 2;
            // Except 32-64 tiles with at most 64 k-tiles and the weight stored [N][K]: there the 4-wave kernel's 128-256
            // tiles of 128 x 128 beat two to four K slices (bf16, bench.py --only dispatch: 256 x 11008 x 4096 45 against
            // 55 us, 256 x 14336 x 4096 45 against 58, 1024 x 4096 x 4096 46 against 62, 1024 x 2048 x 2048 26 against
            // 35, 512 x 4096 x 4096 even; 16 tiles and 128 k-tiles stay sliced). A weight stored [K][N] keeps the
            // ping-pong kernel, which reads it in place; the 4-wave kernel would pack it on every call.
            const bool fourWave = batches == 1 && t256 >= 32 && t256 <= 64 && kt <= 64 && core.B.s_r != 1;
            core.cfg = (t256 >= 80 || tailSplit || slices) && !fourWave ? KUDNN_CFG_BF16_PINGPONG_256x256
                                                                        : KUDNN_CFG_BF16_128x128;
        }
    } else {
        core.engine = ENGINE_MFMA_F32;
        // 128 x 128 tiles from one full round of the 256 CUs on, except below 1024 tiles when the last round is at
        // most half full: measured on MI355X over 256..640 tiles at K = 1024..5120, 64 x 64 tiles were 8-17 % faster
        // at 288-384 tiles, within 3 % at 576 and 640, and slower at 256, 400-512
        const int64_t t128 = (core.M + 127) / 128 * ((core.N + 127) / 128) * batches;
        const int64_t lastRound = t128 % 256;
        const bool halfRound = t128 > 256 && t128 < 1024 && lastRound != 0 && lastRound <= 128;
        core.cfg = t128 >= 256 && !halfRound ? KUDNN_CFG_F32_128x128 : KUDNN_CFG_F32_64x64;
        // A grid of fewer than 128 tiles of 64 x 64 (which the 64 x 64 kernel would split along K across workgroups)
        // that still makes at least 128 tiles of 16 x 32: one tile per workgroup, K split over its waves. Measured on
        // MI355X it wins up to K = 4096 (C1, 128 x 1024 x 1024: 8.5 against 12.5 us) and for M <= 16 at any K; beyond,
        // its 16 x 32 tiles read more operand bytes per FLOP than the split 64 x 64 tiles (128 x 1024 x 16384: 86
        // against 68 us).
        const int64_t t64 = (core.M + 63) / 64 * ((core.N + 63) / 64) * batches;
        const int64_t tks = (core.M + 15) / 16 * ((core.N + 31) / 32) * batches;
        if (t64 < KUDNN_SPLIT_MAX_TILES && tks >= 128 && (core.kp <= 4096 || core.M <= 16)) {
            core.cfg = KUDNN_CFG_F32_KSLICE_16x32;
        }
    }
    if (const char *force = std::getenv("KUDNN_HIP_FORCE_CFG")) {
        int f = std::atoi(force);
        // The 4-wave and ping-pong configurations need K in whole k-tiles, which the pack guarantees only when the
        // plan was made for them (M > 16 for 16-bit operands): an override is accepted where it keeps that true.
        const bool mfmaOk = !(core.M <= 16 && lowp16);
        bool okBf16 = core.computeDt != KUDNN_DT_F32 &&
                      (((f == KUDNN_CFG_BF16_256x256 || f == KUDNN_CFG_BF16_256x128 || f == KUDNN_CFG_BF16_128x128 ||
                         f == KUDNN_CFG_BF16_PINGPONG_256x256) && mfmaOk) ||
                       (f == KUDNN_CFG_SKINNY_BF16 && core.M >= 2 && core.M <= 16 && lowp16) ||
                       (f == KUDNN_CFG_GEMV_MULTI_BF16 && core.M >= 2 && core.M <= 8 && lowp16) ||
                       (f == KUDNN_CFG_GEMV_KSPLIT_BF16 && core.M >= 2 && core.M <= 16 && lowp16));
        bool okF32 = core.computeDt == KUDNN_DT_F32 &&
                     (f == KUDNN_CFG_F32_128x128 || f == KUDNN_CFG_F32_64x64 || f == KUDNN_CFG_F32_KSLICE_16x32);
        if (okBf16 || okF32) {
            core.cfg = f;
            const bool skinny = f == KUDNN_CFG_SKINNY_BF16 || f == KUDNN_CFG_GEMV_MULTI_BF16 || f == KUDNN_CFG_GEMV_KSPLIT_BF16;
            core.engine = skinny ? ENGINE_SKINNY_BF16 : (okF32 ? ENGINE_MFMA_F32 : ENGINE_MFMA_BF16);
        }
    }
    // A K-major weight (B stored [K][N], N contiguous: C5's W{1,K,N} ABC) is read in place by the ping-pong kernel,
    // through transposing LDS reads, instead of being packed on every run; it needs 64-deep k-tiles, N a multiple of
    // 8 (whole 16-byte column chunks; an edge tile's columns past N are computed and never stored), 16-byte aligned
    // k-rows and batches, and 32-bit offsets.
    const bool bBatchAligned = core.B.bs[0] % 8 == 0 && core.B.bs[1] % 8 == 0 && core.B.bs[2] % 8 == 0;
    if (core.engine == ENGINE_MFMA_BF16 && core.cfg == KUDNN_CFG_BF16_PINGPONG_256x256 &&
        (core.computeDt == KUDNN_DT_BF16 || core.computeDt == KUDNN_DT_F16) && core.B.dt == core.computeDt &&
        core.B.s_r == 1 && core.B.s_k >= core.N && core.B.s_k % 8 == 0 && bBatchAligned && core.K % 64 == 0 &&
        core.N % 8 == 0 && core.K * core.B.s_k * 2 < (int64_t(1) << 31) &&
        core.M * std::max<int64_t>(core.A.s_r, core.kp) * 2 < (int64_t(1) << 31) && !std::getenv("KUDNN_HIP_PACK_KMAJOR")) {
        core.B.kmajor = true;
        core.B.staticPack = false;
    }
    // The same for an fp32 weight stored [K][N] (the reference's Matmul mode passes W in ABCDE,
    // matmul_gtest.cpp:248-257), read in place by the 4-wave fp32 kernels (128 x 128 and 64 x 64) and by the k-slice
    // kernel's whole-line form (K = 256 c, kudnn_kslice_whole_line): it needs K a multiple of the 32-deep k-tile, N a
    // multiple of 4 (whole 16-byte column chunks), 16-byte aligned k-rows and batches.
    const bool f32InPlaceCfg = core.cfg == KUDNN_CFG_F32_128x128 || core.cfg == KUDNN_CFG_F32_64x64 ||
                               (core.cfg == KUDNN_CFG_F32_KSLICE_16x32 && kudnn_kslice_whole_line(core.K));
    if (core.engine == ENGINE_MFMA_F32 && f32InPlaceCfg &&
        core.B.dt == KUDNN_DT_F32 && core.B.s_r == 1 && core.B.s_k >= core.N && core.B.s_k % 4 == 0 &&
        core.B.bs[0] % 4 == 0 && core.B.bs[1] % 4 == 0 && core.B.bs[2] % 4 == 0 && core.K % 32 == 0 &&
        core.N % 4 == 0 && !std::getenv("KUDNN_HIP_PACK_KMAJOR")) {
        core.B.kmajor = true;
        core.B.staticPack = false;
    }
    return KUDNN_STATUS_SUCCESS;
}

const char *CfgName(int cfg)
{
    switch (cfg) {
        case KUDNN_CFG_BF16_256x256: return "mfma_bf16_256x256";
        case KUDNN_CFG_BF16_256x128: return "mfma_bf16_256x128";
        case KUDNN_CFG_BF16_128x128: return "mfma_bf16_128x128";
        case KUDNN_CFG_BF16_PINGPONG_256x256: return "mfma_bf16_pingpong_256x256";
        case KUDNN_CFG_F32_128x128: return "mfma_f32_128x128";
        case KUDNN_CFG_F32_64x64: return "mfma_f32_64x64";
        case KUDNN_CFG_F32_KSLICE_16x32: return "mfma_f32_kslice_16x32";
        case KUDNN_CFG_SKINNY_BF16: return "skinny_bf16_16xK";
        case KUDNN_CFG_GEMV_BF16: return "skinny_bf16_gemv_row";
        case KUDNN_CFG_GEMV_MULTI_BF16: return "skinny_bf16_gemv_rows_xlds";
        case KUDNN_CFG_GEMV_KSPLIT_BF16: return "skinny_bf16_kgemv_xreg";
        default: return "unknown";
    }
}

std::string DescribeCore(const GemmCore &c)
{
    // the 16- and 8-bit configurations carry the bf16 names; name the operand type actually computed
    std::string cfg = CfgName(c.cfg);
    const char *ct = c.computeDt == KUDNN_DT_F16 ? "f16" : (c.computeDt == KUDNN_DT_S8 ? "s8" : nullptr);
    const size_t at = cfg.find("bf16");
    if (ct != nullptr && at != std::string::npos) {
        cfg.replace(at, 4, ct);
    }
    // the ping-pong kernel's tail split, as the launch would make it on the current device
    char split[96] = "";
    if (c.engine == ENGINE_MFMA_BF16 && c.cfg == KUDNN_CFG_BF16_PINGPONG_256x256) {
        GemmOperands shape{};
        shape.M = c.M;
        shape.N = c.N;
        shape.K = c.kp;
        shape.b_kmajor = c.B.kmajor ? 1 : 0;
        int dp = 0, tail = 0, iters = 0;
        const int slices = kudnn_pingpong_slices(shape, c.Batches(), c.computeDt);
        kudnn_pingpong_split(shape, c.Batches(), c.computeDt, &dp, &tail, &iters);
        const int sliceTail = slices >= 2 ? kudnn_pingpong_slice_tail(shape, c.Batches(), c.computeDt) : 0;
        if (slices >= 2 && sliceTail > 0) {
            std::snprintf(split, sizeof(split), " kslices=%d tail=%d", slices, sliceTail);
        } else if (slices >= 2) {
            std::snprintf(split, sizeof(split), " kslices=%d", slices);
        } else if (tail > 0) {
            std::snprintf(split, sizeof(split), " split=%d+%d/%d", dp, tail, iters);
        }
    }
    char buf[320];
    std::snprintf(buf, sizeof(buf), "%s M=%lld N=%lld K=%lld batches=%lld%s%s%s%s", cfg.c_str(),
                  static_cast<long long>(c.M), static_cast<long long>(c.N), static_cast<long long>(c.K),
                  static_cast<long long>(c.Batches()), c.A.staticPack ? " packA" : "",
                  c.B.staticPack ? " packB" : (c.B.kmajor ? " kmajorB" : ""),
                  c.serial ? " serial" : "", split);
    return buf;
}

bool Aligned(const void *p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// Epilogue extras that are fixed per op (besides C and bias, which come from the core).
struct EpiExtras {
    int act = KUDNN_ACT_UNIMPLEMENTED;
    float actAlpha = 0.0f;
    float actBeta = 0.0f;
    int bin = KUDNN_BINARY_NONE;
    bool storeC = false;  // y is a separate tensor and C must be written too
    bool hasY = false;    // y != C
    TensorSpec Y;         // when hasY
    bool hasSrc = false;
    TensorSpec Src;
};

bool Vec4Ok(const void *p, int dt, const TensorSpec &t, bool needAlign16)
{
    if (t.sn != 1 || t.sm % 4 != 0) {
        return false;
    }
    for (int s = 0; s < 3; ++s) {
        if (t.bs[s] % 4 != 0) {
            return false;
        }
    }
    int align = needAlign16 ? 16 : (dt == KUDNN_DT_BF16 ? 8 : (dt == KUDNN_DT_F32 ? 16 : 2));
    return Aligned(p, align);
}

// Device workspace owned by a plan: packed operands and split-K partial tiles. It grows on demand (hipMalloc, which
// happens on the first runs only) and is used in stream order. A run on another stream than the previous one first
// waits for an event recorded after that run, so overlapping runs of one plan on several streams stay correct
// (they are serialised on the workspace); runs on one stream add no wait. A copy of a plan gets its own workspace.
class Workspace {
public:
    Workspace() = default;
    // Fixed memory (the allocation-free entry point): `fixed` holds `fixedBytes` of workspace and `counters` the
    // split-K arrival counters (zero, and left zero by every split launch). Acquire never allocates, waits or locks;
    // a request beyond fixedBytes is refused.
    Workspace(void *fixed, size_t fixedBytes, uint32_t *counters)
        : fixed_(fixed), fixedBytes_(fixedBytes), fixedCnt_(counters)
    {
    }
    Workspace(const Workspace &) {}
    Workspace &operator=(const Workspace &) { return *this; }
    // Whether this is the fixed memory of the allocation-free entry point, and its size.
    bool Fixed() const { return fixed_ != nullptr; }
    size_t FixedBytes() const { return fixedBytes_; }
    ~Workspace()
    {
        if (ptr_ != nullptr) {
            (void)hipFree(ptr_);  // waits for work that still uses it
        }
        if (cnt_ != nullptr) {
            (void)hipFree(cnt_);
        }
        if (done_ != nullptr) {
            (void)hipEventDestroy(done_);
        }
    }

    // Locks the workspace and returns at least `bytes` of device memory ordered after its previous use, or nullptr
    // with `rc` set. Every successful Acquire is paired with one Release on the same stream. With `counters`, also
    // hands out the split-K arrival counters: a separate buffer of KUDNN_SPLIT_MAX_TILES uint32 that nothing else
    // writes, zeroed on the stream when it is allocated and left zero by every split launch.
    void *Acquire(size_t bytes, hipStream_t stream, int &rc, uint32_t **counters = nullptr)
    {
        rc = KUDNN_STATUS_SUCCESS;
        if (fixed_ != nullptr) {
            if (bytes > fixedBytes_) {
                rc = Fail(KUDNN_STATUS_UNSUPPORTED, "this plan needs " + std::to_string(bytes) +
                                                        " bytes of device workspace; the allocation-free entry point "
                                                        "has " + std::to_string(fixedBytes_));
                return nullptr;
            }
            if (counters != nullptr) {
                *counters = fixedCnt_;
            }
            return fixed_;
        }
        m_.lock();
        if (counters != nullptr) {
            if (cnt_ == nullptr) {
                const size_t cb = KUDNN_SPLIT_MAX_TILES * sizeof(uint32_t);
                hipError_t e = hipMalloc(&cnt_, cb);
                if (e == hipSuccess) {
                    e = hipMemsetAsync(cnt_, 0, cb, stream);
                }
                if (e != hipSuccess) {
                    if (cnt_ != nullptr) {
                        (void)hipFree(cnt_);
                        cnt_ = nullptr;
                    }
                    m_.unlock();
                    rc = Fail(KUDNN_STATUS_ALLOC_FAILED, std::string("split-K counters: ") + hipGetErrorString(e));
                    return nullptr;
                }
            }
            *counters = static_cast<uint32_t *>(cnt_);
        }
        if (bytes > bytes_) {
            if (ptr_ != nullptr) {
                (void)hipFree(ptr_);
                ptr_ = nullptr;
                bytes_ = 0;
            }
            const size_t want = (bytes + (size_t(2) << 20) - 1) / (size_t(2) << 20) * (size_t(2) << 20);
            hipError_t e = hipMalloc(&ptr_, want);
            if (e != hipSuccess) {
                ptr_ = nullptr;
                m_.unlock();
                rc = Fail(KUDNN_STATUS_ALLOC_FAILED, std::string("workspace allocation failed: ") + hipGetErrorString(e));
                return nullptr;
            }
            bytes_ = want;
            used_ = false;  // fresh memory: nothing to wait for
        }
        if (done_ == nullptr) {
            hipError_t e = hipEventCreateWithFlags(&done_, hipEventDisableTiming);
            if (e != hipSuccess) {
                done_ = nullptr;
                m_.unlock();
                rc = HipFail(e, "workspace event");
                return nullptr;
            }
        }
        if (used_ && last_ != stream) {
            hipError_t e = hipStreamWaitEvent(stream, done_, 0);
            if (e != hipSuccess) {
                m_.unlock();
                rc = HipFail(e, "workspace ordering");
                return nullptr;
            }
        }
        return ptr_;
    }

    void Release(hipStream_t stream)
    {
        if (fixed_ != nullptr) {
            return;
        }
        if (hipEventRecord(done_, stream) == hipSuccess) {
            last_ = stream;
            used_ = true;
        } else {
            (void)hipGetLastError();
            (void)hipDeviceSynchronize();  // no event: make the next user safe the slow way
            used_ = false;
        }
        m_.unlock();
    }

private:
    void *fixed_ = nullptr;
    size_t fixedBytes_ = 0;
    uint32_t *fixedCnt_ = nullptr;
    std::mutex m_;
    void *ptr_ = nullptr;
    void *cnt_ = nullptr;
    size_t bytes_ = 0;
    hipEvent_t done_ = nullptr;
    hipStream_t last_ = nullptr;
    bool used_ = false;
};

// Launches one GEMM core. Pointers are device pointers.
int LaunchCore(const GemmCore &core, const EpiExtras &x, const void *a, const void *b, void *c, const void *bias,
               const void *src, void *y, float alpha, float beta, float gamma, Workspace &wsp, hipStream_t stream)
{
    const int es = DtSize(core.computeDt);
    const bool packA = core.A.staticPack || !Aligned(a, 16);
    const bool packB = core.B.staticPack || !Aligned(b, 16);
    const int64_t batches = core.Batches();

    auto allBroadcast = [](const OperandSpec &o) { return o.bs[0] == 0 && o.bs[1] == 0 && o.bs[2] == 0; };
    auto packedBytes = [&](const OperandSpec &o) {
        int64_t copies = allBroadcast(o) ? 1 : batches;
        return copies * o.rows * core.kp * es;
    };
    auto align256 = [](size_t v) { return (v + 255) / 256 * 256; };
    size_t wsA = packA ? align256(static_cast<size_t>(packedBytes(core.A))) : 0;
    size_t wsB = packB ? align256(static_cast<size_t>(packedBytes(core.B))) : 0;

    GemmOperands op{};
    op.M = core.M;
    op.N = core.N;
    // MFMA kernels run whole k-tiles: when K is not a multiple of the tile both operands were packed with
    // zero padding up to kp (and kp == K otherwise). The skinny kernel masks its own K tail.
    op.K = core.engine == ENGINE_SKINNY_BF16 ? core.K : core.kp;
    auto setupOperand = [&](const OperandSpec &o, const void *ptr, bool pack, void *dst, const void *&outPtr,
                            int64_t &ld, int64_t outBs[3]) -> int {
        if (!pack) {
            outPtr = ptr;
            ld = o.kmajor ? o.s_k : o.s_r;  // a K-major B is addressed by its k-row pitch
            for (int s = 0; s < 3; ++s) outBs[s] = o.bs[s];
            return 0;
        }
        PackArgs p{};
        p.src = ptr;
        p.src_dt = o.dt;
        p.rows = o.rows;
        p.cols = core.K;
        p.s_r = o.s_r;
        p.s_k = o.s_k;
        for (int s = 0; s < 3; ++s) {
            p.bdim[s] = core.bdim[s];
            p.bs[s] = o.bs[s];
        }
        p.dst = dst;
        p.dst_dt = core.computeDt;
        p.kp = core.kp;
        p.shift = core.computeDt == KUDNN_DT_S8 && o.dt == KUDNN_DT_U8 ? 128 : 0;
        const bool bc = allBroadcast(o);
        p.dst_bstride = bc ? 0 : o.rows * core.kp;
        int64_t packBatches = bc ? 1 : batches;
        if (bc) {
            p.bdim[0] = p.bdim[1] = p.bdim[2] = 1;
        }
        if (kudnn_launch_pack(p, packBatches, stream) != 0) {
            return -1;
        }
        outPtr = dst;
        ld = core.kp;
        if (bc) {
            outBs[0] = outBs[1] = outBs[2] = 0;
        } else {
            outBs[2] = o.rows * core.kp;
            outBs[1] = core.bdim[2] * outBs[2];
            outBs[0] = core.bdim[1] * outBs[1];
        }
        return 0;
    };
    // workspace: packed A, packed B, split-K partials of the 4-wave kernels
    GemmOperands shape{};
    shape.M = core.M;
    shape.N = core.N;
    shape.K = core.kp;
    const bool mfma4 = core.engine == ENGINE_MFMA_F32 ||
                       (core.engine == ENGINE_MFMA_BF16 && core.cfg != KUDNN_CFG_BF16_PINGPONG_256x256);
    const size_t wsS = mfma4 ? align256(kudnn_gemm_workspace_bytes(shape, batches, core.cfg, core.computeDt)) : 0;
    // the ping-pong kernel's tail split: partial tiles and arrival counters
    const bool pingpong = core.engine == ENGINE_MFMA_BF16 && core.cfg == KUDNN_CFG_BF16_PINGPONG_256x256;
    // K slices write f32 sums of the whole output per slice. The allocation-free entry point runs the same kernels
    // as the allocating one, so a plan whose slices and packs exceed its fixed scratch is refused there (Acquire),
    // never run unsliced: that would change the f32 summation order and so the results.
    const bool slicesOk = true;
    const size_t wsK = pingpong ? align256(kudnn_pingpong_workspace_bytes(shape, batches, core.computeDt, true)) : 0;
    void *ws = nullptr;
    bool acquired = false;
    // u8 operands of an integer GEMM: correction vectors (row sums of the other packed operand, scaled by 128)
    const bool aU8 = core.computeDt == KUDNN_DT_S8 && core.A.dt == KUDNN_DT_U8;
    const bool bU8 = core.computeDt == KUDNN_DT_S8 && core.B.dt == KUDNN_DT_U8;
    const int64_t copiesA = allBroadcast(core.A) ? 1 : batches, copiesB = allBroadcast(core.B) ? 1 : batches;
    const size_t wsCm = bU8 ? align256(static_cast<size_t>(copiesA * core.M) * sizeof(int32_t)) : 0;
    const size_t wsCn = aU8 ? align256(static_cast<size_t>(copiesB * core.N) * sizeof(int32_t)) : 0;
    uint32_t *counters = nullptr;
    if (wsA + wsB + wsS + wsK + wsCm + wsCn > 0) {
        int arc = KUDNN_STATUS_SUCCESS;
        ws = wsp.Acquire(wsA + wsB + wsS + wsK + wsCm + wsCn, stream, arc, wsS > 0 ? &counters : nullptr);
        if (ws == nullptr) {
            return arc;
        }
        acquired = true;
    }
    struct ReleaseGuard {
        Workspace &w;
        hipStream_t s;
        bool on;
        ~ReleaseGuard()
        {
            if (on) w.Release(s);
        }
    } guard{wsp, stream, acquired};
    void *splitWs = wsS > 0 ? static_cast<char *>(ws) + wsA + wsB : nullptr;
    void *tailWs = wsK > 0 ? static_cast<char *>(ws) + wsA + wsB + wsS : nullptr;
    int rc = setupOperand(core.A, a, packA, ws, op.a, op.lda, op.a_bs);
    if (rc == 0) {
        rc = setupOperand(core.B, b, packB, static_cast<char *>(ws) + wsA, op.b, op.ldb, op.b_bs);
        op.b_kmajor = core.B.kmajor && !packB ? 1 : 0;
    }
    if (rc != 0) {
        return HipFail(hipGetLastError(), "pack launch");
    }
    int32_t *corrM = wsCm > 0 ? reinterpret_cast<int32_t *>(static_cast<char *>(ws) + wsA + wsB + wsS + wsK) : nullptr;
    int32_t *corrN = wsCn > 0 ? reinterpret_cast<int32_t *>(static_cast<char *>(ws) + wsA + wsB + wsS + wsK + wsCm)
                              : nullptr;
    if (corrM != nullptr && kudnn_launch_rowsum_s8(static_cast<const int8_t *>(op.a), core.M, core.kp, copiesA,
                                                   copiesA > 1 ? core.M * core.kp : 0, 128u, corrM, stream) != 0) {
        return HipFail(hipGetLastError(), "row-sum launch");
    }
    if (corrN != nullptr && kudnn_launch_rowsum_s8(static_cast<const int8_t *>(op.b), core.N, core.kp, copiesB,
                                                   copiesB > 1 ? core.N * core.kp : 0, 128u, corrN, stream) != 0) {
        return HipFail(hipGetLastError(), "row-sum launch");
    }

    EpiParams ep{};
    ep.alpha = alpha;
    ep.beta = beta;
    ep.act = x.act;
    ep.act_alpha = x.actAlpha;
    ep.act_beta = x.actBeta;
    ep.bin = x.bin;
    ep.gamma = gamma;
    ep.corr_m = corrM;
    ep.corr_n = corrN;
    ep.corr_m_bs = copiesA > 1 ? core.M : 0;
    ep.corr_n_bs = copiesB > 1 ? core.N : 0;
    ep.corr_c = aU8 && bU8 ? static_cast<int32_t>(static_cast<uint32_t>(128u * 128u) * static_cast<uint32_t>(core.K))
                           : 0;
    ep.c_dt = core.C.dt;
    ep.c = c;
    ep.c_sm = core.C.sm;
    ep.c_sn = core.C.sn;
    ep.store_c = x.storeC ? 1 : 0;
    for (int s = 0; s < 3; ++s) {
        ep.bdim[s] = core.bdim[s];
        ep.c_bs[s] = core.C.bs[s];
    }
    if (core.hasBias) {
        ep.bias = bias;
        ep.bias_dt = core.Bias.dt;
        ep.bias_sm = core.Bias.sm;
        ep.bias_sn = core.Bias.sn;
        for (int s = 0; s < 3; ++s) ep.bias_bs[s] = core.Bias.bs[s];
    }
    const TensorSpec &Y = x.hasY ? x.Y : core.C;
    ep.y = x.hasY ? y : c;
    ep.y_dt = Y.dt;
    ep.y_sm = Y.sm;
    ep.y_sn = Y.sn;
    for (int s = 0; s < 3; ++s) ep.y_bs[s] = Y.bs[s];
    if (x.hasSrc) {
        ep.src = src;
        ep.src_dt = x.Src.dt;
        ep.src_sm = x.Src.sm;
        ep.src_sn = x.Src.sn;
        for (int s = 0; s < 3; ++s) ep.src_bs[s] = x.Src.bs[s];
    }
    ep.acc_i32 = core.computeDt == KUDNN_DT_S8 ? 1 : 0;
    bool fast = beta == 0.0f && Vec4Ok(ep.y, Y.dt, Y, false);
    if (!ep.acc_i32 && (!IsFp(Y.dt) || !IsFp(core.C.dt) || (core.hasBias && !IsFp(core.Bias.dt)))) {
        fast = false;  // integer tensors around a float sum take the element-wise epilogue
    }
    if (x.storeC) {
        fast = fast && Vec4Ok(c, core.C.dt, core.C, false);
    }
    if (core.hasBias && core.Bias.sn != 0) {
        fast = fast && (core.Bias.dt != KUDNN_DT_F32 || Vec4Ok(bias, core.Bias.dt, core.Bias, true));
        fast = fast && core.Bias.sn == 1;
    }
    if (x.hasSrc) {
        fast = fast && Vec4Ok(src, x.Src.dt, x.Src, false);
    }
    ep.fast4 = fast ? 1 : 0;
    // 8-wide: 16-byte vector accesses on y / src / bf16 bias, rows and batches 8-element aligned
    auto vec8 = [](const void *p, const TensorSpec &t) {
        if (t.sn != 1 || t.sm % 8 != 0) return false;
        for (int s = 0; s < 3; ++s) {
            if (t.bs[s] % 8 != 0) return false;
        }
        return Aligned(p, 16);
    };
    bool fast8 = fast && vec8(ep.y, Y);
    if (x.hasSrc) {
        fast8 = fast8 && vec8(src, x.Src);
    }
    if (core.hasBias && core.Bias.sn != 0) {
        fast8 = fast8 && vec8(bias, core.Bias);
    }
    ep.fast8 = fast8 ? 1 : 0;

    int lrc = 0;
    if (core.engine == ENGINE_SKINNY_BF16) {
        lrc = kudnn_launch_skinny(op, ep, batches, core.computeDt, core.cfg, stream);
    } else if (core.engine == ENGINE_MFMA_BF16) {
        if (core.cfg == KUDNN_CFG_BF16_PINGPONG_256x256 && kudnn_pingpong_eligible(op, core.computeDt)) {
            lrc = kudnn_launch_gemm_pingpong(op, ep, batches, core.computeDt, tailWs, slicesOk, stream);
        } else if (op.b_kmajor) {
            // only the ping-pong kernel reads a K-major B (the plan's conditions make it eligible)
            return Fail(KUDNN_STATUS_UNSUPPORTED, "GEMM: a K-major weight the ping-pong kernel cannot address");
        } else {
            // operands the ping-pong kernel cannot address (e.g. offsets beyond 2 GiB) use the 4-wave kernel
            // (no split-K workspace was reserved for the ping-pong configuration: runs unsplit)
            const int cfg = core.cfg == KUDNN_CFG_BF16_PINGPONG_256x256 ? KUDNN_CFG_BF16_256x256 : core.cfg;
            lrc = kudnn_launch_gemm_mfma(op, ep, batches, cfg, core.computeDt, splitWs, counters, stream);
        }
    } else if (core.cfg == KUDNN_CFG_F32_KSLICE_16x32 && kudnn_kslice_eligible(op)) {
        lrc = kudnn_launch_gemm_f32_kslice(op, ep, batches, stream);
    } else {
        // (an operand the k-slice kernel cannot address runs on the 64 x 64 kernel, unsplit: no workspace was reserved)
        const int cfg = core.cfg == KUDNN_CFG_F32_KSLICE_16x32 ? KUDNN_CFG_F32_64x64 : core.cfg;
        lrc = kudnn_launch_gemm_f32(op, ep, batches, cfg, cfg == core.cfg ? splitWs : nullptr,
                                    cfg == core.cfg ? counters : nullptr, stream);
    }
    hipError_t le = hipGetLastError();
    if (lrc != 0 || le != hipSuccess) {
        return HipFail(le, "GEMM launch");
    }
    return KUDNN_STATUS_SUCCESS;
}

// Launches `core` over its batch dims in order: one launch per index of the outer `split` dims, each covering the
// inner dims; with split 3, each launch covers `chunk` consecutive indices of the last dim (the reference's batch loop,
// kudnn_gemm.cpp:783-807).
int RunSplit(const GemmCore &core, int split, int64_t chunk, const EpiExtras &x, const void *a, const void *b, void *c,
             const void *bias, const void *src, void *y, float alpha, float beta, float gamma, Workspace &wsp,
             hipStream_t stream)
{
    GemmCore one = core;
    one.serial = false;
    int64_t outer[3] = {1, 1, 1};
    for (int s = 0; s < split; ++s) {
        outer[s] = core.bdim[s];
        one.bdim[s] = 1;
    }
    const int64_t step2 = split == 3 ? chunk : 1;
    for (int64_t i0 = 0; i0 < outer[0]; ++i0) {
        for (int64_t i1 = 0; i1 < outer[1]; ++i1) {
            for (int64_t i2 = 0; i2 < outer[2]; i2 += step2) {
                if (split == 3) {
                    one.bdim[2] = std::min(chunk, outer[2] - i2);
                }
                auto off = [&](const int64_t bs[3], int dt) {
                    return (i0 * bs[0] + i1 * bs[1] + i2 * bs[2]) * DtSize(dt);
                };
                const char *pa = static_cast<const char *>(a) + off(core.A.bs, core.A.dt);
                const char *pb = static_cast<const char *>(b) + off(core.B.bs, core.B.dt);
                char *pc = static_cast<char *>(c) + off(core.C.bs, core.C.dt);
                const char *pbias = core.hasBias ? static_cast<const char *>(bias) + off(core.Bias.bs, core.Bias.dt) : nullptr;
                const char *psrc = x.hasSrc ? static_cast<const char *>(src) + off(x.Src.bs, x.Src.dt) : nullptr;
                char *py = x.hasY ? static_cast<char *>(y) + off(x.Y.bs, x.Y.dt) : nullptr;
                int rc = LaunchCore(one, x, pa, pb, pc, pbias, psrc, py, alpha, beta, gamma, wsp, stream);
                if (rc != KUDNN_STATUS_SUCCESS) {
                    return rc;
                }
            }
        }
    }
    return KUDNN_STATUS_SUCCESS;
}

// Runs a core: batch by batch in order when C is broadcast over a looped batch dim (the reference's sequential batch
// loop, kudnn_gemm.cpp:783-807, then leaves the last batch's result); in several launches over the batch dims when the
// batches exceed what one launch's grid carries (65535 rows of workgroups); otherwise in one launch.
int RunCore(const GemmCore &core, const EpiExtras &x, const void *a, const void *b, void *c, const void *bias,
            const void *src, void *y, float alpha, float beta, float gamma, Workspace &wsp, hipStream_t stream)
{
    constexpr int64_t kMaxGridBatches = 65535;
    if (core.serial) {
        return RunSplit(core, 3, 1, x, a, b, c, bias, src, y, alpha, beta, gamma, wsp, stream);
    }
    if (core.Batches() > kMaxGridBatches) {
        const int split = core.bdim[1] * core.bdim[2] <= kMaxGridBatches ? 1 : (core.bdim[2] <= kMaxGridBatches ? 2 : 3);
        return RunSplit(core, split, kMaxGridBatches, x, a, b, c, bias, src, y, alpha, beta, gamma, wsp, stream);
    }
    return LaunchCore(core, x, a, b, c, bias, src, y, alpha, beta, gamma, wsp, stream);
}

// ---------------------------------------------------------------------------------------------------
// host-pointer staging

bool IsDevicePtr(const void *p)
{
    if (p == nullptr) {
        return true;
    }
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

// Device copies of host buffers for one call; outputs are copied back by Finish().
struct Staging {
    struct Buf {
        void *host;
        void *dev;
        size_t bytes;
        bool output;
    };
    Buf bufs[8];
    int n = 0;
    bool any = false;
    hipStream_t stream = nullptr;

    // Returns the pointer to use on the device (the original if it already is device memory).
    int Add(const void *host, size_t bytes, bool input, bool output, void **devOut)
    {
        *devOut = const_cast<void *>(host);
        if (host == nullptr || bytes == 0 || IsDevicePtr(host)) {
            return KUDNN_STATUS_SUCCESS;
        }
        any = true;
        void *d = nullptr;
        hipError_t e = hipMalloc(&d, bytes);
        if (e != hipSuccess) {
            return Fail(KUDNN_STATUS_ALLOC_FAILED, std::string("staging allocation failed: ") + hipGetErrorString(e));
        }
        bufs[n++] = Buf{const_cast<void *>(host), d, bytes, output};
        if (input) {
            e = hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, stream);
            if (e != hipSuccess) {
                return HipFail(e, "staging copy");
            }
        }
        *devOut = d;
        return KUDNN_STATUS_SUCCESS;
    }
    int Finish(int status)
    {
        if (any) {
            for (int i = 0; i < n && status == KUDNN_STATUS_SUCCESS; ++i) {
                if (bufs[i].output) {
                    hipError_t e = hipMemcpyAsync(bufs[i].host, bufs[i].dev, bufs[i].bytes, hipMemcpyDeviceToHost, stream);
                    if (e != hipSuccess) {
                        status = HipFail(e, "staging copy back");
                    }
                }
            }
            hipError_t e = hipStreamSynchronize(stream);
            if (e != hipSuccess && status == KUDNN_STATUS_SUCCESS) {
                status = HipFail(e, "stream synchronize");
            }
        }
        for (int i = 0; i < n; ++i) {
            (void)hipFree(bufs[i].dev);
        }
        n = 0;
        return status;
    }
};

int CopyDesc(const kudnn_tensor_desc *in, kudnn_tensor_desc &out)
{
    if (IsNone(in)) {
        std::memset(&out, 0, sizeof(out));
        return 0;
    }
    out = *in;
    return 0;
}

// ---------------------------------------------------------------------------------------------------
// plan objects

enum PlanKind { PLAN_GEMM = 1, PLAN_LINEAR_ACT, PLAN_LINEAR_RES, PLAN_LINEAR_POSTOPS };

struct PlanBase {
    int kind;
    std::string desc;
    explicit PlanBase(int k) : kind(k) {}
    virtual ~PlanBase() = default;
};

int64_t DescExtentBytes(const kudnn_tensor_desc &d) { return Extent(d) * DtSize(d.dtype); }

}  // namespace

struct kudnn_gemm_plan : PlanBase {
    kudnn_gemm_plan() : PlanBase(PLAN_GEMM) {}
    kudnn_tensor_desc a{}, b{}, c{}, bias{};
    GemmCore core;
    mutable Workspace ws;
};

struct kudnn_linear_act_plan : PlanBase {
    kudnn_linear_act_plan() : PlanBase(PLAN_LINEAR_ACT) {}
    kudnn_tensor_desc a{}, b{}, c{}, bias{};
    GemmCore core;
    EpiExtras x;
    mutable Workspace ws;
};

struct kudnn_linear_res_plan : PlanBase {
    kudnn_linear_res_plan() : PlanBase(PLAN_LINEAR_RES) {}
    kudnn_tensor_desc a{}, b{}, c{}, bias{}, res{}, lr{};
    int resKind = 0;
    GemmCore core;
    GemmCore mul;   // RES_MUL: linearRes = C x res
    EpiExtras x;
    mutable Workspace ws;
};

struct kudnn_linear_postops_plan : PlanBase {
    kudnn_linear_postops_plan() : PlanBase(PLAN_LINEAR_POSTOPS) {}
    kudnn_tensor_desc a{}, b{}, y{}, bias{}, src{};
    GemmCore core;
    EpiExtras x;
    mutable Workspace ws;
};

namespace {

TensorSpec SpecOf(const kudnn_tensor_desc &d)
{
    TensorSpec t;
    t.dt = d.dtype;
    t.sm = d.strides[d.ndims - 2];
    t.sn = d.strides[d.ndims - 1];
    int64_t dims[3];
    BatchStrides(d, t.bs, dims);
    t.extent = Extent(d);
    return t;
}


}  // namespace

// =====================================================================================================
// device scratch of the allocation-free entry point (kudnn_linear_postops_run_noalloc)

namespace {

// Layout: the split-K arrival counters (KUDNN_SPLIT_MAX_TILES uint32, padded to 512 bytes), then the workspace.
constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr size_t kScratchCounterBytes = 512;
static_assert(KUDNN_SPLIT_MAX_TILES * sizeof(uint32_t) <= kScratchCounterBytes, "counter region");

}  // namespace

// One copy per GPU, zero when the code object is loaded, held until the process ends. In host code `scratch` is
// only the runtime's handle for the symbol: its device address comes from hipGetSymbolAddress (ScratchOf).
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// The device address of `scratch` on the current device, looked up once per device (with that device current).
void *ScratchOf(int &rc)
{
    static std::atomic<void *> addr[64] = {};
    rc = KUDNN_STATUS_SUCCESS;
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) {
        rc = e != hipSuccess ? HipFail(e, "hipGetDevice") : Fail(KUDNN_STATUS_INTERNAL, "device index out of range");
        return nullptr;
    }
    void *p = addr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            rc = HipFail(e, "hipGetSymbolAddress(scratch)");
            return nullptr;
        }
        addr[dev].store(p, std::memory_order_release);
    }
    return p;
}

}  // namespace

// =====================================================================================================
// exported C ABI

extern "C" {

const char *kudnn_last_error(void) { return g_lastError.c_str(); }

const char *kudnn_version(void) { return "kudnn-mi355x 0.1.0 (gfx950)"; }

int kudnn_stream_synchronize(void *stream)
{
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? KUDNN_STATUS_SUCCESS : HipFail(e, "hipStreamSynchronize");
}

int kudnn_tensor_desc_init(kudnn_tensor_desc *desc, int32_t ndims, const int64_t *dims, int32_t dtype, int32_t layout)
{
    if (desc == nullptr || (ndims > 0 && dims == nullptr)) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "Tensor Info: null descriptor or dims");
    }
    std::memset(desc, 0, sizeof(*desc));
    if (dtype <= KUDNN_DT_UNDEFINED || dtype > KUDNN_DT_U8) {
        return Fail(KUDNN_STATUS_BAD_ARGUMENTS, "Tensor Info: Undefined data type of tensor");
    }
    if (ndims < 1 || ndims > KUDNN_HIP_MAX_DIMS) {
        return Fail(KUDNN_STATUS_BAD_ARGUMENTS, "Tensor Info: tensor dimensionality is incorrect");
    }
    if (!kudnn_layout::IsValidFor(layout, ndims)) {
        return Fail(KUDNN_STATUS_BAD_ARGUMENTS, "Tensor Info: incorrect layout for " + std::to_string(ndims) + "D tensor");
    }
    for (int i = 0; i < ndims; ++i) {
        if (dims[i] < 0) {
            return Fail(KUDNN_STATUS_BAD_ARGUMENTS, "Shape: negative dimension");
        }
    }
    desc->ndims = ndims;
    desc->dtype = dtype;
    desc->layout = layout;
    for (int i = 0; i < ndims; ++i) {
        desc->dims[i] = dims[i];
    }
    kudnn_layout::MinStrides(layout, ndims, desc->dims, desc->strides);
    return KUDNN_STATUS_SUCCESS;
}

int kudnn_tensor_desc_init_strided(kudnn_tensor_desc *desc, int32_t ndims, const int64_t *dims, int32_t dtype,
                                   int32_t layout, const int64_t *strides)
{
    if (strides == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "Tensor Info: null strides");
    }
    int s = kudnn_tensor_desc_init(desc, ndims, dims, dtype, layout);
    if (s != KUDNN_STATUS_SUCCESS) {
        return s;
    }
    int64_t mins[KUDNN_HIP_MAX_DIMS];
    for (int i = 0; i < ndims; ++i) {
        mins[i] = desc->strides[i];
    }
    for (int i = 0; i < ndims; ++i) {
        if (strides[i] < mins[i]) {
            std::memset(desc, 0, sizeof(*desc));
            return Fail(KUDNN_STATUS_BAD_ARGUMENTS, "Tensor Info: incorrect strides");
        }
        desc->strides[i] = (dims[i] == 1) ? 0 : strides[i];
    }
    return KUDNN_STATUS_SUCCESS;
}

int kudnn_tensor_desc_is_dense(const kudnn_tensor_desc *desc) { return desc != nullptr && DescIsDense(*desc) ? 1 : 0; }

// threading --------------------------------------------------------------------------------------------

int kudnn_threading_get_max_num_threads(void) { return MaxThreads(); }

int kudnn_threading_set_max_num_threads(int n)
{
    int old = Thr().maxThreads;
    if (n > 0 && n <= Thr().available) {
        Thr().maxThreads = n;
        Thr().control = 1;
    }
    return old;
}

int kudnn_threading_set_fixed_num_threads(int n)
{
    int old = Thr().fixedThreads;
    if (n > 0 && n <= Thr().available) {
        Thr().fixed = true;
        Thr().fixedThreads = n;
        Thr().control = 1;
    }
    return old;
}

int kudnn_threading_set_num_threads_local(int n)
{
    int old = g_localThreads;
    if (n >= 1 && n <= Thr().available) {
        g_localThreads = n;
        Thr().control = 1;
    }
    return old;
}

int kudnn_threading_should_calculate_opt_threads(void) { return Thr().fixed ? 0 : 1; }

int kudnn_threading_set_env_mode(int mode)
{
    Thr().envMode = mode;
    return Thr().envMode;
}

int kudnn_threading_get_control_status(void) { return Thr().control; }

// Gemm ------------------------------------------------------------------------------------------------

int kudnn_gemm_validate(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b, const kudnn_tensor_desc *c,
                        const kudnn_tensor_desc *bias, int num_threads)
{
    if (a == nullptr || b == nullptr || c == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "GEMM: null descriptor");
    }
    return ValidateGemm(*a, *b, *c, bias, num_threads);
}

int kudnn_gemm_create(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b, const kudnn_tensor_desc *c,
                      const kudnn_tensor_desc *bias, int num_threads, kudnn_gemm_t *plan)
{
    if (plan == nullptr || a == nullptr || b == nullptr || c == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "GEMM: null argument");
    }
    *plan = nullptr;
    int s = ValidateGemm(*a, *b, *c, bias, num_threads);
    if (s != KUDNN_STATUS_SUCCESS) {
        return FailStatus(s, "GEMM");
    }
    auto *p = new (std::nothrow) kudnn_gemm_plan();
    if (p == nullptr) {
        return Fail(KUDNN_STATUS_ALLOC_FAILED, "GEMM: plan allocation failed");
    }
    p->a = *a;
    p->b = *b;
    p->c = *c;
    CopyDesc(bias, p->bias);
    s = BuildCore(*a, *b, *c, &p->bias, p->core, "GEMM");
    if (s != KUDNN_STATUS_SUCCESS) {
        delete p;
        return s;
    }
    p->desc = DescribeCore(p->core);
    *plan = p;
    return KUDNN_STATUS_SUCCESS;
}

int kudnn_gemm_run(kudnn_gemm_t plan, const void *a, const void *b, void *c, const void *bias, float alpha, float beta,
                   int num_threads, void *stream)
{
    if (plan == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "GEMM: null plan");
    }
    if (a == nullptr || b == nullptr || c == nullptr || (plan->core.hasBias && bias == nullptr)) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "Matmul Layer: one of input matrices is nullptr");
    }
    if (!plan->core.hasBias && bias != nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "Matmul Layer: bias isn't nullptr, but bias TensorInfo has 0 total size");
    }
    if (num_threads < 0 || num_threads > MaxThreads()) {
        return FailStatus(KUDNN_STATUS_BAD_ARGUMENTS, "GEMM");
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const GemmCore &core = plan->core;
    if (core.computeDt == KUDNN_DT_S8 && (alpha != 1.0f || beta != 0.0f)) {
        // cblas_gemm_s8s8s32's scaling of an int32 result by float alpha / beta is KML-internal and unpinned
        return Fail(KUDNN_STATUS_UNSUPPORTED, "GEMM: s8 x s8 -> s32 runs with alpha = 1 and beta = 0 only");
    }
    // cblas_bgemm takes bf16 alpha/beta when a bf16 C has no bias (kudnn_gemm.cpp:222-226).
    if (core.bf16Scalars) {
        alpha = RoundBf16(alpha);
        beta = RoundBf16(beta);
    }
    Staging stg;
    stg.stream = st;
    void *da, *db, *dc, *dbias;
    int rc = stg.Add(a, DescExtentBytes(plan->a), true, false, &da);
    if (rc == 0) rc = stg.Add(b, DescExtentBytes(plan->b), true, false, &db);
    if (rc == 0) rc = stg.Add(c, DescExtentBytes(plan->c), beta != 0.0f, true, &dc);
    if (rc == 0) rc = stg.Add(bias, plan->core.hasBias ? DescExtentBytes(plan->bias) : 0, true, false, &dbias);
    if (rc == 0) {
        EpiExtras x;
        rc = RunCore(core, x, da, db, dc, dbias, nullptr, nullptr, alpha, beta, 0.0f, plan->ws, st);
    }
    return stg.Finish(rc);
}

int kudnn_gemm_clone(kudnn_gemm_t plan, kudnn_gemm_t *copy)
{
    if (plan == nullptr || copy == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "GEMM: null plan");
    }
    *copy = new (std::nothrow) kudnn_gemm_plan(*plan);
    return *copy ? KUDNN_STATUS_SUCCESS : Fail(KUDNN_STATUS_ALLOC_FAILED, "GEMM: plan allocation failed");
}

int kudnn_gemm_destroy(kudnn_gemm_t plan)
{
    delete plan;
    return KUDNN_STATUS_SUCCESS;
}

// LinearActivationLayerFWD ---------------------------------------------------------------------------------

int kudnn_linear_act_validate(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b, const kudnn_tensor_desc *c,
                              const kudnn_tensor_desc *bias, float alpha, float beta, int kind, int num_threads)
{
    if (a == nullptr || b == nullptr || c == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearActivationLayerFWD: null descriptor");
    }
    int s = ValidateGemm(*a, *b, *c, bias, num_threads);
    if (s != KUDNN_STATUS_SUCCESS) {
        return s;
    }
    return ValidateActivation(*c, kind, alpha, beta);
}

int kudnn_linear_act_create(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b, const kudnn_tensor_desc *c,
                            const kudnn_tensor_desc *bias, float alpha, float beta, int kind, int num_threads,
                            kudnn_linear_act_t *plan)
{
    if (plan == nullptr || a == nullptr || b == nullptr || c == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearActivationLayerFWD: null argument");
    }
    *plan = nullptr;
    // Same order of checks as the reference constructor (kudnn_linear_activationlayer.cpp:30-38): the Gemm member,
    // then the activation member, which is built as activationlayerfwd(cInfo, cInfo, kind, alpha) and so validates
    // with its default second parameter 0, then the layer's own ValidateInput with the caller's beta.
    int s = ValidateGemm(*a, *b, *c, bias, num_threads);
    if (s != KUDNN_STATUS_SUCCESS) {
        return FailStatus(s, "GEMM");
    }
    s = ValidateActivation(*c, kind, alpha, 0.0f);
    if (s != KUDNN_STATUS_SUCCESS) {
        return FailStatus(s, "Activation layer");
    }
    s = ValidateActivation(*c, kind, alpha, beta);
    if (s != KUDNN_STATUS_SUCCESS) {
        return FailStatus(s, "LinearActivationLayerFWD");
    }
    if (!ActImplemented(kind)) {
        return Fail(KUDNN_STATUS_UNSUPPORTED,
                    "LinearActivationLayerFWD: activation kind " + std::to_string(kind) +
                        " is not a forward activation kind");
    }
    auto *p = new (std::nothrow) kudnn_linear_act_plan();
    if (p == nullptr) {
        return Fail(KUDNN_STATUS_ALLOC_FAILED, "LinearActivationLayerFWD: plan allocation failed");
    }
    p->a = *a;
    p->b = *b;
    p->c = *c;
    CopyDesc(bias, p->bias);
    s = BuildCore(*a, *b, *c, &p->bias, p->core, "LinearActivationLayerFWD");
    if (s == KUDNN_STATUS_SUCCESS && (p->core.computeDt == KUDNN_DT_S8 || !IsFp(c->dtype))) {
        // the reference activates an integer C through ReorderLayer's f32 round trip (kudnn_eltwise.cpp:511-585)
        s = Fail(KUDNN_STATUS_UNSUPPORTED, "LinearActivationLayerFWD: integer GEMMs and outputs run through Gemm only");
    }
    if (s != KUDNN_STATUS_SUCCESS) {
        delete p;
        return s;
    }
    // the layer's beta never reaches the activation (kudnn_linear_activationlayer.cpp:33): it runs with 0
    p->x.act = kind;
    p->x.actAlpha = alpha;
    p->x.actBeta = 0.0f;
    p->desc = DescribeCore(p->core) + " act=" + std::to_string(kind);
    *plan = p;
    return KUDNN_STATUS_SUCCESS;
}

int kudnn_linear_act_run(kudnn_linear_act_t plan, const void *a, const void *b, void *c, const void *bias,
                         int num_threads, void *stream)
{
    if (plan == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearActivationLayerFWD: null plan");
    }
    if (a == nullptr || b == nullptr || c == nullptr || (plan->core.hasBias && bias == nullptr)) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "Matmul Layer: one of input matrices is nullptr");
    }
    if (!plan->core.hasBias && bias != nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "Matmul Layer: bias isn't nullptr, but bias TensorInfo has 0 total size");
    }
    if (num_threads < 0 || num_threads > MaxThreads()) {
        return FailStatus(KUDNN_STATUS_BAD_ARGUMENTS, "GEMM");
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    Staging stg;
    stg.stream = st;
    void *da, *db, *dc, *dbias;
    int rc = stg.Add(a, DescExtentBytes(plan->a), true, false, &da);
    if (rc == 0) rc = stg.Add(b, DescExtentBytes(plan->b), true, false, &db);
    if (rc == 0) rc = stg.Add(c, DescExtentBytes(plan->c), false, true, &dc);
    if (rc == 0) rc = stg.Add(bias, plan->core.hasBias ? DescExtentBytes(plan->bias) : 0, true, false, &dbias);
    if (rc == 0) {
        rc = RunCore(plan->core, plan->x, da, db, dc, dbias, nullptr, nullptr, 1.0f, 0.0f, 0.0f, plan->ws, st);
    }
    return stg.Finish(rc);
}

int kudnn_linear_act_clone(kudnn_linear_act_t plan, kudnn_linear_act_t *copy)
{
    if (plan == nullptr || copy == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearActivationLayerFWD: null plan");
    }
    *copy = new (std::nothrow) kudnn_linear_act_plan(*plan);
    return *copy ? KUDNN_STATUS_SUCCESS : Fail(KUDNN_STATUS_ALLOC_FAILED, "plan allocation failed");
}

int kudnn_linear_act_destroy(kudnn_linear_act_t plan)
{
    delete plan;
    return KUDNN_STATUS_SUCCESS;
}

// LinearResFWD ------------------------------------------------------------------------------------------------

int kudnn_linear_res_validate(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b, const kudnn_tensor_desc *c,
                              const kudnn_tensor_desc *bias, const kudnn_tensor_desc *res,
                              const kudnn_tensor_desc *linear_res, int kind, int num_threads)
{
    if (a == nullptr || b == nullptr || c == nullptr || res == nullptr || linear_res == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearResFWD: null descriptor");
    }
    return ValidateRes(*a, *b, *c, bias, *res, *linear_res, kind, num_threads);
}

int kudnn_linear_res_create(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b, const kudnn_tensor_desc *c,
                            const kudnn_tensor_desc *bias, const kudnn_tensor_desc *res,
                            const kudnn_tensor_desc *linear_res, float alpha, float beta, float gamma, int kind,
                            int num_threads, kudnn_linear_res_t *plan)
{
    (void)alpha;
    (void)beta;
    (void)gamma;
    if (plan == nullptr || a == nullptr || b == nullptr || c == nullptr || res == nullptr || linear_res == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearResFWD: null argument");
    }
    *plan = nullptr;
    int s = ValidateGemm(*a, *b, *c, bias, num_threads);
    if (s != KUDNN_STATUS_SUCCESS) {
        return FailStatus(s, "GEMM");
    }
    s = ValidateRes(*a, *b, *c, bias, *res, *linear_res, kind, num_threads);
    if (s != KUDNN_STATUS_SUCCESS) {
        return FailStatus(s, "LinearResFWD");
    }
    auto *p = new (std::nothrow) kudnn_linear_res_plan();
    if (p == nullptr) {
        return Fail(KUDNN_STATUS_ALLOC_FAILED, "LinearResFWD: plan allocation failed");
    }
    p->a = *a;
    p->b = *b;
    p->c = *c;
    CopyDesc(bias, p->bias);
    p->res = *res;
    p->lr = *linear_res;
    p->resKind = kind;
    if (kind != KUDNN_RES_MUL) {
        p->x.Y = SpecOf(*linear_res);
        p->x.Src = SpecOf(*linear_res);   // res is read in linearRes's memory order
        p->x.Src.dt = res->dtype;
        s = BuildCore(*a, *b, *c, &p->bias, p->core, "LinearResFWD", &p->x.Y, &p->x.Src);
    } else {
        s = BuildCore(*a, *b, *c, &p->bias, p->core, "LinearResFWD");
    }
    // AddOps reads C, res and linearRes as f16, bf16 or f32 (kudnn_linear_res.cpp:57-122, 192-200)
    if (s == KUDNN_STATUS_SUCCESS &&
        (p->core.computeDt == KUDNN_DT_S8 || !IsFp(c->dtype) || !IsFp(res->dtype) || !IsFp(linear_res->dtype))) {
        s = Fail(KUDNN_STATUS_UNSUPPORTED, "LinearResFWD: integer GEMMs and outputs run through Gemm only");
    }
    if (s == KUDNN_STATUS_SUCCESS && kind == KUDNN_RES_MUL) {
        kudnn_tensor_desc none{};
        s = BuildCore(*c, *res, *linear_res, &none, p->mul, "LinearResFWD");
        p->desc = DescribeCore(p->core) + " | res_mul " + DescribeCore(p->mul);
    } else if (s == KUDNN_STATUS_SUCCESS) {
        // AddOps walks C, res and linearRes as flat arrays of linearRes's size (kudnn_linear_res.cpp:57-75):
        // element i of each is added. The fused epilogue computes C at logical (m, n); it matches the flat
        // walk when C and linearRes share dims and layout, which is what is supported here.
        const kudnn_tensor_desc &cc = *c, &lr = *linear_res, &rr = *res;
        bool same = cc.ndims == lr.ndims && cc.layout == lr.layout && cc.dtype == lr.dtype && rr.dtype == lr.dtype &&
                    DescIsDense(lr);
        for (int i = 0; same && i < cc.ndims; ++i) {
            same = cc.dims[i] == lr.dims[i] && cc.dims[i] == rr.dims[i];
        }
        if (!same) {
            s = Fail(KUDNN_STATUS_UNSUPPORTED,
                     "LinearResFWD: C, res and linearRes must share dims, layout and dtype on the fused path");
        } else {
            p->x.bin = (kind == KUDNN_RES_EXT) ? KUDNN_BINARY_EXT : KUDNN_BINARY_ADD;
            p->x.storeC = true;
            p->x.hasY = true;
            p->x.hasSrc = true;
            p->desc = DescribeCore(p->core) + (kind == KUDNN_RES_EXT ? " res_ext" : " res_add");
        }
    }
    if (s != KUDNN_STATUS_SUCCESS) {
        delete p;
        return s;
    }
    *plan = p;
    return KUDNN_STATUS_SUCCESS;
}

int kudnn_linear_res_run(kudnn_linear_res_t plan, const void *a, const void *b, void *c, const void *bias,
                         const void *res, void *linear_res, float gamma, int num_threads, void *stream)
{
    if (plan == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearResFWD: null plan");
    }
    if (a == nullptr || b == nullptr || c == nullptr || (plan->core.hasBias && bias == nullptr)) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "Matmul Layer: one of input matrices is nullptr");
    }
    if (!plan->core.hasBias && bias != nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "Matmul Layer: bias isn't nullptr, but bias TensorInfo has 0 total size");
    }
    if (res == nullptr || linear_res == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearResFWD: res or linearRes is nullptr");
    }
    if (num_threads < 0 || num_threads > MaxThreads()) {
        return FailStatus(KUDNN_STATUS_BAD_ARGUMENTS, "GEMM");
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    Staging stg;
    stg.stream = st;
    void *da, *db, *dc, *dbias, *dres, *dlr;
    const bool mul = plan->resKind == KUDNN_RES_MUL;
    int rc = stg.Add(a, DescExtentBytes(plan->a), true, false, &da);
    if (rc == 0) rc = stg.Add(b, DescExtentBytes(plan->b), true, false, &db);
    if (rc == 0) rc = stg.Add(c, DescExtentBytes(plan->c), false, true, &dc);
    if (rc == 0) rc = stg.Add(bias, plan->core.hasBias ? DescExtentBytes(plan->bias) : 0, true, false, &dbias);
    const size_t resBytes = mul ? static_cast<size_t>(DescExtentBytes(plan->res))
                                : static_cast<size_t>(Extent(plan->lr)) * DtSize(plan->res.dtype);
    if (rc == 0) rc = stg.Add(res, resBytes, true, false, &dres);
    if (rc == 0) rc = stg.Add(linear_res, DescExtentBytes(plan->lr), false, true, &dlr);
    if (rc == 0) {
        if (mul) {
            EpiExtras none;
            rc = RunCore(plan->core, none, da, db, dc, dbias, nullptr, nullptr, 1.0f, 0.0f, 0.0f, plan->ws, st);
            if (rc == 0) {
                float one = 1.0f, zero = 0.0f;
                rc = RunCore(plan->mul, none, dc, dres, dlr, nullptr, nullptr, nullptr, one, zero, 0.0f, plan->ws, st);
            }
        } else {
            rc = RunCore(plan->core, plan->x, da, db, dc, dbias, dres, dlr, 1.0f, 0.0f, gamma, plan->ws, st);
        }
    }
    return stg.Finish(rc);
}

int kudnn_linear_res_clone(kudnn_linear_res_t plan, kudnn_linear_res_t *copy)
{
    if (plan == nullptr || copy == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearResFWD: null plan");
    }
    *copy = new (std::nothrow) kudnn_linear_res_plan(*plan);
    return *copy ? KUDNN_STATUS_SUCCESS : Fail(KUDNN_STATUS_ALLOC_FAILED, "plan allocation failed");
}

int kudnn_linear_res_destroy(kudnn_linear_res_t plan)
{
    delete plan;
    return KUDNN_STATUS_SUCCESS;
}

// Linear + post-op chain -------------------------------------------------------------------------------

int kudnn_linear_postops_create(const kudnn_tensor_desc *a, const kudnn_tensor_desc *b, const kudnn_tensor_desc *y,
                                const kudnn_tensor_desc *bias, int act_kind, float act_alpha, float act_beta,
                                int binary_kind, const kudnn_tensor_desc *src, float gamma, int num_threads,
                                kudnn_linear_postops_t *plan)
{
    (void)gamma;
    if (plan == nullptr || a == nullptr || b == nullptr || y == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearPostOpsFWD: null argument");
    }
    *plan = nullptr;
    int s = ValidateGemm(*a, *b, *y, bias, num_threads);
    if (s != KUDNN_STATUS_SUCCESS) {
        return FailStatus(s, "GEMM");
    }
    if (act_kind != KUDNN_ACT_UNIMPLEMENTED) {
        s = ValidateActivation(*y, act_kind, act_alpha, act_beta);
        if (s != KUDNN_STATUS_SUCCESS) {
            return FailStatus(s, "Activation layer");
        }
        if (!ActImplemented(act_kind)) {
            return Fail(KUDNN_STATUS_UNSUPPORTED, "LinearPostOpsFWD: activation kind not implemented as an epilogue");
        }
    }
    if (binary_kind < KUDNN_BINARY_NONE || binary_kind > KUDNN_BINARY_MUL) {
        return FailStatus(KUDNN_STATUS_UNSUPPORTED, "LinearPostOpsFWD");
    }
    if (binary_kind != KUDNN_BINARY_NONE) {
        if (IsNone(src) || src->ndims != y->ndims || !IsFp(src->dtype)) {
            return FailStatus(KUDNN_STATUS_BAD_ARGUMENTS, "LinearPostOpsFWD");
        }
        for (int i = 0; i < y->ndims; ++i) {
            if (src->dims[i] != y->dims[i]) {
                return FailStatus(KUDNN_STATUS_BAD_ARGUMENTS, "LinearPostOpsFWD");
            }
        }
    }
    auto *p = new (std::nothrow) kudnn_linear_postops_plan();
    if (p == nullptr) {
        return Fail(KUDNN_STATUS_ALLOC_FAILED, "LinearPostOpsFWD: plan allocation failed");
    }
    p->a = *a;
    p->b = *b;
    p->y = *y;
    CopyDesc(bias, p->bias);
    CopyDesc(src, p->src);
    if (binary_kind != KUDNN_BINARY_NONE) {
        p->x.hasSrc = true;
        p->x.Src = SpecOf(*src);
    }
    s = BuildCore(*a, *b, *y, &p->bias, p->core, "LinearPostOpsFWD", p->x.hasSrc ? &p->x.Src : nullptr);
    if (s == KUDNN_STATUS_SUCCESS && !IsFp(y->dtype) && (act_kind != KUDNN_ACT_UNIMPLEMENTED || p->x.hasSrc)) {
        s = Fail(KUDNN_STATUS_UNSUPPORTED, "LinearPostOpsFWD: a Linear into an integer output takes no activation or "
                                           "binary operand");
    }
    if (s != KUDNN_STATUS_SUCCESS) {
        delete p;
        return s;
    }
    p->x.act = act_kind;
    p->x.actAlpha = act_alpha;
    p->x.actBeta = act_beta;
    p->x.bin = binary_kind;
    p->desc = DescribeCore(p->core) + " act=" + std::to_string(act_kind) + " bin=" + std::to_string(binary_kind);
    *plan = p;
    return KUDNN_STATUS_SUCCESS;
}

int kudnn_linear_postops_run(kudnn_linear_postops_t plan, const void *a, const void *b, void *y, const void *bias,
                             const void *src, float gamma, void *stream)
{
    if (plan == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearPostOpsFWD: null plan");
    }
    if (a == nullptr || b == nullptr || y == nullptr || (plan->core.hasBias && bias == nullptr) ||
        (plan->x.hasSrc && src == nullptr)) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearPostOpsFWD: one of input matrices is nullptr");
    }
    if (!plan->core.hasBias && bias != nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearPostOpsFWD: bias isn't nullptr, but bias TensorInfo has 0 total size");
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    Staging stg;
    stg.stream = st;
    void *da, *db, *dy, *dbias, *dsrc;
    int rc = stg.Add(a, DescExtentBytes(plan->a), true, false, &da);
    if (rc == 0) rc = stg.Add(b, DescExtentBytes(plan->b), true, false, &db);
    if (rc == 0) rc = stg.Add(y, DescExtentBytes(plan->y), false, true, &dy);
    if (rc == 0) rc = stg.Add(bias, plan->core.hasBias ? DescExtentBytes(plan->bias) : 0, true, false, &dbias);
    if (rc == 0) rc = stg.Add(src, plan->x.hasSrc ? DescExtentBytes(plan->src) : 0, true, false, &dsrc);
    if (rc == 0) {
        rc = RunCore(plan->core, plan->x, da, db, dy, dbias, dsrc, nullptr, 1.0f, 0.0f, gamma, plan->ws, st);
    }
    return stg.Finish(rc);
}

int kudnn_linear_postops_run_noalloc(kudnn_linear_postops_t plan, const void *a, const void *b, void *y,
                                     const void *bias, const void *src, float gamma, void *stream)
{
    if (plan == nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearPostOpsFWD: null plan");
    }
    if (a == nullptr || b == nullptr || y == nullptr || (plan->core.hasBias && bias == nullptr) ||
        (plan->x.hasSrc && src == nullptr)) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearPostOpsFWD: one of input matrices is nullptr");
    }
    if (!plan->core.hasBias && bias != nullptr) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "LinearPostOpsFWD: bias isn't nullptr, but bias TensorInfo has 0 total size");
    }
    // host buffers would need staging copies in allocated device memory
    for (const void *p : {a, b, static_cast<const void *>(y), bias, src}) {
        if (!IsDevicePtr(p)) {
            return Fail(KUDNN_STATUS_BAD_ARGUMENTS,
                        "LinearPostOpsFWD (no allocation): every buffer must be device memory");
        }
    }
    int rc = KUDNN_STATUS_SUCCESS;
    void *base = ScratchOf(rc);
    if (base == nullptr) {
        return rc;
    }
    Workspace fixed(static_cast<char *>(base) + kScratchCounterBytes, kScratchBytes - kScratchCounterBytes,
                    static_cast<uint32_t *>(base));
    return RunCore(plan->core, plan->x, a, b, y, bias, src, nullptr, 1.0f, 0.0f, gamma, fixed,
                   static_cast<hipStream_t>(stream));
}

int kudnn_linear_postops_destroy(kudnn_linear_postops_t plan)
{
    delete plan;
    return KUDNN_STATUS_SUCCESS;
}

int kudnn_plan_describe(const void *plan, char *buf, int len)
{
    if (plan == nullptr || buf == nullptr || len <= 0) {
        return Fail(KUDNN_STATUS_NULL_POINTER, "describe: null argument");
    }
    const auto *p = static_cast<const PlanBase *>(plan);
    std::snprintf(buf, static_cast<size_t>(len), "%s", p->desc.c_str());
    return KUDNN_STATUS_SUCCESS;
}

}  // extern "C"
