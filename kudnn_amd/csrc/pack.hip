// Operand packing: any strided layout / floating dtype -> K-contiguous rows in the compute dtype.
//
// The reference reorders non-standard layouts into f32 temporaries before calling BLAS
// (BatchedExtendedGemm, src/dnn/src/kudnn_gemm.cpp:725-765) and widens mismatched dtypes through
// MatrixConverter (:655-670). Here a single kernel does both for the operands that the MFMA kernels
// cannot read directly: it transposes through an LDS tile so that both the strided read and the
// K-contiguous write are coalesced, converts the element type exactly (bf16/f16 -> f32, or bf16 copy; u8 -> s8
// shifted by -128 for the integer MFMA), and zero-fills the row tail up to the padded pitch so the GEMM needs no
// K-tail handling.
#include "device_common.h"
#include "kernels.h"

using namespace kudnn_dev;

namespace {

constexpr int kTile = 64;

__global__ __launch_bounds__(256) void pack_kernel(PackArgs p)
{
    __shared__ float tile[kTile][kTile + 1];
    const int tid = threadIdx.x;
    // rows on x (up to 2^31 - 1 workgroups: a folded batch makes M large), K on y
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kTile;
    const int64_t k0 = static_cast<int64_t>(blockIdx.y) * kTile;
    const int64_t b = blockIdx.z;
    const int64_t i2 = b % p.bdim[2];
    const int64_t i1 = (b / p.bdim[2]) % p.bdim[1];
    const int64_t i0 = b / (p.bdim[2] * p.bdim[1]);
    const int64_t srcOff = i0 * p.bs[0] + i1 * p.bs[1] + i2 * p.bs[2];

    // Read so that consecutive threads touch consecutive source addresses.
    const bool rFast = (p.s_r == 1 && p.s_k != 1);
    for (int i = 0; i < kTile * kTile / 256; ++i) {
        int e = tid + i * 256;
        int rr = rFast ? (e % kTile) : (e / kTile);
        int kk = rFast ? (e / kTile) : (e % kTile);
        int64_t r = r0 + rr, k = k0 + kk;
        float v = 0.0f;
        if (r < p.rows && k < p.cols) {
            v = load_elem(p.src, p.src_dt, srcOff + r * p.s_r + k * p.s_k) - static_cast<float>(p.shift);
        }
        tile[rr][kk] = v;
    }
    __syncthreads();
    for (int i = 0; i < kTile * kTile / 256; ++i) {
        int e = tid + i * 256;
        int rr = e / kTile, kk = e % kTile;
        int64_t r = r0 + rr, k = k0 + kk;
        if (r < p.rows && k < p.kp) {
            store_elem(p.dst, p.dst_dt, b * p.dst_bstride + r * p.kp + k, tile[rr][kk]);
        }
    }
}

// One wave per row of a packed int8 operand: sums its kp elements (16 per lane and step), then scales.
__global__ __launch_bounds__(256) void rowsum_s8_kernel(const int8_t *p, int64_t rows, int64_t kp, int64_t copies,
                                                        int64_t bstride, uint32_t scale, int32_t *out)
{
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows * copies) {
        return;  // no barrier below
    }
    const int64_t c = row / rows, r = row - c * rows;
    const int8_t *src = p + c * bstride + r * kp;
    int32_t sum = 0;
    // kp is a multiple of the 128-element k-tile, so whole 16-byte chunks are in bounds
    for (int64_t k = static_cast<int64_t>(lane) * 16; k < kp; k += 64 * 16) {
        const int4 v = *reinterpret_cast<const int4 *>(src + k);
        const int w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int b = 0; b < 4; ++b) sum += static_cast<int8_t>(static_cast<uint32_t>(w[j]) >> (8 * b));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        sum += __shfl_xor(sum, o);
    }
    if (lane == 0) {
        out[c * rows + r] = static_cast<int32_t>(static_cast<uint32_t>(sum) * scale);
    }
}

}  // namespace

int kudnn_launch_rowsum_s8(const int8_t *p, int64_t rows, int64_t kp, int64_t copies, int64_t bstride, uint32_t scale,
                           int32_t *out, hipStream_t stream)
{
    if (kp % 16 != 0) {
        return -1;
    }
    const int64_t total = rows * copies;
    hipLaunchKernelGGL(rowsum_s8_kernel, dim3(static_cast<unsigned>((total + 3) / 4)), dim3(256), 0, stream, p, rows,
                       kp, copies, bstride, scale, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int kudnn_launch_pack(const PackArgs &p, int64_t batches, hipStream_t stream)
{
    dim3 grid(static_cast<unsigned>((p.rows + kTile - 1) / kTile), static_cast<unsigned>((p.kp + kTile - 1) / kTile),
              static_cast<unsigned>(batches));
    hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
