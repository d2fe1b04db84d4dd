// Operand packing: any strided layout / floating dtype -> K-contiguous rows in the compute dtype.
//
// The reference reorders non-standard layouts into f32 temporaries before calling BLAS
// (BatchedExtendedGemm, src/dnn/src/kudnn_gemm.cpp:725-765) and widens mismatched dtypes through
// MatrixConverter (:655-670). Here a single kernel does both for the operands that the MFMA kernels
// cannot read directly: it transposes through an LDS tile so that both the strided read and the
// K-contiguous write are coalesced, converts the element type exactly (bf16/f16 -> f32, or bf16 copy),
// and zero-fills the row tail up to the padded pitch so the GEMM needs no K-tail handling.
#include "device_common.h"
#include "kernels.h"

using namespace kudnn_dev;

namespace {

constexpr int kTile = 64;

__global__ __launch_bounds__(256) void pack_kernel(PackArgs p)
{
    __shared__ float tile[kTile][kTile + 1];
    const int tid = threadIdx.x;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kTile;
    const int64_t k0 = static_cast<int64_t>(blockIdx.x) * kTile;
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
            v = load_elem(p.src, p.src_dt, srcOff + r * p.s_r + k * p.s_k);
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

}  // namespace

int kudnn_launch_pack(const PackArgs &p, int64_t batches, hipStream_t stream)
{
    dim3 grid(static_cast<unsigned>((p.kp + kTile - 1) / kTile), static_cast<unsigned>((p.rows + kTile - 1) / kTile),
              static_cast<unsigned>(batches));
    hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
