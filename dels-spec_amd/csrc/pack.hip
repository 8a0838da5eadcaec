// Repacking of bf16 weights into the MFMA-16 block layout.
//
// Block (bi, bj) covers rows 16*bi..16*bi+15 and columns 32*bj..32*bj+31 of
// W [rows, cols]; blocks are stored row-block-major (bj fastest), each as 1 KiB
// in wave64 lane order: lane l holds W[16*bi + l%16][32*bj + 8*(l/16) + e],
// e = 0..7.  Out-of-range rows/columns are zero.  A 16-row MFMA operand tile
// for one 32-wide K step is then a single contiguous KiB, which the kernels
// load with one coalesced dwordx4 per lane.
#include <algorithm>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

__global__ void pack_mfma16_kernel(const uint16_t* __restrict__ W, int64_t ldw, int64_t rows, int64_t cols,
                                   int64_t col_blocks, int64_t chunks, uint16_t* __restrict__ P) {
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < chunks;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(idx & 63);
        const int64_t blk = idx >> 6;
        const int64_t bj = blk % col_blocks, bi = blk / col_blocks;
        const int64_t row = bi * 16 + (lane & 15);
        const int64_t c0 = bj * 32 + 8 * (lane >> 4);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (row < rows) {
            const uint16_t* src = W + row * ldw + c0;
            if (c0 + 8 <= cols) {
                v = *reinterpret_cast<const u32x4*>(src);
            } else {
                uint16_t e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                for (int k = 0; k < 8 && c0 + k < cols; ++k) e[k] = src[k];
                __builtin_memcpy(&v, e, 16);
            }
        }
        *reinterpret_cast<u32x4*>(P + idx * 8) = v;
    }
}

hipError_t launch_pack_mfma16(const uint16_t* W, int64_t ldw, int64_t rows, int64_t cols, uint16_t* P,
                              hipStream_t s) {
    const int64_t col_blocks = packed_col_blocks(cols);
    const int64_t chunks = packed_row_blocks(rows) * col_blocks * 64;
    if (chunks == 0) return hipSuccess;
    const int blocks = (int)std::min<int64_t>(4096, (chunks + 255) / 256);
    hipLaunchKernelGGL(pack_mfma16_kernel, dim3(blocks), dim3(256), 0, s, W, ldw, rows, cols, col_blocks, chunks,
                       P);
    return hipGetLastError();
}

}  // namespace dels
