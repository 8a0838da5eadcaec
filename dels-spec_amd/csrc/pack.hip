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

// kchunk > 0 (col_blocks a multiple of it): the blocks go K-chunk-major instead,
// block (bi, bj) at ((bj / kchunk) * row_blocks + bi) * kchunk + bj % kchunk, so
// that kchunk consecutive K blocks of every row block -- one K chunk of the whole
// matrix -- are one contiguous run (the LM head's stream order).
__global__ void pack_mfma16_kernel(const uint16_t* __restrict__ W, int64_t ldw, int64_t rows, int64_t cols,
                                   int64_t col_blocks, int64_t chunks, int64_t kchunk, int64_t row_blocks,
                                   uint16_t* __restrict__ P) {
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
        const int64_t dst = kchunk > 0 ? ((bj / kchunk) * row_blocks + bi) * kchunk + bj % kchunk : blk;
        *reinterpret_cast<u32x4*>(P + (dst * 64 + lane) * 8) = v;
    }
}

hipError_t launch_pack_mfma16(const uint16_t* W, int64_t ldw, int64_t rows, int64_t cols, uint16_t* P,
                              hipStream_t s, int64_t kchunk) {
    const int64_t col_blocks = packed_col_blocks(cols);
    const int64_t row_blocks = packed_row_blocks(rows);
    const int64_t chunks = row_blocks * col_blocks * 64;
    if (chunks == 0) return hipSuccess;
    const int blocks = (int)std::min<int64_t>(4096, (chunks + 255) / 256);
    hipLaunchKernelGGL(pack_mfma16_kernel, dim3(blocks), dim3(256), 0, s, W, ldw, rows, cols, col_blocks, chunks,
                       kchunk, row_blocks, P);
    return hipGetLastError();
}

// e4m3 weights (bytes, row-major W [rows, cols]) into the fp8 block layouts:
//  * K128: block (bi, bj) covers rows 16*bi.. and columns 128*bj.. as 2 KiB
//    [half h][lane l][16 bytes], lane l holding W[16*bi + l%16][128*bj + 32*(l/16) + 16*h + e];
//  * K32: block (bi, bj) covers columns 32*bj.. as 512 bytes [lane l][8 bytes],
//    lane l holding W[16*bi + l%16][32*bj + 8*(l/16) + e].
// Blocks are row-block-major; out-of-range rows/columns are zero.  One thread
// writes one 16-byte (K128) or 8-byte (K32) piece.
__global__ void pack_fp8_kernel(const uint8_t* __restrict__ W, int64_t ldw, int64_t rows, int64_t cols,
                                int64_t col_blocks, int k128, int64_t pieces, uint8_t* __restrict__ P) {
    const int per_block = k128 ? 128 : 64;   // pieces per block
    const int width = k128 ? 16 : 8;         // bytes per piece
    for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < pieces;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(idx % per_block);
        const int64_t blk = idx / per_block;
        const int64_t bj = blk % col_blocks, bi = blk / col_blocks;
        const int lane = c & 63, half = c >> 6;
        const int64_t row = bi * 16 + (lane & 15);
        const int64_t c0 = k128 ? bj * 128 + 32 * (lane >> 4) + 16 * half : bj * 32 + 8 * (lane >> 4);
        uint8_t e[16];
        for (int k = 0; k < 16; ++k) e[k] = 0;
        if (row < rows)
            for (int k = 0; k < width && c0 + k < cols; ++k) e[k] = W[row * ldw + c0 + k];
        uint8_t* dst = P + blk * (int64_t)(per_block * width) + (int64_t)(k128 ? half * 1024 + lane * 16 : lane * 8);
        for (int k = 0; k < width; ++k) dst[k] = e[k];
    }
}

hipError_t launch_pack_fp8(const uint8_t* W, int64_t ldw, int64_t rows, int64_t cols, int layout, uint8_t* P,
                           hipStream_t s) {
    const bool k128 = layout == FP8_K128;
    const int64_t kb = k128 ? 128 : 32;
    const int64_t col_blocks = (cols + kb - 1) / kb;
    const int64_t pieces = ((rows + 15) / 16) * col_blocks * (k128 ? 128 : 64);
    if (pieces == 0) return hipSuccess;
    const int blocks = (int)std::min<int64_t>(4096, (pieces + 255) / 256);
    hipLaunchKernelGGL(pack_fp8_kernel, dim3(blocks), dim3(256), 0, s, W, ldw, rows, cols, col_blocks, k128 ? 1 : 0,
                       pieces, P);
    return hipGetLastError();
}

}  // namespace dels
