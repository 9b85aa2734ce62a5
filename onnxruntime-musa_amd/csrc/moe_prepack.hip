// moe_prepack.hip -- one-time reordering of QMoE expert weights into the
// tile-major layout the decode and prefill kernels read.
//
// The op's layout is row-major per expert: [E, N, K/pack] bytes, K
// contiguous within an output row.  A decode wave's load instruction covers
// 16 rows x 16 bytes per lane group, i.e. 16 separate 64-byte (int4) or
// 128-byte (int8) runs of one chunk of 128 k.  Tile-major stores each
// (16-row tile, chunk) as one contiguous block, so that the same instruction
// reads 1 KB in one run:
//
//   block (tile j, chunk c) at (j * nchunks + c) * CB, CB = 16 * cbytes
//   piece q (16 bytes, k [32 q / kv .. ] of the chunk row) of row r inside
//     it at ((q % kv) * 64 + (q / kv) * 16 + r) * 16
//
// with cbytes = 64 (int4) or 128 (int8) bytes of one row per chunk and kv =
// cbytes / 64 16-byte vectors per 32 k.  Lane l = 16 g + r of a decode wave
// then reads piece kv g + v of row r at v * 1 KB + 16 l, and rows never
// cross an expert (N is a multiple of 16), so the experts can be packed as
// one [E * N, K/pack] matrix.  Scales and biases keep their layouts.
#include "moe_device.h"
#include "moe_launch.h"

namespace moe {
namespace {

// One thread per 16-byte piece, in source order (coalesced reads; each
// group of 64 consecutive pieces of a row lands in 4 or 8 runs of 256 bytes).
__global__ void __launch_bounds__(256) prepack_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                      int64_t npieces, int64_t row_pieces, int cpieces, int kv) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < npieces; q += stride) {
    const int64_t row = q / row_pieces;
    const int64_t p = q - row * row_pieces;  // piece within the row
    const int64_t c = p / cpieces;           // chunk
    const int pc = static_cast<int>(p - c * cpieces);
    const int64_t nchunks = row_pieces / cpieces;
    const int64_t blk = (row / 16) * nchunks + c;
    const int64_t at = blk * (16 * cpieces) + (pc % kv) * 64 + (pc / kv) * 16 + (row % 16);
    dst[at] = src[q];
  }
}

}  // namespace

hipError_t launch_prepack(const uint8_t* src, uint8_t* dst, int64_t rows, int64_t row_bytes, int cbytes,
                          hipStream_t stream) {
  if (rows % 16 || row_bytes % cbytes || (cbytes != 64 && cbytes != 128)) return hipErrorInvalidValue;
  const int64_t row_pieces = row_bytes / 16;
  const int64_t npieces = rows * row_pieces;
  if (npieces == 0) return hipSuccess;
  const int64_t want = (npieces + 255) / 256;
  const unsigned blocks = static_cast<unsigned>(want < 65536 ? want : 65536);
  hipLaunchKernelGGL(prepack_kernel, dim3(blocks), dim3(256), 0, stream, reinterpret_cast<const u32x4_t*>(src),
                     reinterpret_cast<u32x4_t*>(dst), npieces, row_pieces, cbytes / 16, cbytes / 64);
  return hipGetLastError();
}

}  // namespace moe
