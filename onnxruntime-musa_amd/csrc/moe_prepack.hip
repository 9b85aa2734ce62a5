// moe_prepack.hip -- one-time reordering of expert weights (QMoE int4 /
// int8, MoE fp16 / bf16) into the tile-major layout the decode and prefill
// kernels read.
//
// The op's layout is row-major per expert: [E, N, K/pack] bytes, K
// contiguous within an output row.  A decode wave's load instruction covers
// 16 rows x 16 bytes per lane group, i.e. 16 separate 64-byte (int4),
// 128-byte (int8) or 256-byte (16-bit) runs of one chunk of 128 k, and a
// prefill wave's 32 rows x 2 halves likewise.  Tile-major stores each
// (16-row tile, chunk) as one contiguous block, so that the same instruction
// reads 1 KB in one run:
//
//   block (tile j, chunk c) at (j * nchunks + c) * CB, CB = 16 * cbytes
//   piece q (16 bytes, k [32 q / kv .. ] of the chunk row) of row r inside
//     it at ((q % kv) * 64 + (q / kv) * 16 + r) * 16
//
// with cbytes = 64 (int4), 128 (int8) or 256 (16-bit) bytes of one row per
// chunk and kv = cbytes / 64 16-byte vectors per 32 k.  Lane l = 16 g + r of a decode wave
// then reads piece kv g + v of row r at v * 1 KB + 16 l, and rows never
// cross an expert (N is a multiple of 16), so the experts can be packed as
// one [E * N, K/pack] matrix.
//
// K that is not whole chunks (gpt-oss: 2880 = 22.5 chunks) is padded with
// zero bytes to nchunks * cbytes per row.  The fused fc1 of interleaved
// SwiGLU (gate row 2f, linear row 2f + 1) is stored de-interleaved, gate
// rows [0, N/2) then linear rows [N/2, N) of each expert, so that a 16-row
// tile holds one kind; its scales and biases keep their layouts.
#include "moe_device.h"
#include "moe_launch.h"

namespace moe {
namespace {

// One thread per 16-byte piece of the packed copy, in packed order
// (coalesced writes); the source piece of row srow, or zeros past the row.
__global__ void __launch_bounds__(256) prepack_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                      int64_t npieces, int64_t nchunks, int64_t src_row_pieces,
                                                      int cpieces, int kv, int64_t expert_rows, int deint) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t bpieces = 16 * cpieces;  // pieces of one (tile, chunk) block
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < npieces; q += stride) {
    const int64_t blk = q / bpieces;
    const int o = static_cast<int>(q - blk * bpieces);
    const int64_t tile = blk / nchunks, c = blk - tile * nchunks;
    const int r = o % 16;
    const int pc = ((o / 16) % 4) * kv + o / 64;  // piece of the chunk row
    const int64_t row = tile * 16 + r;
    int64_t srow = row;
    if (deint) {
      const int64_t e = row / expert_rows, l = row - e * expert_rows, half = expert_rows / 2;
      srow = e * expert_rows + (l < half ? 2 * l : 2 * (l - half) + 1);
    }
    const int64_t sp = c * cpieces + pc;
    dst[q] = sp < src_row_pieces ? src[srow * src_row_pieces + sp] : u32x4_t{0u, 0u, 0u, 0u};
  }
}

// Block scales of the step-scale decode kernels, one thread per packed
// element: block (tile j, chunk c) of 16 rows x nb scales (nb = 128 / block
// size) at (j * nchunks + c) * 16 * nb elements, scale b of row r at r * nb
// + b; rows de-interleaved like their weights; blocks past K are zero.
template <typename E>
__global__ void __launch_bounds__(256) prepack_scales_kernel(const E* __restrict__ src, E* __restrict__ dst,
                                                             int64_t nelems, int64_t nchunks, int nb, int64_t nblk,
                                                             int64_t expert_rows, int deint) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < nelems; q += stride) {
    const int64_t blk = q / (16 * nb);
    const int o = static_cast<int>(q - blk * 16 * nb);
    const int64_t tile = blk / nchunks, c = blk - tile * nchunks;
    const int64_t row = tile * 16 + o / nb;
    int64_t srow = row;
    if (deint) {
      const int64_t e = row / expert_rows, l = row - e * expert_rows, half = expert_rows / 2;
      srow = e * expert_rows + (l < half ? 2 * l : 2 * (l - half) + 1);
    }
    const int64_t b = c * nb + o % nb;
    dst[q] = b < nblk ? src[srow * nblk + b] : E{0};
  }
}

}  // namespace

hipError_t launch_prepack_scales(const void* src, void* dst, int elem_bytes, int64_t rows, int64_t nblk, int block,
                                 int64_t expert_rows, bool deint, hipStream_t stream) {
  if (rows % 16 || (block != 32 && block != 64) || (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4) ||
      expert_rows <= 0 ||
      rows % expert_rows || (deint && expert_rows % 32))
    return hipErrorInvalidValue;
  const int nb = 128 / block;
  const int64_t nchunks = (nblk * block + 127) / 128;
  const int64_t nelems = rows * nchunks * nb;
  if (nelems == 0) return hipSuccess;
  const int64_t want = (nelems + 255) / 256;
  const unsigned blocks = static_cast<unsigned>(want < 65536 ? want : 65536);
  if (elem_bytes == 1)
    hipLaunchKernelGGL(prepack_scales_kernel<uint8_t>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), nelems, nchunks, nb, nblk,
                       expert_rows, deint ? 1 : 0);
  else if (elem_bytes == 2)
    hipLaunchKernelGGL(prepack_scales_kernel<uint16_t>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), nelems, nchunks, nb, nblk,
                       expert_rows, deint ? 1 : 0);
  else
    hipLaunchKernelGGL(prepack_scales_kernel<uint32_t>, dim3(blocks), dim3(256), 0, stream,
                       static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), nelems, nchunks, nb, nblk,
                       expert_rows, deint ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_prepack(const uint8_t* src, uint8_t* dst, int64_t rows, int64_t row_bytes, int cbytes,
                          int64_t expert_rows, bool deint, hipStream_t stream) {
  if (rows % 16 || row_bytes % 16 || (cbytes != 64 && cbytes != 128 && cbytes != 256) || expert_rows <= 0 ||
      rows % expert_rows ||
      (deint && expert_rows % 32))
    return hipErrorInvalidValue;
  const int64_t nchunks = (row_bytes + cbytes - 1) / cbytes;
  const int cpieces = cbytes / 16;
  const int64_t npieces = rows * nchunks * cpieces;
  if (npieces == 0) return hipSuccess;
  const int64_t want = (npieces + 255) / 256;
  const unsigned blocks = static_cast<unsigned>(want < 65536 ? want : 65536);
  hipLaunchKernelGGL(prepack_kernel, dim3(blocks), dim3(256), 0, stream, reinterpret_cast<const u32x4_t*>(src),
                     reinterpret_cast<u32x4_t*>(dst), npieces, nchunks, row_bytes / 16, cpieces, cbytes / 64,
                     expert_rows, deint ? 1 : 0);
  return hipGetLastError();
}

}  // namespace moe
