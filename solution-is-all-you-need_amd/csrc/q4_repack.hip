// q4_repack.hip -- GGUF Q4_0 <-> MFMA-ordered repacked layout, and an fp32
// dequantiser.  Load-time kernels; the layout is described in moe_common.h.
//
// Q4_0 block (python/phantom/loader/gguf_loader.py:72, :362-381): 18 bytes,
// fp16 scale d then 16 bytes qs; element j = (qs[j] & 15) - 8, element
// j + 16 = (qs[j] >> 4) - 8, both times d.
#include "moe_common.h"
#include "moe_launch.h"

namespace pmoe {

// One thread per (row tile, quad, lane): gathers 4 x 4 qs bytes of one row.
__global__ __launch_bounds__(256) void q4_repack_kernel(const uint8_t* __restrict__ src, int64_t rows,
                                                        int64_t Kg, int64_t Kq,
                                                        uint8_t* __restrict__ nib,
                                                        uint16_t* __restrict__ scale) {
  const int64_t total = (rows / kRowTile) * Kq * kWave;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i % kWave);
    const int64_t tq = i / kWave;  // rt * Kq + q
    const int64_t q = tq % Kq;
    const int64_t rt = tq / Kq;
    const int n = lane % 16;
    const int p = lane / 16;
    const int64_t row = rt * kRowTile + n;
    uint32_t words[4];
    uint16_t sc[4];
    for (int gi = 0; gi < 4; ++gi) {
      const int64_t g = q * 4 + gi;
      if (g < Kg) {
        const uint8_t* blk = src + (row * Kg + g) * 18;
        sc[gi] = (uint16_t)(blk[0] | (blk[1] << 8));
        const uint8_t* qs = blk + 2 + 4 * p;
        words[gi] = (uint32_t)qs[0] | ((uint32_t)qs[1] << 8) | ((uint32_t)qs[2] << 16) |
                    ((uint32_t)qs[3] << 24);
      } else {
        sc[gi] = 0;               // padded group: scale 0 ...
        words[gi] = 0x88888888u;  // ... and q = 0
      }
    }
    u32x4 v = {words[0], words[1], words[2], words[3]};
    *reinterpret_cast<u32x4*>(nib + i * 16) = v;
    if (p == 0) {
      uint16_t* s = scale + tq * kQuadScales + n * 4;
      for (int gi = 0; gi < 4; ++gi) s[gi] = sc[gi];
    }
  }
}

// One thread per Q4_0 block (row, group): rebuilds its 18 bytes.
__global__ __launch_bounds__(256) void q4_unrepack_kernel(const uint8_t* __restrict__ nib,
                                                          const uint16_t* __restrict__ scale,
                                                          int64_t rows, int64_t Kg, int64_t Kq,
                                                          uint8_t* __restrict__ dst) {
  const int64_t total = rows * Kg;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / Kg;
    const int64_t g = i % Kg;
    const int64_t rt = row / kRowTile;
    const int n = (int)(row % kRowTile);
    const int64_t q = g / 4;
    const int gi = (int)(g % 4);
    const int64_t tq = rt * Kq + q;
    uint8_t* blk = dst + i * 18;
    const uint16_t s = scale[tq * kQuadScales + n * 4 + gi];
    blk[0] = (uint8_t)(s & 0xff);
    blk[1] = (uint8_t)(s >> 8);
    for (int p = 0; p < 4; ++p) {
      const uint8_t* w = nib + ((tq * kWave) + p * 16 + n) * 16 + gi * 4;
      for (int b = 0; b < 4; ++b) blk[2 + 4 * p + b] = w[b];
    }
  }
}

// One thread per Q4_0 block: 32 fp32 values.
__global__ __launch_bounds__(256) void q4_dequant_f32_kernel(const uint8_t* __restrict__ src,
                                                             int64_t n_blocks,
                                                             float* __restrict__ out) {
  for (int64_t b = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; b < n_blocks;
       b += (int64_t)gridDim.x * blockDim.x) {
    const uint8_t* blk = src + b * 18;
    const float d = half_bits_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
    float* o = out + b * 32;
    for (int j = 0; j < 16; ++j) {
      const int v = blk[2 + j];
      o[j] = (float)((v & 15) - 8) * d;
      o[j + 16] = (float)((v >> 4) - 8) * d;
    }
  }
}

static int grid_for(int64_t n) {
  int64_t g = ceil_div(n, 256);
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

hipError_t launch_q4_repack(const uint8_t* src, int64_t rows, int64_t K, uint8_t* nib,
                            uint16_t* scale, hipStream_t stream) {
  const int64_t Kg = K / kGroup;
  const int64_t Kq = ceil_div(K, kQuad);
  const int64_t total = (rows / kRowTile) * Kq * kWave;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(q4_repack_kernel, dim3(grid_for(total)), dim3(256), 0, stream, src, rows, Kg,
                     Kq, nib, scale);
  return hipGetLastError();
}

hipError_t launch_q4_unrepack(const uint8_t* nib, const uint16_t* scale, int64_t rows, int64_t K,
                              uint8_t* dst, hipStream_t stream) {
  const int64_t Kg = K / kGroup;
  const int64_t Kq = ceil_div(K, kQuad);
  const int64_t total = rows * Kg;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(q4_unrepack_kernel, dim3(grid_for(total)), dim3(256), 0, stream, nib, scale,
                     rows, Kg, Kq, dst);
  return hipGetLastError();
}

hipError_t launch_q4_dequant_f32(const uint8_t* src, int64_t n_blocks, float* out,
                                 hipStream_t stream) {
  if (n_blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(q4_dequant_f32_kernel, dim3(grid_for(n_blocks)), dim3(256), 0, stream, src,
                     n_blocks, out);
  return hipGetLastError();
}

}  // namespace pmoe
