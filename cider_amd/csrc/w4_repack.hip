// Repack of the reference W4 layout into the library's W4 layout.
//
//   src [K/2, N]: element (k, n) = high nibble of src[k/2][n] for even k, low
//                 nibble for odd k; value = nibble - 8   (cider/ops.py:93-116,
//                 cider/kernels/w4a8_matmul.metal:47-70)
//   dst [N, K/2]: element (n, k) = low nibble of dst[n][k/2] for even k, high
//                 nibble for odd k; two's-complement int4
//
// value - 8 in 4-bit two's complement is nibble ^ 8, so
//   dst[n][j] = ((src[j][n] >> 4) ^ 8) | (((src[j][n] & 15) ^ 8) << 4).
// A 64 x 64 byte tile is transposed through LDS so both the reads (along n)
// and the writes (along j) are coalesced.
#include "common.hpp"
#include "kernels.hpp"

namespace cider {

__global__ __launch_bounds__(256) void w4_repack_kernel(const uint8_t* __restrict__ src,
                                                        uint8_t* __restrict__ dst,
                                                        int N, int J) {
  __shared__ uint8_t tile[64][65];
  const int j0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int j = j0 + r, n = n0 + tx;
    tile[r][tx] = (j < J && n < N) ? src[(int64_t)j * N + n] : 0;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int n = n0 + r, j = j0 + tx;
    if (n < N && j < J) {
      const uint32_t b = tile[tx][r];
      dst[(int64_t)n * J + j] = (uint8_t)(((b >> 4) ^ 8u) | (((b & 15u) ^ 8u) << 4));
    }
  }
}

hipError_t launch_w4_repack_ref(const uint8_t* src_kn, uint8_t* dst_nk, int N,
                                int K, hipStream_t s) {
  const int J = K / 2;
  const dim3 grid((N + 63) / 64, (J + 63) / 64), block(256);
  w4_repack_kernel<<<grid, block, 0, s>>>(src_kn, dst_nk, N, J);
  return hipGetLastError();
}

}  // namespace cider
