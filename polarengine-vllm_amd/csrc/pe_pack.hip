// Load-time code format kernels (bit-exact integer work, HBM-bound).
//
//  * pe_pack_nibble: int8 codes [rows, K] -> half-block nibbles [rows, K/2],
//    byte[64b + i] = code[128b + 64 + i] << 4 | code[128b + i]. Replaces
//    pack_codes_int4 (kernels/polar_gemv.py:263-283) as run by
//    process_weights_after_loading (linear_method.py:243-248); same mapping as
//    packing.py:22-60.
//  * pe_unpack_q5: on-disk LSB-first Q5 (8 codes in 5 bytes) -> int8 codes.
//    Replaces unpack_codes_q5 (packing.py:163-209) used by loader.py:412-417.
//  * pe_tile_weights: row-major codes/norms -> the tiled-16 runtime layout
//    (16 rows x one block contiguous), rows padded to 16 with zeros.
//
// One lane per 16 output bytes; both are pure streaming kernels.

#include "pe_common.h"

namespace pe {

// lane t handles bytes 16t..16t+15 of the packed output of its row
__global__ __launch_bounds__(256) void pack_nibble_kernel(const uint8_t* __restrict__ codes,
                                                          uint8_t* __restrict__ packed,
                                                          int64_t rows, int64_t K) {
  const int64_t per_row = K / 32;  // 16-byte output chunks per row
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * per_row) return;
  const int64_t r = t / per_row;
  const int64_t c = t - r * per_row;      // chunk within the row
  const int64_t b = c >> 2;               // 128-block
  const int64_t i0 = (c & 3) * 16;        // first pair index in the block
  const uint8_t* src = codes + r * K + b * kBlock + i0;
  const uint4 lo = *reinterpret_cast<const uint4*>(src);
  const uint4 hi = *reinterpret_cast<const uint4*>(src + 64);
  const uint32_t l[4] = {lo.x, lo.y, lo.z, lo.w}, h[4] = {hi.x, hi.y, hi.z, hi.w};
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = (l[j] & 0x0f0f0f0fu) | ((h[j] & 0x0f0f0f0fu) << 4);
  *reinterpret_cast<uint4*>(packed + r * (K / 2) + b * 64 + i0) = make_uint4(o[0], o[1], o[2], o[3]);
}

// lane t handles one 5-byte group -> 8 codes
__global__ __launch_bounds__(256) void unpack_q5_kernel(const uint8_t* __restrict__ packed,
                                                        int8_t* __restrict__ codes,
                                                        int64_t groups) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= groups) return;
  const uint8_t* p = packed + t * 5;
  const uint32_t b0 = p[0], b1 = p[1], b2 = p[2], b3 = p[3], b4 = p[4];
  uint32_t c[8];
  c[0] = b0 & 0x1f;
  c[1] = ((b0 >> 5) | (b1 << 3)) & 0x1f;
  c[2] = (b1 >> 2) & 0x1f;
  c[3] = ((b1 >> 7) | (b2 << 1)) & 0x1f;
  c[4] = ((b2 >> 4) | (b3 << 4)) & 0x1f;
  c[5] = (b3 >> 1) & 0x1f;
  c[6] = ((b3 >> 6) | (b4 << 2)) & 0x1f;
  c[7] = (b4 >> 3) & 0x1f;
  const uint32_t w0 = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
  const uint32_t w1 = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  *reinterpret_cast<uint2*>(codes + t * 8) = make_uint2(w0, w1);
}

// HLWQ bitpack_5, MSB-first: lane t turns 5 bytes into 8 codes; groups past
// `total` codes are cut on the last group (codes beyond total are not written)
__global__ __launch_bounds__(256) void unpack_q5_hlwq_kernel(const uint8_t* __restrict__ packed,
                                                             int8_t* __restrict__ codes,
                                                             int64_t total) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t first = t * 8;
  if (first >= total) return;
  const uint8_t* p = packed + t * 5;
  const uint32_t b0 = p[0], b1 = p[1], b2 = p[2], b3 = p[3], b4 = p[4];
  // the 40 bits b0..b4 read MSB-first; code j = bits 35 - 5 j .. 39 - 5 j
  const uint64_t w = ((uint64_t)b0 << 32) | ((uint64_t)b1 << 24) | ((uint64_t)b2 << 16) |
                     ((uint64_t)b3 << 8) | (uint64_t)b4;
  int8_t c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] = (int8_t)((w >> (35 - 5 * j)) & 0x1f);
  const int64_t n = total - first < 8 ? total - first : 8;
  for (int j = 0; j < n; ++j) codes[first + j] = c[j];
}

// lane t moves 16 bytes of codes: destination chunk t of codes_t
// [tiles][nb][16][bpb], source row tile*16 + r, block b, bytes c*16 .. +15
__global__ __launch_bounds__(256) void tile_codes_kernel(const uint8_t* __restrict__ codes,
                                                         uint8_t* __restrict__ codes_t,
                                                         int64_t N, int row_bytes, int nb,
                                                         int64_t chunks) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= chunks) return;
  const int bpb16 = row_bytes / nb / 16;  // 16-byte chunks per block (4 or 8)
  const int64_t c = t % bpb16;
  int64_t u = t / bpb16;
  const int r = (int)(u & 15);
  u >>= 4;
  const int64_t b = u % nb, tile = u / nb;
  const int64_t n = tile * 16 + r;
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (n < N) v = *reinterpret_cast<const uint4*>(codes + n * row_bytes + b * (bpb16 * 16) + c * 16);
  *reinterpret_cast<uint4*>(codes_t + t * 16) = v;
}

// lane t writes norms_t[t] of [tiles][nb][16]
__global__ __launch_bounds__(256) void tile_norms_kernel(const uint16_t* __restrict__ norms,
                                                         uint16_t* __restrict__ norms_t,
                                                         int64_t N, int nb, int64_t total) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const int r = (int)(t & 15);
  const int64_t u = t >> 4;
  const int64_t b = u % nb, tile = u / nb;
  const int64_t n = tile * 16 + r;
  norms_t[t] = n < N ? norms[n * nb + b] : (uint16_t)0;
}

}  // namespace pe

extern "C" int pe_tile_weights(const void* codes, const uint16_t* norms, int64_t N, int row_bytes,
                               int nb, void* codes_t, uint16_t* norms_t, void* stream) {
  if (!codes || !norms || !codes_t || !norms_t) return PE_ERR_NULL;
  if (N <= 0 || nb <= 0 || row_bytes <= 0) return PE_ERR_DIMS;
  if (row_bytes != nb * 64 && row_bytes != nb * pe::kBlock) return PE_ERR_DIMS;
  if (!pe::aligned16(codes) || !pe::aligned16(codes_t)) return PE_ERR_ALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t tiles = (N + 15) / 16;
  const int64_t chunks = tiles * 16 * row_bytes / 16;
  const int64_t nnorm = tiles * 16 * nb;
  if (chunks > (int64_t(1) << 31) || nnorm > (int64_t(1) << 31)) return PE_ERR_DIMS;
  pe::tile_codes_kernel<<<dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st>>>(
      reinterpret_cast<const uint8_t*>(codes), reinterpret_cast<uint8_t*>(codes_t), N, row_bytes,
      nb, chunks);
  if (int rc = pe::launch_status()) return rc;
  pe::tile_norms_kernel<<<dim3((unsigned)((nnorm + 255) / 256)), dim3(256), 0, st>>>(
      norms, norms_t, N, nb, nnorm);
  return pe::launch_status();
}

extern "C" int pe_pack_nibble(const int8_t* codes, uint8_t* packed, int64_t rows, int64_t K,
                              void* stream) {
  if (!codes || !packed) return PE_ERR_NULL;
  if (rows < 0 || K <= 0 || K % pe::kBlock) return PE_ERR_DIMS;
  if (!pe::aligned16(codes) || !pe::aligned16(packed)) return PE_ERR_ALIGN;
  if (rows == 0) return PE_OK;
  const int64_t work = rows * (K / 32);
  if (work > (int64_t(1) << 31)) return PE_ERR_DIMS;
  pe::pack_nibble_kernel<<<dim3((unsigned)((work + 255) / 256)), dim3(256), 0,
                           reinterpret_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint8_t*>(codes), packed, rows, K);
  return pe::launch_status();
}

extern "C" int pe_unpack_q5(const uint8_t* packed, int8_t* codes, int64_t rows, int64_t K,
                            void* stream) {
  if (!codes || !packed) return PE_ERR_NULL;
  if (rows < 0 || K <= 0 || K % pe::kBlock) return PE_ERR_DIMS;
  if (reinterpret_cast<uintptr_t>(codes) & 7) return PE_ERR_ALIGN;
  if (rows == 0) return PE_OK;
  const int64_t groups = rows * (K / 8);
  if (groups > (int64_t(1) << 31)) return PE_ERR_DIMS;
  pe::unpack_q5_kernel<<<dim3((unsigned)((groups + 255) / 256)), dim3(256), 0,
                         reinterpret_cast<hipStream_t>(stream)>>>(packed, codes, groups);
  return pe::launch_status();
}

extern "C" int pe_unpack_q5_hlwq(const uint8_t* packed, int64_t packed_bytes, int8_t* codes,
                                 int64_t total, void* stream) {
  if (!codes || !packed) return PE_ERR_NULL;
  if (packed_bytes < 0 || packed_bytes % 5 || total < 0) return PE_ERR_DIMS;
  if (total > packed_bytes / 5 * 8) return PE_ERR_DIMS;
  if (total == 0) return PE_OK;
  const int64_t groups = (total + 7) / 8;
  if (groups > (int64_t(1) << 31)) return PE_ERR_DIMS;
  pe::unpack_q5_hlwq_kernel<<<dim3((unsigned)((groups + 255) / 256)), dim3(256), 0,
                              reinterpret_cast<hipStream_t>(stream)>>>(packed, codes, total);
  return pe::launch_status();
}
