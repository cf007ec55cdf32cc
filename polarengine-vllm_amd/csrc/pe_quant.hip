// PolarQuant quantizer on gfx950: weight [N, K] -> codes + fp16 block norms,
// one 16-lane group per (row, 128-block).
//
// Replaces PolarQuantizer.quantize_tensor (polarengine_vllm/quantizer.py:
// 206-257): pad K to the block with zeros, per-block L2 norm clamped at
// 1e-10, unit block rotated by the Hadamard transform and scaled by
// sqrt(128) -- i.e. the unnormalised transform H v with entries +-1 -- and
// code = the first index of the smallest |r - ct[l]| over the raw Lloyd-Max
// centroids; norms are stored as fp16 (round to nearest even).
//
// The transform is the butterfly (DPP / swizzle across the 16 lanes, each
// lane holding 8 consecutive positions) in fp32; the reference's fp32 matmul
// rounds differently, so a code can differ where r sits within a few ulps of
// the midpoint between two centroids. pack = 1 writes the half-block nibble
// layout directly (bits <= 4).

#include "pe_internal.h"

namespace pe {

template <int DT>
__device__ __forceinline__ float load_w(const void* w, int64_t i) {
  if constexpr (DT == PE_DTYPE_F16) return h2f(reinterpret_cast<const uint16_t*>(w)[i]);
  else if constexpr (DT == PE_DTYPE_BF16) return bf2f(reinterpret_cast<const uint16_t*>(w)[i]);
  else return reinterpret_cast<const float*>(w)[i];
}

template <int DT, bool PACK>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ w, int64_t ldw,
                                                       int N, int K, int nb,
                                                       const float* __restrict__ ct, int n_levels,
                                                       uint8_t* __restrict__ codes,
                                                       uint16_t* __restrict__ norms) {
  const int lane = threadIdx.x & 63;
  const int q = lane & 15;
  const int64_t item = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);  // (row, block)
  const bool live = item < (int64_t)N * nb;
  const int64_t it = live ? item : 0;  // dead groups compute on item 0 and store nothing
  const int n = (int)(it / nb), b = (int)(it - (int64_t)n * nb);
  const int k0 = b * kBlock + 8 * q;

  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    v[i] = (k0 + i < K) ? load_w<DT>(w, (int64_t)n * ldw + k0 + i) : 0.f;

  // L2 norm of the block: lane partial, then across the 16 lanes
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(v[i], v[i], ss);
  ss += lane_xor<1>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<8>(ss);
  float nrm = __builtin_sqrtf(ss);
  nrm = nrm > 1e-10f ? nrm : 1e-10f;

#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = v[i] / nrm;
  fwht128_group16_raw(v, q);

  // nearest centroid, first index on ties (ct ascending or not: a full scan)
  uint32_t c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float best = __builtin_fabsf(v[i] - ct[0]);
    uint32_t bi = 0;
    for (int l = 1; l < n_levels; ++l) {
      const float d = __builtin_fabsf(v[i] - ct[l]);
      if (d < best) {
        best = d;
        bi = (uint32_t)l;
      }
    }
    c[i] = bi;
  }
  if (!live) return;
  if (q == 0) norms[it] = f2h_bits(nrm);
  if constexpr (!PACK) {
    const uint32_t lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    const uint32_t hi = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
    *reinterpret_cast<uint2*>(codes + (int64_t)n * nb * kBlock + k0) = make_uint2(lo, hi);
  } else {
    // byte 64 b + i = code[128 b + 64 + i] << 4 | code[128 b + i]: lanes q < 8
    // hold positions 8q..8q+7 of the low half, lane q + 8 the same of the high
    const uint32_t lo = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
    const uint32_t hi = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
    const uint32_t olo = (uint32_t)__builtin_bit_cast(int, lane_xor<8>(__builtin_bit_cast(float, lo)));
    const uint32_t ohi = (uint32_t)__builtin_bit_cast(int, lane_xor<8>(__builtin_bit_cast(float, hi)));
    if (q < 8) {
      *reinterpret_cast<uint2*>(codes + (int64_t)n * nb * 64 + b * 64 + 8 * q) =
          make_uint2(lo | (olo << 4), hi | (ohi << 4));
    }
  }
}

template <int DT>
static int launch_quant(const void* w, int64_t ldw, int N, int K, int nb, const float* ct,
                        int n_levels, int pack, void* codes, uint16_t* norms, hipStream_t st) {
  const int64_t items = (int64_t)N * nb;
  const unsigned grid = (unsigned)((items + 15) / 16);
  uint8_t* c = reinterpret_cast<uint8_t*>(codes);
  if (pack) quantize_kernel<DT, true><<<grid, 256, 0, st>>>(w, ldw, N, K, nb, ct, n_levels, c, norms);
  else quantize_kernel<DT, false><<<grid, 256, 0, st>>>(w, ldw, N, K, nb, ct, n_levels, c, norms);
  return launch_status();
}

}  // namespace pe

extern "C" int pe_quantize(const void* w, int w_dtype, int64_t N, int K, int64_t ldw,
                           const float* ct, int n_levels, int pack, void* codes,
                           uint16_t* norms_f16, void* stream) {
  if (!w || !ct || !codes || !norms_f16) return PE_ERR_NULL;
  if (N < 0 || K <= 0 || ldw < K || N > INT32_MAX) return PE_ERR_DIMS;
  if (n_levels < 2 || n_levels > 256 || (pack && n_levels > 16) || (pack & ~1)) return PE_ERR_BITS;
  if (reinterpret_cast<uintptr_t>(codes) & 7) return PE_ERR_ALIGN;
  if (N == 0) return PE_OK;
  const int nb = (K + pe::kBlock - 1) / pe::kBlock;
  if ((int64_t)N * nb > ((int64_t)1 << 35)) return PE_ERR_DIMS;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (w_dtype) {
    case PE_DTYPE_F16: return pe::launch_quant<PE_DTYPE_F16>(w, ldw, (int)N, K, nb, ct, n_levels, pack, codes, norms_f16, st);
    case PE_DTYPE_BF16: return pe::launch_quant<PE_DTYPE_BF16>(w, ldw, (int)N, K, nb, ct, n_levels, pack, codes, norms_f16, st);
    case PE_DTYPE_F32: return pe::launch_quant<PE_DTYPE_F32>(w, ldw, (int)N, K, nb, ct, n_levels, pack, codes, norms_f16, st);
    default: return PE_ERR_DTYPE;
  }
}
