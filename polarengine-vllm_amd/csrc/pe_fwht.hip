// Blockwise FWHT-128 for gfx950.
//
// Replaces the reference's fwht_matmul (kernels/fwht.py:77-108), which runs
// x.reshape(-1, 128) @ H as one fp32 SGEMM (128x the additions of a
// butterfly), and the unwired CUDA butterfly (kernels/cuda/fwht_cuda.cu:35-86).
// Here a 16-lane group owns one 128-block: 8 values per lane, 3 in-lane
// stages and 4 cross-lane stages (lane xor 1/2/4/8), one 16-byte load and one
// 16/32-byte store per lane. HBM-bound: 2*2 bytes per element for f16 in and
// pair-f16 out.

#include <cmath>

#include "pe_internal.h"

namespace pe {

template <int XDT, int YL, bool XFORM = true>
__global__ __launch_bounds__(256) void fwht128_kernel(const void* x, void* y, int64_t rows,
                                                      int nbc, int64_t ldx) {
  const int64_t total = rows * (int64_t)nbc;
  int64_t bid = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int q = threadIdx.x & 15;
  const bool live = bid < total;
  if (!live) bid = total - 1;  // keep the 16-lane group converged; store is masked
  const int64_t r = bid / nbc;
  const int cb = (int)(bid - r * nbc);
  constexpr int esz = XDT == PE_DTYPE_F32 ? 4 : 2;
  const char* src = reinterpret_cast<const char*>(x) + ((r * ldx) + (int64_t)cb * kBlock + q * 8) * esz;
  float v[8];
  load8<XDT>(src, v);
  if constexpr (XFORM) fwht128_group16(v, q);

  if constexpr (YL == PE_XTF_PAIR_F16) {
    store_pair_block(v, q, reinterpret_cast<uint32_t*>(y) + bid * 64, live);
  } else if constexpr (YL == PE_XTF_F32) {
    if (!live) return;
    float* dst = reinterpret_cast<float*>(y) + (r * (int64_t)nbc * kBlock + (int64_t)cb * kBlock + q * 8);
    reinterpret_cast<float4*>(dst)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(dst)[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    if (!live) return;
    uint16_t* dst = reinterpret_cast<uint16_t*>(y) + (r * (int64_t)nbc * kBlock + (int64_t)cb * kBlock + q * 8);
    uint4 w;
    if constexpr (YL == PE_XTF_BF16) {
      w.x = f2bf_bits(v[0]) | ((uint32_t)f2bf_bits(v[1]) << 16);
      w.y = f2bf_bits(v[2]) | ((uint32_t)f2bf_bits(v[3]) << 16);
      w.z = f2bf_bits(v[4]) | ((uint32_t)f2bf_bits(v[5]) << 16);
      w.w = f2bf_bits(v[6]) | ((uint32_t)f2bf_bits(v[7]) << 16);
    } else {
      w.x = pack_h2(v[0], v[1]); w.y = pack_h2(v[2], v[3]);
      w.z = pack_h2(v[4], v[5]); w.w = pack_h2(v[6], v[7]);
    }
    *reinterpret_cast<uint4*>(dst) = w;
  }
}

template <int XDT>
static int launch_fwht(const void* x, int64_t rows, int nbc, int64_t ldx, void* y, int yl,
                       hipStream_t st) {
  const int64_t groups = rows * (int64_t)nbc;
  const dim3 grid((unsigned)((groups + 15) / 16)), block(256);
  switch (yl) {
    case PE_XTF_F32: fwht128_kernel<XDT, PE_XTF_F32><<<grid, block, 0, st>>>(x, y, rows, nbc, ldx); break;
    case PE_XTF_F16: fwht128_kernel<XDT, PE_XTF_F16><<<grid, block, 0, st>>>(x, y, rows, nbc, ldx); break;
    case PE_XTF_PAIR_F16: fwht128_kernel<XDT, PE_XTF_PAIR_F16><<<grid, block, 0, st>>>(x, y, rows, nbc, ldx); break;
    case PE_XTF_BF16: fwht128_kernel<XDT, PE_XTF_BF16><<<grid, block, 0, st>>>(x, y, rows, nbc, ldx); break;
    default: return PE_ERR_DTYPE;
  }
  return launch_status();
}

int fwht128(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx, void* y,
            int y_layout, hipStream_t st) {
  if (!x || !y) return PE_ERR_NULL;
  if (rows < 0 || cols <= 0 || cols % kBlock || ldx < cols) return PE_ERR_DIMS;
  if (rows == 0) return PE_OK;
  // grid = ceil(rows*nb/16) workgroups of 256 lanes; keep the lane count < 2^32.
  if (cols / kBlock > (int64_t)INT32_MAX || rows * (cols / kBlock) > (int64_t(1) << 26)) return PE_ERR_DIMS;
  if (!aligned16(x) || !aligned16(y)) return PE_ERR_ALIGN;
  const int esz = x_dtype == PE_DTYPE_F32 ? 4 : 2;
  if ((ldx * esz) % 16) return PE_ERR_ALIGN;
  const int nbc = (int)(cols / kBlock);
  switch (x_dtype) {
    case PE_DTYPE_F16: return launch_fwht<PE_DTYPE_F16>(x, rows, nbc, ldx, y, y_layout, st);
    case PE_DTYPE_BF16: return launch_fwht<PE_DTYPE_BF16>(x, rows, nbc, ldx, y, y_layout, st);
    case PE_DTYPE_F32: return launch_fwht<PE_DTYPE_F32>(x, rows, nbc, ldx, y, y_layout, st);
    default: return PE_ERR_DTYPE;
  }
}

// Already-transformed fp32 activations (natural layout) -> pair f16, no
// transform: the input of the reference API's batched polar_matmul.
int repack_pair(const float* x, int64_t rows, int64_t cols, void* y, hipStream_t st) {
  if (!x || !y) return PE_ERR_NULL;
  if (rows < 0 || cols <= 0 || cols % kBlock || rows * (cols / kBlock) > (int64_t(1) << 26)) return PE_ERR_DIMS;
  if (!aligned16(x) || !aligned16(y)) return PE_ERR_ALIGN;
  if (rows == 0) return PE_OK;
  const int nbc = (int)(cols / kBlock);
  const int64_t groups = rows * (int64_t)nbc;
  fwht128_kernel<PE_DTYPE_F32, PE_XTF_PAIR_F16, false>
      <<<dim3((unsigned)((groups + 15) / 16)), dim3(256), 0, st>>>(x, y, rows, nbc, cols);
  return launch_status();
}

// ---------------------------------------------------------------------------
// Whole-row FWHT of any power-of-two length n <= 2^15: the reference's
// fwht_butterfly (kernels/fwht.py:160-190), stages h = 1, 2, 4, ..., n/2
// pairing (a, b) -> (a + b, a - b) over the whole last dimension, then a
// division by sqrt(n). The rows of one workgroup sit in LDS as fp32 (n or, for
// short rows, 2048 elements: several rows), every stage is one pass of the
// 256 lanes over the pairs, and the result is rounded once to the output type.
// ---------------------------------------------------------------------------
constexpr int kPow2MaxLog = 15;
constexpr int kPow2WgElems = 2048;  // elements per workgroup for rows shorter than this

__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dt) {
  if (dt == PE_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
  const uint16_t b = reinterpret_cast<const uint16_t*>(p)[i];
  return dt == PE_DTYPE_BF16 ? bf2f(b) : h2f(b);
}

__global__ __launch_bounds__(256) void fwht_pow2_kernel(const void* x, int xdt, void* y, int ydt,
                                                        int64_t rows, int logn, int64_t ldx,
                                                        float sqrt_n) {
  extern __shared__ float s[];
  const int n = 1 << logn;
  const int rpw = n >= kPow2WgElems ? 1 : kPow2WgElems >> logn;  // rows per workgroup
  const int64_t r0 = (int64_t)blockIdx.x * rpw;
  const int nr = (int)(rows - r0 < rpw ? rows - r0 : rpw);
  const int elems = nr << logn;
  for (int i = threadIdx.x; i < elems; i += blockDim.x) {
    const int rr = i >> logn, c = i & (n - 1);
    s[i] = load_elem(x, (r0 + rr) * ldx + c, xdt);
  }
  __syncthreads();
  for (int lh = 0; lh < logn; ++lh) {
    const int h = 1 << lh;
    for (int p = threadIdx.x; p < (elems >> 1); p += blockDim.x) {
      const int i = ((p >> lh) << (lh + 1)) | (p & (h - 1));
      const float a = s[i], b = s[i + h];
      s[i] = a + b;
      s[i + h] = a - b;
    }
    __syncthreads();
  }
  const int64_t base = r0 << logn;  // output rows are contiguous
  for (int i = threadIdx.x; i < elems; i += blockDim.x) {
    const float v = s[i] / sqrt_n;
    if (ydt == PE_DTYPE_F32) reinterpret_cast<float*>(y)[base + i] = v;
    else if (ydt == PE_DTYPE_BF16) reinterpret_cast<uint16_t*>(y)[base + i] = f2bf_bits(v);
    else reinterpret_cast<uint16_t*>(y)[base + i] = f2h_bits(v);
  }
}

int fwht_pow2(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t ldx, void* y,
              int y_dtype, hipStream_t st) {
  if (!x || !y) return PE_ERR_NULL;
  if (x_dtype < PE_DTYPE_F16 || x_dtype > PE_DTYPE_F32 || y_dtype < PE_DTYPE_F16 ||
      y_dtype > PE_DTYPE_F32)
    return PE_ERR_DTYPE;
  if (rows < 0 || n < 1 || (n & (n - 1)) || n > (int64_t(1) << kPow2MaxLog) || ldx < n)
    return PE_ERR_DIMS;
  if (rows == 0) return PE_OK;
  int logn = 0;
  while ((int64_t(1) << logn) < n) ++logn;
  const int rpw = n >= kPow2WgElems ? 1 : kPow2WgElems >> logn;
  const int64_t grid = (rows + rpw - 1) / rpw;
  if (grid > INT32_MAX) return PE_ERR_DIMS;
  const size_t lds = (size_t)(n >= kPow2WgElems ? n : kPow2WgElems) * sizeof(float);
  static const bool attr_ok = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(fwht_pow2_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  const float sqrt_n = (float)std::sqrt((double)n);
  fwht_pow2_kernel<<<dim3((unsigned)grid), dim3(256), lds, st>>>(x, x_dtype, y, y_dtype, rows, logn,
                                                                 ldx, sqrt_n);
  return launch_status();
}

}  // namespace pe

extern "C" int pe_fwht128(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx,
                          void* y, int y_layout, void* stream) {
  return pe::fwht128(x, x_dtype, rows, cols, ldx, y, y_layout, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pe_fwht_pow2(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t ldx,
                            void* y, int y_dtype, void* stream) {
  return pe::fwht_pow2(x, x_dtype, rows, n, ldx, y, y_dtype, reinterpret_cast<hipStream_t>(stream));
}
