// PolarQuant KV-cache compression on gfx950: quantize K/V vectors into
// packed codes + bf16 norms, and expand them back to bf16.
//
// Replaces PolarKVQuantizer.quantize / dequantize (polarengine_vllm/kv_cache/
// cache.py:201-256) and the hybrid torch/Triton ops of kv_cache/
// triton_kernels.py:139-228: per vector of head_dim D (64, 128 or 256), L2 norm
// clamped at 1e-10, unit vector times the unnormalised Hadamard transform (=
// (x / |x|) @ H * sqrt(D)), code = first index of the nearest of the 2^nbits
// KV centroids, codes packed MSB-first exactly as BitPacker does
// (cache.py:98-128): 2 bits -> c0<<6|c1<<4|c2<<2|c3, 3 bits -> 8 codes in 3
// bytes, 4 bits -> c[2i]<<4 | c[2i+1]; norms stored as bf16. Dequantize:
// (ct[code] / sqrt(D)) @ H * norm, cast to bf16.
//
// One vector per D/8 lanes, 8 consecutive positions per lane; the transform
// is the in-lane butterfly plus DPP/swizzle exchanges (inside one 32-lane
// half), so one wave handles 8, 4 or 2 vectors (D = 64, 128, 256).

#include "pe_internal.h"

namespace pe {

template <int L>  // lanes per vector: 8, 16 or 32 (D = 64, 128, 256)
__device__ __forceinline__ void fwht_lanes_raw(float v[8], int q) {
#pragma unroll
  for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if ((i & h) == 0) {
        const float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
    }
  }
  fwht_xstage<1>(v, q);
  fwht_xstage<2>(v, q);
  fwht_xstage<4>(v, q);
  if constexpr (L >= 16) fwht_xstage<8>(v, q);
  if constexpr (L >= 32) fwht_xstage<16>(v, q);  // ds_swizzle inside 32 lanes
}

template <int L>
__device__ __forceinline__ float lanes_sum(float s) {
  s += lane_xor<1>(s);
  s += lane_xor<2>(s);
  s += lane_xor<4>(s);
  if constexpr (L >= 16) s += lane_xor<8>(s);
  if constexpr (L >= 32) s += lane_xor<16>(s);
  return s;
}

template <int DT>
__device__ __forceinline__ float kv_load(const void* x, int64_t i) {
  if constexpr (DT == PE_DTYPE_F16) return h2f(reinterpret_cast<const uint16_t*>(x)[i]);
  else if constexpr (DT == PE_DTYPE_BF16) return bf2f(reinterpret_cast<const uint16_t*>(x)[i]);
  else return reinterpret_cast<const float*>(x)[i];
}

// 8 codes of one lane -> NB bytes (the lane's share of the row), MSB first
template <int NB>
__device__ __forceinline__ void kv_pack8(const uint32_t (&c)[8], uint8_t (&b)[NB]) {
  if constexpr (NB == 2) {
    b[0] = (uint8_t)((c[0] << 6) | (c[1] << 4) | (c[2] << 2) | c[3]);
    b[1] = (uint8_t)((c[4] << 6) | (c[5] << 4) | (c[6] << 2) | c[7]);
  } else if constexpr (NB == 3) {
    b[0] = (uint8_t)((c[0] << 5) | (c[1] << 2) | (c[2] >> 1));
    b[1] = (uint8_t)(((c[2] & 1) << 7) | (c[3] << 4) | (c[4] << 1) | (c[5] >> 2));
    b[2] = (uint8_t)(((c[5] & 3) << 6) | (c[6] << 3) | c[7]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = (uint8_t)((c[2 * i] << 4) | c[2 * i + 1]);
  }
}

template <int NB>
__device__ __forceinline__ void kv_unpack8(const uint8_t (&b)[NB], uint32_t (&c)[8]) {
  if constexpr (NB == 2) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      c[4 * j] = (b[j] >> 6) & 3;
      c[4 * j + 1] = (b[j] >> 4) & 3;
      c[4 * j + 2] = (b[j] >> 2) & 3;
      c[4 * j + 3] = b[j] & 3;
    }
  } else if constexpr (NB == 3) {
    c[0] = (b[0] >> 5) & 7;
    c[1] = (b[0] >> 2) & 7;
    c[2] = ((b[0] & 3) << 1) | ((b[1] >> 7) & 1);
    c[3] = (b[1] >> 4) & 7;
    c[4] = (b[1] >> 1) & 7;
    c[5] = ((b[1] & 1) << 2) | ((b[2] >> 6) & 3);
    c[6] = (b[2] >> 3) & 7;
    c[7] = b[2] & 7;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[2 * i] = (b[i] >> 4) & 15;
      c[2 * i + 1] = b[i] & 15;
    }
  }
}

// LDS table of the cell count (see kv_quantize_kernel)
template <int NL>
struct KvCells {
  uint32_t* lo;   // [64] midpoints below cell c's lower bound (c - 32) w
  float* mid;     // [64] the midpoint in cell c, divided by w; +inf if none
  float inv_w;    // 1 / w = 2^-e
};

// Builds the table in LDS (the whole workgroup: it ends in a barrier) and
// returns whether the midpoints fit: ascending, finite, at most one per cell.
template <int NL>
__device__ bool kv_cells_setup(const float (&mid)[NL - 1], KvCells<NL>& t) {
  __shared__ uint32_t lo[64];
  __shared__ float tm[64];
  float amax = 0.f, gmin = INFINITY;
  bool ok = true;
#pragma unroll
  for (int l = 0; l < NL - 1; ++l) {
    ok = ok && (mid[l] == mid[l]) && fabsf(mid[l]) < 1e30f;
    amax = fmaxf(amax, fabsf(mid[l]));
    if (l + 1 < NL - 1) gmin = fminf(gmin, mid[l + 1] - mid[l]);
  }
  // smallest power of two w with 31 w >= amax
  int e = 0;
  (void)frexpf(amax / 31.f, &e);
  float w = ldexpf(1.f, e);
  if (31.f * w < amax) w *= 2.f;
  ok = ok && amax > 0.f && w <= gmin && w >= 0x1p-100f;
  t.lo = lo;
  t.mid = tm;
  t.inv_w = 1.f / w;  // exact: a power of two
  if (ok && threadIdx.x < 64) {
    const float b = (float)((int)threadIdx.x - 32) * w;  // exact
    uint32_t n = 0;
    float m = INFINITY;
#pragma unroll
    for (int l = 0; l < NL - 1; ++l) {
      n += mid[l] < b ? 1u : 0u;
      if (mid[l] >= b && (threadIdx.x == 63 || mid[l] < b + w)) m = mid[l] * t.inv_w;
    }
    lo[threadIdx.x] = threadIdx.x == 0 ? 0u : n;
    tm[threadIdx.x] = m;
  }
  __syncthreads();
  return ok;
}

// Grid-stride: each workgroup builds the cell table once, then quantizes
// 256 / (D / 8) vectors per step.
template <int D, int NBITS, int DT>
__global__ __launch_bounds__(256) void kv_quantize_kernel(const void* __restrict__ x, int64_t ldx,
                                                          int64_t n_vec,
                                                          const float* __restrict__ ct,
                                                          uint8_t* __restrict__ packed,
                                                          uint16_t* __restrict__ norms) {
  constexpr int L = D / 8;
  constexpr int VPS = 256 / L;        // vectors per workgroup step
  constexpr int RB = D * NBITS / 8;  // packed bytes per vector
  const int q = threadIdx.x & (L - 1);
  // First-index argmin of |r - ct[l]| over ascending centroids = the number
  // of midpoints (ct[l] + ct[l+1]) / 2 strictly below r (a tie at a midpoint
  // keeps the lower index).
  constexpr int NL = 1 << NBITS;
  float mid[NL - 1];
#pragma unroll
  for (int l = 0; l < NL - 1; ++l) mid[l] = (ct[l] + ct[l + 1]) * 0.5f;
  // The count by cell: cells of width w = 2^e over [-32 w, 32 w), w chosen
  // so that every midpoint lies in [-31 w, 31 w] and no cell holds two
  // (uniform per workgroup). Scaling by a power of two is exact, so
  // t = r / w computed as v * (inv / w) equals round(v * inv) / w, its floor
  // is r's cell exactly, and r > m <=> t > m / w. Entry c holds the number
  // of midpoints below the cell and the cell's own midpoint / w (+inf if
  // none): one compare per element instead of NL - 1.
  KvCells<NL> cells;
  const bool by_cell = kv_cells_setup<NL>(mid, cells);
  for (int64_t v0 = (int64_t)blockIdx.x * VPS; v0 < n_vec; v0 += (int64_t)gridDim.x * VPS) {
    const int64_t vec = v0 + threadIdx.x / L;
    const bool live = vec < n_vec;
    const int64_t vr = live ? vec : 0;  // dead groups work on vector 0, store nothing
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = kv_load<DT>(x, vr * ldx + 8 * q + i);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(v[i], v[i], ss);
    ss = lanes_sum<L>(ss);
    float nrm = __builtin_sqrtf(ss);
    nrm = nrm > 1e-10f ? nrm : 1e-10f;
    // rotated = (x / |x|) @ H * sqrt(D) = (raw transform of x) / |x|: the
    // transform runs on x and one reciprocal scales the result
    fwht_lanes_raw<L>(v, q);
    const float inv = 1.f / nrm;
    uint32_t c[8];
    if (by_cell) {  // uniform
      const float s = inv * cells.inv_w;
      // the cell from t clamped to [-32, 31] (IEEE max: a NaN goes to cell
      // 0, where it compares false: code 0, as the count gives); the compare
      // on t itself. All eight table reads go out before the first compare.
      float t[8], md[8];
      uint32_t lo[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        t[i] = v[i] * s;
        const int cell = (int)__builtin_floorf(fminf(fmaxf(t[i], -32.f), 31.f)) + 32;
        lo[i] = cells.lo[cell];
        md[i] = cells.mid[cell];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = lo[i] + (t[i] > md[i] ? 1u : 0u);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float r = v[i] * inv;
        uint32_t k = 0;
#pragma unroll
        for (int l = 0; l < NL - 1; ++l) k += r > mid[l] ? 1u : 0u;
        c[i] = k;
      }
    }
    if (live) {
      uint8_t b[NBITS];
      kv_pack8<NBITS>(c, b);
      uint8_t* dst = packed + vec * RB + q * NBITS;
#pragma unroll
      for (int i = 0; i < NBITS; ++i) dst[i] = b[i];
      if (q == 0) norms[vec] = f2bf_bits(nrm);
    }
  }
}

// ---------------------------------------------------------------------------
// D = 128 from bf16 or fp16: the transform on the matrix cores. One wave
// quantizes 32 vectors per step, y^T = H x^T as 4 x 8 MFMAs 32x32x16 (A = a
// 32 x 16 block of H, B = 16 positions x 32 vectors of x: lane l loads 8
// consecutive positions of vector l % 32, one 16-byte load). Products of
// bf16 / fp16 values by +-1 are exact and the sums fp32, as in the butterfly
// (in another order). The sign blocks come from four register sets:
// H[r][c] = (-1)^popcount(r & c), and for r = 32 mb + m (m = the lane's row)
// and c = 16 kt + 8 h + j (h = lane / 32) the sign is the lane's base
// F[j] = (-1)^(popcount(m & j & 7) + m3 h), times (-1)^(m4 kt0), times
// (-1)^(mb0 kt1 + mb1 kt2), a compile-time constant: the block is +-F for
// even kt and +-G, G = (-1)^m4 F, for odd kt. The accumulators come out with
// lane l holding positions 32 mb + 8 (e / 4) + 4 h + e % 4 of vector l % 32:
// half of every 8-position code group, the other half in lane l ^ 32.
// ---------------------------------------------------------------------------
template <int DT>
struct KvMfma {  // fp16
  static constexpr uint32_t kOne2 = 0x3C003C00u;
  static __device__ __forceinline__ float16v mma(u32x4v a, u32x4v b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8v, a),
                                                 __builtin_bit_cast(half8v, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return h2f((uint16_t)(w & 0xffff)); }
  static __device__ __forceinline__ float hi(uint32_t w) { return h2f((uint16_t)(w >> 16)); }
};
template <>
struct KvMfma<PE_DTYPE_BF16> {
  static constexpr uint32_t kOne2 = 0x3F803F80u;
  static __device__ __forceinline__ float16v mma(u32x4v a, u32x4v b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, a),
                                                  __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
};

// MFMAs per step: 4 m-blocks x 8 k-steps
constexpr int kKvmVecs = 32;  // vectors per wave step

template <int NBITS, int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void kv_quantize_mfma_kernel(const void* __restrict__ x, int64_t ldx, int64_t n_vec,
                             const float* __restrict__ ct, uint8_t* __restrict__ packed,
                             uint16_t* __restrict__ norms) {
  using K = KvMfma<DT>;
  constexpr int D = 128, RB = D * NBITS / 8, NL = 1 << NBITS;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar step bases
  const int n = lane & 31, h = lane >> 5;
  float mid[NL - 1];
#pragma unroll
  for (int l = 0; l < NL - 1; ++l) mid[l] = (ct[l] + ct[l + 1]) * 0.5f;
  KvCells<NL> cells;
  const bool by_cell = kv_cells_setup<NL>(mid, cells);
  // sign blocks F, -F, G, -G (pairs of 16-bit +-1)
  u32x4v F, nF, G, nG;
  {
    const uint32_t hb = (uint32_t)(((n >> 3) & 1) & h);
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      const uint32_t s0 = ((uint32_t)__builtin_popcount(n & (2 * jp) & 7) + hb) & 1u;
      const uint32_t s1 = ((uint32_t)__builtin_popcount(n & (2 * jp + 1) & 7) + hb) & 1u;
      F[jp] = K::kOne2 | (s0 << 15) | (s1 << 31);
      nF[jp] = F[jp] ^ 0x80008000u;
    }
    const bool m4 = (n >> 4) & 1;
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      G[jp] = m4 ? nF[jp] : F[jp];
      nG[jp] = m4 ? F[jp] : nF[jp];
    }
  }
  const int64_t stride = (int64_t)gridDim.x * 4 * kKvmVecs;
  for (int64_t v0 = ((int64_t)blockIdx.x * 4 + wave) * kKvmVecs; v0 < n_vec; v0 += stride) {
    const int64_t vec = v0 + n;
    const bool live = vec < n_vec;
    const int64_t vr = live ? vec : n_vec - 1;  // dead lanes repeat the last vector, store nothing
    const char* src = reinterpret_cast<const char*>(x) + (vr * ldx + 8 * h) * 2;
    u32x4v b[8];
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) b[kt] = *reinterpret_cast<const u32x4v*>(src + kt * 32);
    // |x|: this lane's 64 positions, then the other half from lane ^ 32
    float ss = 0.f;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float a0 = K::lo(b[kt][w]), a1 = K::hi(b[kt][w]);
        ss = __builtin_fmaf(a0, a0, ss);
        ss = __builtin_fmaf(a1, a1, ss);
      }
    ss += __shfl_xor(ss, 32, 64);
    float nrm = __builtin_sqrtf(ss);
    nrm = nrm > 1e-10f ? nrm : 1e-10f;
    const float inv = 1.f / nrm;
    // m-blocks in pairs (two accumulators live); each pair's codes before
    // the next pair's MFMAs. half[g]: the 4 codes of group g (positions
    // 8 g + 4 h + 0..3)
    uint32_t half[16];
    const float s = inv * cells.inv_w;
#pragma unroll
    for (int mp = 0; mp < 2; ++mp) {
      float16v acc[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[u][e] = 0.f;
#pragma unroll
      for (int kt = 0; kt < 8; ++kt)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int mb = 2 * mp + u;
          const bool neg = (((mb & 1) & (kt >> 1)) ^ ((mb >> 1) & (kt >> 2))) & 1;
          const u32x4v a = (kt & 1) ? (neg ? nG : G) : (neg ? nF : F);
          acc[u] = K::mma(a, b[kt], acc[u]);
        }
      uint32_t k[2][16];
      if (by_cell) {  // uniform
        // every table read of an m-block issued before the first compare
        // (read, wait, compare per element left each read's latency exposed)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          float t[16], md[16];
          uint32_t lo[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            t[e] = acc[u][e] * s;
            const int cell = (int)__builtin_floorf(fminf(fmaxf(t[e], -32.f), 31.f)) + 32;
            lo[e] = cells.lo[cell];
            md[e] = cells.mid[cell];
          }
#pragma unroll
          for (int e = 0; e < 16; ++e) k[u][e] = lo[e] + (t[e] > md[e] ? 1u : 0u);
        }
      } else {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const float r = acc[u][e] * inv;
            uint32_t c = 0;
#pragma unroll
            for (int l = 0; l < NL - 1; ++l) c += r > mid[l] ? 1u : 0u;
            k[u][e] = c;
          }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          uint32_t hv = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) hv |= k[u][4 * jj + i] << (NBITS * (3 - i));
          half[4 * (2 * mp + u) + jj] = hv;
        }
    }
    // whole groups: lane h = 0 keeps groups 0..7, h = 1 groups 8..15
    uint32_t full[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const uint32_t send = h ? half[g] : half[8 + g];
      const uint32_t recv = (uint32_t)__shfl_xor((int)send, 32, 64);
      full[g] = h ? ((recv << (4 * NBITS)) | half[8 + g]) : ((half[g] << (4 * NBITS)) | recv);
    }
    // MSB-first bytes of the 8 groups: 8 NBITS bytes at byte 8 NBITS h of the row
    uint32_t wds[2 * NBITS];
#pragma unroll
    for (int k = 0; k < 2 * NBITS; ++k) {
      uint32_t wd = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int by = 4 * k + q, g = by / NBITS, bi = by % NBITS;
        wd |= ((full[g] >> (8 * (NBITS - 1 - bi))) & 0xffu) << (8 * q);
      }
      wds[k] = wd;
    }
    if (live) {
      uint2* dst = reinterpret_cast<uint2*>(packed + vec * RB + h * (8 * NBITS));
#pragma unroll
      for (int k = 0; k < NBITS; ++k) dst[k] = make_uint2(wds[2 * k], wds[2 * k + 1]);
      if (h == 0) norms[vec] = f2bf_bits(nrm);
    }
  }
}

// bf16 pair; the conversion from float is gfx950's round-to-nearest-even
// v_cvt_pk_bf16_f32
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Expansion at D = 128 on the matrix cores: x^T = H v^T with
// v = ct[code] / sqrt(D) / sqrt(D) (fp32, split into an fp16 hi + lo pair so
// the two products keep fp32 accuracy), then x * norm in bf16. The
// B operand (8 consecutive positions of one vector per lane) comes from the
// lane's 8-code group: group 2 kt + h of the packed row, read as one 8-byte
// window and a per-lane shift, the values by ds_bpermute from the lanes
// holding the codebook. The compile-time part of the sign, (-1)^(mb0 kt1 +
// mb1 kt2), is a 4-point Hadamard over the m-blocks: four partial sums
// S[kt1 + 2 kt2] = sum over kt0 of (F or G) x B(kt) take 16 MFMAs per 32
// vectors (8 k-steps x hi/lo), and D[mb] = sum (-1)^(mb0 a + mb1 b) S[a + 2b]
// two add stages.
// ---------------------------------------------------------------------------
template <int NBITS>
__device__ __forceinline__ uint32_t kv_group(const uint32_t (&d)[4 * NBITS], int kt, int h) {
  // bytes [(2 kt + h) NBITS, + NBITS) of the row, MSB first
  constexpr int W = 4 * NBITS;
  const int off0 = 2 * kt * NBITS, w0 = off0 / 4;
  const uint64_t win = (uint64_t)d[w0] | ((uint64_t)(w0 + 1 < W ? d[w0 + 1] : 0u) << 32);
  const uint32_t b = (uint32_t)(win >> (8 * (off0 % 4) + 8 * NBITS * h));
  if constexpr (NBITS == 2) return ((b & 0xffu) << 8) | ((b >> 8) & 0xffu);
  else if constexpr (NBITS == 3) return ((b & 0xffu) << 16) | (b & 0xff00u) | ((b >> 16) & 0xffu);
  else return __builtin_bswap32(b);
}

constexpr int kKvtRow = 66;  // dwords per LDS tile row: 256 bytes + 8 of padding
constexpr int kKvBufFlags = 0x00020000;  // raw buffer, 32-bit data format (dword 3 of the resource)

template <int NBITS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void kv_dequantize_mfma_kernel(const uint8_t* __restrict__ packed,
                               const uint16_t* __restrict__ norms, int64_t n_vec,
                               const float* __restrict__ ct, uint16_t* __restrict__ out,
                               int64_t ldo) {
  constexpr int RB = 128 * NBITS / 8, NL = 1 << NBITS;
  __shared__ uint32_t kvt[4 * kKvmVecs * kKvtRow];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar step bases
  const int n = lane & 31, h = lane >> 5;
  // lane j holds (hi, lo) of the value of code j mod 2^NBITS as two fp16
  uint32_t tv;
  {
    // ct / sqrt(D) as the reference divides, times 1 / sqrt(D) of the
    // normalised transform (one product per output left: the norm)
    const float val = ct[lane & (NL - 1)] / 11.313708498984761f * kInvSqrt128;
    const _Float16 vh = (_Float16)val;
    const _Float16 vl = (_Float16)(val - (float)vh);
    tv = (uint32_t)__builtin_bit_cast(uint16_t, vh) | ((uint32_t)__builtin_bit_cast(uint16_t, vl) << 16);
  }
  u32x4v F, G;
  {
    const uint32_t hb = (uint32_t)(((n >> 3) & 1) & h);
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      const uint32_t s0 = ((uint32_t)__builtin_popcount(n & (2 * jp) & 7) + hb) & 1u;
      const uint32_t s1 = ((uint32_t)__builtin_popcount(n & (2 * jp + 1) & 7) + hb) & 1u;
      F[jp] = 0x3C003C00u | (s0 << 15) | (s1 << 31);
    }
    const uint32_t m4 = ((n >> 4) & 1) ? 0x80008000u : 0u;
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) G[jp] = F[jp] ^ m4;
  }
  // this lane's store offset within a step's rows: row lane / 16 of each
  // group of four, 16-byte chunk lane % 16
  const uint32_t o_voff = (uint32_t)(((lane >> 4) * ldo + 8 * (lane & 15)) * 2);
  const int64_t stride = (int64_t)gridDim.x * 4 * kKvmVecs;
  for (int64_t v0 = ((int64_t)blockIdx.x * 4 + wave) * kKvmVecs; v0 < n_vec; v0 += stride) {
    const int64_t vr = v0 + n < n_vec ? v0 + n : n_vec - 1;  // past the end: the last vector
    uint32_t d[4 * NBITS];
    {
      const u32x4v* src = reinterpret_cast<const u32x4v*>(packed + vr * RB);
#pragma unroll
      for (int i = 0; i < NBITS; ++i) {
        const u32x4v q = src[i];
#pragma unroll
        for (int k = 0; k < 4; ++k) d[4 * i + k] = q[k];
      }
    }
    const float nrm = bf2f(norms[vr]);
    float16v S[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 16; ++e) S[u][e] = 0.f;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
      const uint32_t grp = kv_group<NBITS>(d, kt, h);
      uint32_t w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // code j at address bits 2.. (ds_bpermute takes lane = bits 2..7);
        // higher codes left in bits 2 + NBITS..7 select the same value, the
        // table repeating every 2^NBITS lanes
        const int s2 = NBITS * (7 - j) - 2;
        const uint32_t addr = s2 >= 0 ? grp >> (s2 >= 0 ? s2 : 0) : grp << (s2 < 0 ? -s2 : 0);
        w[j] = (uint32_t)__builtin_amdgcn_ds_bpermute((int)addr, (int)tv);
      }
      u32x4v bh, bl;
#pragma unroll
      for (int jp = 0; jp < 4; ++jp) {
        bh[jp] = __builtin_amdgcn_perm(w[2 * jp + 1], w[2 * jp], 0x05040100u);
        bl[jp] = __builtin_amdgcn_perm(w[2 * jp + 1], w[2 * jp], 0x07060302u);
      }
      const u32x4v a = (kt & 1) ? G : F;
      const int ab = (kt >> 1) & 3;  // kt1 + 2 kt2
      S[ab] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8v, a),
                                                     __builtin_bit_cast(half8v, bh), S[ab], 0, 0, 0);
      S[ab] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8v, a),
                                                     __builtin_bit_cast(half8v, bl), S[ab], 0, 0, 0);
    }
    // D[0] = S0 + S1 + S2 + S3, D[1] = S0 - S1 + S2 - S3, D[2] = S0 + S1 - S2 - S3,
    // D[3] = S0 - S1 - S2 + S3; lane l holds positions 32 mb + 8 (e / 4) + 4 h + e % 4
    // of vector l % 32. The wave's 32 x 256-byte tile goes through LDS (rows
    // padded by 8 bytes so the 8-byte writes of 32 rows hit distinct banks)
    // and leaves as 16-byte stores, 16 lanes per row.
    uint32_t* tile = kvt + wave * (kKvmVecs * kKvtRow);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * jj + i;
          const float t0 = S[0][e] + S[1][e], t1 = S[0][e] - S[1][e];
          const float t2 = S[2][e] + S[3][e], t3 = S[2][e] - S[3][e];
          const float yy = mb == 0 ? t0 + t2 : mb == 1 ? t1 + t3 : mb == 2 ? t0 - t2 : t1 - t3;
          y[i] = yy * nrm;
        }
        bf16x2v o0, o1;
        o0.x = (__bf16)y[0];
        o0.y = (__bf16)y[1];
        o1.x = (__bf16)y[2];
        o1.y = (__bf16)y[3];
        *reinterpret_cast<uint2*>(tile + n * kKvtRow + 16 * mb + 4 * jj + 2 * h) =
            make_uint2(__builtin_bit_cast(uint32_t, o0), __builtin_bit_cast(uint32_t, o1));
      }
    }
    // the step's rows through a buffer resource whose extent ends at the
    // last vector: stores past it are dropped by the hardware, so each
    // address is the lane's offset plus a scalar row offset (host: ldo <
    // 2^24, so every offset fits 31 bits)
    const int64_t rows = n_vec - v0 < kKvmVecs ? n_vec - v0 : kKvmVecs;
    const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
        out + v0 * ldo, (short)0, (int)(rows * ldo * 2), kKvBufFlags);
#pragma unroll
    for (int i = 0; i < kKvmVecs / 4; ++i) {
      const int r = 4 * i + (lane >> 4), c = lane & 15;
      const u32x4v q = *reinterpret_cast<const u32x4v*>(tile + r * kKvtRow + 4 * c);
      __builtin_amdgcn_raw_buffer_store_b128(q, ors, o_voff, (int)(4 * i * ldo * 2), 0);
    }
  }
}

template <int D, int NBITS>
__global__ __launch_bounds__(256) void kv_dequantize_kernel(const uint8_t* __restrict__ packed,
                                                            const uint16_t* __restrict__ norms,
                                                            int64_t n_vec,
                                                            const float* __restrict__ ct,
                                                            uint16_t* __restrict__ out,
                                                            int64_t ldo) {
  constexpr int L = D / 8;
  constexpr int RB = D * NBITS / 8;
  const int q = threadIdx.x & (L - 1);
  const int64_t vec = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / L;
  const bool live = vec < n_vec;
  const int64_t vr = live ? vec : 0;
  uint8_t b[NBITS];
  const uint8_t* src = packed + vr * RB + q * NBITS;
#pragma unroll
  for (int i = 0; i < NBITS; ++i) b[i] = src[i];
  uint32_t c[8];
  kv_unpack8<NBITS>(b, c);
  // (ct[c] / sqrt(D)) @ H: the division as the reference does it (fp32 by
  // fp32(sqrt(D))), the normalised transform as the raw one times 1/sqrt(D).
  // Lane j holds ct[j mod 2^NBITS] / sqrt(D); a code's value is fetched from
  // lane `code` with ds_bpermute (every lane of the wave takes part).
  const float sq = D == 64 ? 8.f : D == 128 ? 11.313708498984761f : 16.f;
  const float inv = D == 64 ? 0.125f : D == 128 ? kInvSqrt128 : 0.0625f;
  const int lane = threadIdx.x & 63;
  const int ctv = __builtin_bit_cast(int, ct[lane & ((1 << NBITS) - 1)] / sq);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((int)(c[i] << 2), ctv));
  fwht_lanes_raw<L>(v, q);
  const float nrm = bf2f(norms[vr]);
  if (!live) return;
  bf16x2v o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[i].x = (__bf16)(v[2 * i] * inv * nrm);
    o[i].y = (__bf16)(v[2 * i + 1] * inv * nrm);
  }
  *reinterpret_cast<uint4*>(out + vec * ldo + 8 * q) =
      make_uint4(__builtin_bit_cast(uint32_t, o[0]), __builtin_bit_cast(uint32_t, o[1]),
                 __builtin_bit_cast(uint32_t, o[2]), __builtin_bit_cast(uint32_t, o[3]));
}

// quantize workgroups: at most 8 per CU (grid-stride beyond that)
constexpr int kKvqWgsPerCu = 8;

template <int D, int NBITS>
static int launch_kv_q(const void* x, int dt, int64_t ldx, int64_t n, const float* ct,
                       uint8_t* packed, uint16_t* norms, hipStream_t st) {
  const int64_t steps = (n * (D / 8) + 255) / 256;
  const int64_t cap = (int64_t)num_cus() * kKvqWgsPerCu;
  const unsigned grid = (unsigned)(steps < cap ? steps : cap);
  switch (dt) {
    case PE_DTYPE_BF16: kv_quantize_kernel<D, NBITS, PE_DTYPE_BF16><<<grid, 256, 0, st>>>(x, ldx, n, ct, packed, norms); break;
    case PE_DTYPE_F16: kv_quantize_kernel<D, NBITS, PE_DTYPE_F16><<<grid, 256, 0, st>>>(x, ldx, n, ct, packed, norms); break;
    case PE_DTYPE_F32: kv_quantize_kernel<D, NBITS, PE_DTYPE_F32><<<grid, 256, 0, st>>>(x, ldx, n, ct, packed, norms); break;
    default: return PE_ERR_DTYPE;
  }
  return launch_status();
}

template <int D, int NBITS>
static int launch_kv_d(const uint8_t* packed, const uint16_t* norms, int64_t n, const float* ct,
                       uint16_t* out, int64_t ldo, hipStream_t st) {
  // D = 128 with 16-byte aligned packed rows: the transform on the matrix
  // cores (its buffer stores take 31-bit offsets: ldo < 2^24)
  if (D == 128 && aligned16(packed) && ldo < ((int64_t)1 << 24)) {
    const int64_t steps = (n + 4 * kKvmVecs - 1) / (4 * kKvmVecs);
    const int64_t cap = (int64_t)num_cus() * kKvqWgsPerCu;
    const unsigned g = (unsigned)(steps < cap ? steps : cap);
    kv_dequantize_mfma_kernel<NBITS><<<g, 256, 0, st>>>(packed, norms, n, ct, out, ldo);
    return launch_status();
  }
  const int64_t threads = n * (D / 8);
  const unsigned grid = (unsigned)((threads + 255) / 256);
  kv_dequantize_kernel<D, NBITS><<<grid, 256, 0, st>>>(packed, norms, n, ct, out, ldo);
  return launch_status();
}

template <int NBITS>
static int launch_kv_q_mfma(const void* x, int dt, int64_t ldx, int64_t n, const float* ct,
                            uint8_t* packed, uint16_t* norms, hipStream_t st) {
  const int64_t steps = (n + 4 * kKvmVecs - 1) / (4 * kKvmVecs);
  const int64_t cap = (int64_t)num_cus() * kKvqWgsPerCu;
  const unsigned grid = (unsigned)(steps < cap ? steps : cap);
  if (dt == PE_DTYPE_BF16)
    kv_quantize_mfma_kernel<NBITS, PE_DTYPE_BF16><<<grid, 256, 0, st>>>(x, ldx, n, ct, packed, norms);
  else
    kv_quantize_mfma_kernel<NBITS, PE_DTYPE_F16><<<grid, 256, 0, st>>>(x, ldx, n, ct, packed, norms);
  return launch_status();
}

template <int D>
static int kv_q_bits(int nbits, const void* x, int dt, int64_t ldx, int64_t n, const float* ct,
                     uint8_t* packed, uint16_t* norms, hipStream_t st) {
  // D = 128 from 16-bit input with 16-byte aligned rows and codes: the
  // transform on the matrix cores
  if (D == 128 && (dt == PE_DTYPE_BF16 || dt == PE_DTYPE_F16) && aligned16(x) &&
      (ldx * 2) % 16 == 0 && aligned16(packed)) {
    switch (nbits) {
      case 2: return launch_kv_q_mfma<2>(x, dt, ldx, n, ct, packed, norms, st);
      case 3: return launch_kv_q_mfma<3>(x, dt, ldx, n, ct, packed, norms, st);
      case 4: return launch_kv_q_mfma<4>(x, dt, ldx, n, ct, packed, norms, st);
      default: return PE_ERR_BITS;
    }
  }
  switch (nbits) {
    case 2: return launch_kv_q<D, 2>(x, dt, ldx, n, ct, packed, norms, st);
    case 3: return launch_kv_q<D, 3>(x, dt, ldx, n, ct, packed, norms, st);
    case 4: return launch_kv_q<D, 4>(x, dt, ldx, n, ct, packed, norms, st);
    default: return PE_ERR_BITS;
  }
}

template <int D>
static int kv_d_bits(int nbits, const uint8_t* packed, const uint16_t* norms, int64_t n,
                     const float* ct, uint16_t* out, int64_t ldo, hipStream_t st) {
  switch (nbits) {
    case 2: return launch_kv_d<D, 2>(packed, norms, n, ct, out, ldo, st);
    case 3: return launch_kv_d<D, 3>(packed, norms, n, ct, out, ldo, st);
    case 4: return launch_kv_d<D, 4>(packed, norms, n, ct, out, ldo, st);
    default: return PE_ERR_BITS;
  }
}

}  // namespace pe

extern "C" int pe_kv_quantize(const void* x, int x_dtype, int64_t n_vec, int head_dim,
                              int64_t ldx, const float* ct, int nbits, uint8_t* packed,
                              uint16_t* norms_bf16, void* stream) {
  if (!x || !ct || !packed || !norms_bf16) return PE_ERR_NULL;
  if (n_vec < 0 || (head_dim != 64 && head_dim != 128 && head_dim != 256) || ldx < head_dim)
    return PE_ERR_DIMS;
  if (nbits < 2 || nbits > 4) return PE_ERR_BITS;
  if (n_vec == 0) return PE_OK;
  if (n_vec * (head_dim / 8) > ((int64_t)1 << 38)) return PE_ERR_DIMS;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (head_dim == 64) return pe::kv_q_bits<64>(nbits, x, x_dtype, ldx, n_vec, ct, packed, norms_bf16, st);
  if (head_dim == 128) return pe::kv_q_bits<128>(nbits, x, x_dtype, ldx, n_vec, ct, packed, norms_bf16, st);
  return pe::kv_q_bits<256>(nbits, x, x_dtype, ldx, n_vec, ct, packed, norms_bf16, st);
}

extern "C" int pe_kv_dequantize(const uint8_t* packed, const uint16_t* norms_bf16, int64_t n_vec,
                                int head_dim, const float* ct, int nbits, uint16_t* out_bf16,
                                int64_t ldo, void* stream) {
  if (!packed || !norms_bf16 || !ct || !out_bf16) return PE_ERR_NULL;
  if (n_vec < 0 || (head_dim != 64 && head_dim != 128 && head_dim != 256) || ldo < head_dim)
    return PE_ERR_DIMS;
  if (nbits < 2 || nbits > 4) return PE_ERR_BITS;
  if (!pe::aligned16(out_bf16) || (ldo * 2) % 16) return PE_ERR_ALIGN;
  if (n_vec == 0) return PE_OK;
  if (n_vec * (head_dim / 8) > ((int64_t)1 << 38)) return PE_ERR_DIMS;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (head_dim == 64) return pe::kv_d_bits<64>(nbits, packed, norms_bf16, n_vec, ct, out_bf16, ldo, st);
  if (head_dim == 128) return pe::kv_d_bits<128>(nbits, packed, norms_bf16, n_vec, ct, out_bf16, ldo, st);
  return pe::kv_d_bits<256>(nbits, packed, norms_bf16, n_vec, ct, out_bf16, ldo, st);
}
