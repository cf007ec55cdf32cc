// Shared device and host helpers for the gfx950 PolarEngine kernels.
//
// Conventions used by every kernel in this library:
//  * wave64; a "block" is one 128-wide quantization block (never a HIP block,
//    which is called a workgroup here);
//  * the codebook lookup goes through an LDS table replicated once per lane:
//    entry e of lane l lives at byte (e << 8) | (l << 2), so a lane only ever
//    touches its own bank and a v_perm_b32 builds the address from a code
//    byte in one instruction;
//  * activations enter MFMA/dot2 paths as "pairs" (x[p], x[p + 64]) of one
//    128-block, matching the half-block nibble packing where one byte holds
//    the codes of positions p and p + 64.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/polarengine_amd.h"

namespace pe {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

constexpr int kBlock = 128;           // quantization block (fixed by the format)
constexpr float kInvSqrt128 = 0.08838834764831845f;  // fp32(2^-3.5)

// ---------------------------------------------------------------------------
// bit helpers
// ---------------------------------------------------------------------------

// 16-byte streaming load (non-temporal: weights are read once per call)
__device__ __forceinline__ u32x4v ld_nt16v(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
}
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

__device__ __forceinline__ float h2f(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}
__device__ __forceinline__ uint16_t f2h_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// host side fp32 -> fp16 bits, round to nearest even like v_cvt_f16_f32
inline uint16_t host_f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return (uint32_t)f2h_bits(lo) | ((uint32_t)f2h_bits(hi) << 16);
}
// bfloat16 <-> float, round-to-nearest-even on the way down (NaN kept quiet).
__device__ __forceinline__ float bf2f(uint16_t bits) {
  return __builtin_bit_cast(float, (uint32_t)bits << 16);
}
__device__ __forceinline__ uint16_t f2bf_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// fp32 -> bf16 bits, round to nearest even in hardware (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint16_t f2bf_rne(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// 16-bit activation / output element: bf16 when `bf`, else fp16
__device__ __forceinline__ float f16or_bf(uint16_t bits, bool bf) {
  return bf ? bf2f(bits) : h2f(bits);
}
__device__ __forceinline__ uint16_t to16(float f, bool bf) { return bf ? f2bf_rne(f) : f2h_bits(f); }
__device__ __forceinline__ uint32_t pack16x2(float lo, float hi, bool bf) {
  return (uint32_t)to16(lo, bf) | ((uint32_t)to16(hi, bf) << 16);
}
// One output element of a linear epilogue: the fp32 result rounded to the
// 16-bit output type, then the bias (same type) added in fp32 and rounded
// again -- the reference's `output.half()` then `+ bias.half()`
// (linear_method.py:219-221), in the output type of the activation.
__device__ __forceinline__ uint16_t out16(float v, const uint16_t* bias, int64_t n, bool bf) {
  uint16_t r = to16(v, bf);
  if (bias) r = to16(f16or_bf(r, bf) + f16or_bf(bias[n], bf), bf);
  return r;
}

// Raw LDS access by byte address. The kernels of this library declare no
// static LDS, so their dynamic LDS block starts at address 0 and a table
// address built by v_perm is used as is (no base add per lookup).
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(3))) u32x4v lds_u32x4;
__device__ __forceinline__ uint32_t lds_ld32(uint32_t addr) {
  return *reinterpret_cast<const lds_u32*>(static_cast<uintptr_t>(addr));
}
__device__ __forceinline__ void lds_st128(uint32_t addr, u32x4v v) {
  *reinterpret_cast<lds_u32x4*>(static_cast<uintptr_t>(addr)) = v;
}
__device__ __forceinline__ void lds_st32(uint32_t addr, uint32_t v) {
  *reinterpret_cast<lds_u32*>(static_cast<uintptr_t>(addr)) = v;
}
typedef __attribute__((address_space(3))) uint16_t lds_u16;
__device__ __forceinline__ void lds_st16(uint32_t addr, uint16_t v) {
  *reinterpret_cast<lds_u16*>(static_cast<uintptr_t>(addr)) = v;
}
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) u32x2v lds_u32x2;
__device__ __forceinline__ void lds_st64(uint32_t addr, u32x2v v) {
  *reinterpret_cast<lds_u32x2*>(static_cast<uintptr_t>(addr)) = v;
}
__device__ __forceinline__ u32x4v lds_ld128(uint32_t addr) {
  return *reinterpret_cast<const lds_u32x4*>(static_cast<uintptr_t>(addr));
}

// Device-coherent 32-bit accesses for data one workgroup hands to another
// within one launch: agent-scope relaxed atomics, which compile to global
// loads and stores with the sc1 cache policy (the level every XCD sees
// alike). The producer stores with st_dev32, waits for its stores
// (s_waitcnt vmcnt(0)), then counts itself in with a device-scope atomicAdd;
// the workgroup whose increment completes the count reads with ld_dev32. A
// device-scope release/acquire fence in their place would write back and
// invalidate the XCD's whole L2 once per wave.
__device__ __forceinline__ void st_dev32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS table address for code byte `b` (0..3) of dword `w`: (byte << 8) | lane4.
// v_perm_b32 picks byte 0 from src1 (= lane4 < 256) and byte 1 from byte b of
// src0 (= w); bytes 2-3 are zero (selector 0x0c).
template <int B>
__device__ __forceinline__ uint32_t tbl_addr(uint32_t w, uint32_t lane4) {
  return __builtin_amdgcn_perm(w, lane4, 0x0c0c0000u | ((4u + B) << 8));
}

// ---------------------------------------------------------------------------
// Cross-lane moves inside 16-lane rows without LDS data traffic: DPP
// quad_perm for lane xor 1 / xor 2, DPP row_ror:8 for xor 8 (rotating a
// 16-lane row by 8 swaps its halves), ds_swizzle bit mode for xor 4.
// ---------------------------------------------------------------------------
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  const int i = __builtin_bit_cast(int, v);
  int r;
  if constexpr (M == 1) r = __builtin_amdgcn_mov_dpp(i, 0xB1, 0xF, 0xF, false);       // quad_perm [1,0,3,2]
  else if constexpr (M == 2) r = __builtin_amdgcn_mov_dpp(i, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  else if constexpr (M == 8) r = __builtin_amdgcn_mov_dpp(i, 0x128, 0xF, 0xF, false); // row_ror:8
  else r = __builtin_amdgcn_ds_swizzle(i, (M << 10) | 0x1F);                          // and 0x1f, xor M
  return __builtin_bit_cast(float, r);
}

// Sum over the 64 lanes, result in every lane: shuffles (LDS crossbar).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over the 64 lanes, wave-uniform result: DPP/swizzle inside 16-lane
// rows, then the four row sums through readlane (no LDS round trips).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += lane_xor<1>(v);
  v += lane_xor<2>(v);
  v += lane_xor<4>(v);
  v += lane_xor<8>(v);
  const int b = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

// ---------------------------------------------------------------------------
// FWHT-128 on a 16-lane group: each lane holds 8 consecutive values
// (positions 8q..8q+7, q = lane & 15). Stages 1, 2, 4 are in-lane, 8..64 use
// lane xor 1, 2, 4, 8. Result is scaled by 1/sqrt(128).
// ---------------------------------------------------------------------------
// Butterfly across lanes: lower lane v + o, upper lane o - v, as one fma with
// a per-lane sign (exact: a product by +-1 rounds nothing).
template <int M>
__device__ __forceinline__ void fwht_xstage(float v[8], int q) {
  const float sgn = (q & M) ? -1.f : 1.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(sgn, v[i], lane_xor<M>(v[i]));
}

// Unnormalised: v <- H v with H[i][j] = (-1)^popcount(i & j) (entries +-1).
__device__ __forceinline__ void fwht128_group16_raw(float v[8], int q) {
#pragma unroll
  for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if ((i & h) == 0) {
        float a = v[i], b = v[i + h];
        v[i] = a + b;
        v[i + h] = a - b;
      }
    }
  }
  fwht_xstage<1>(v, q);
  fwht_xstage<2>(v, q);
  fwht_xstage<4>(v, q);
  fwht_xstage<8>(v, q);
}

__device__ __forceinline__ void fwht128_group16(float v[8], int q) {
  fwht128_group16_raw(v, q);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] *= kInvSqrt128;
}

// ---------------------------------------------------------------------------
// H128 on the matrix cores: y^T = H x^T for 32 vectors of 128 as 4 m-blocks x
// 8 k-steps of v_mfma_f32_32x32x16 (A = a 32 x 16 block of H, B = 16
// positions x 32 vectors: lane l holds positions 16 kt + 8 h .. + 7 of
// vector l % 32, h = l / 32). Products of 16-bit values by +-1 are exact and
// the sums fp32. For r = 32 mb + m (m = l % 32) and c = 16 kt + 8 h + j,
// H[r][c] = (-1)^popcount(r & c) = F[j] * (-1)^(m4 kt0) * (-1)^(mb0 kt1 +
// mb1 kt2) with the lane's base F[j] = (-1)^(popcount(m & j & 7) + m3 h), so
// every A block is one of F, -F, G = (-1)^m4 F, -G (16 registers). The
// accumulator of m-block mb holds, in lane l, positions
// 32 mb + 8 (e / 4) + 4 h + e % 4 (e = 0..15) of vector l % 32.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));

struct H128Signs {
  u32x4v F, nF, G, nG;
};

// ONE2: two 16-bit ones (fp16 0x3C003C00, bf16 0x3F803F80); the sign bits
// sit at 15 and 31 in both formats
template <uint32_t ONE2>
__device__ __forceinline__ H128Signs h128_signs(int lane) {
  const int n = lane & 31, h = lane >> 5;
  const uint32_t hb = (uint32_t)(((n >> 3) & 1) & h);
  H128Signs s;
#pragma unroll
  for (int jp = 0; jp < 4; ++jp) {
    const uint32_t s0 = ((uint32_t)__builtin_popcount(n & (2 * jp) & 7) + hb) & 1u;
    const uint32_t s1 = ((uint32_t)__builtin_popcount(n & (2 * jp + 1) & 7) + hb) & 1u;
    s.F[jp] = ONE2 | (s0 << 15) | (s1 << 31);
    s.nF[jp] = s.F[jp] ^ 0x80008000u;
  }
  const bool m4 = (n >> 4) & 1;
#pragma unroll
  for (int jp = 0; jp < 4; ++jp) {
    s.G[jp] = m4 ? s.nF[jp] : s.F[jp];
    s.nG[jp] = m4 ? s.F[jp] : s.nF[jp];
  }
  return s;
}

// the A block of H for m-block mb, k-step kt (mb, kt compile-time after unrolling)
__device__ __forceinline__ u32x4v h128_block(const H128Signs& s, int mb, int kt) {
  const bool neg = (((mb & 1) & (kt >> 1)) ^ ((mb >> 1) & (kt >> 2))) & 1;
  return (kt & 1) ? (neg ? s.nG : s.G) : (neg ? s.nF : s.F);
}

// accumulators of m-blocks mb0 and mb1 (raw H x, no normalisation) from the
// lane's eight 16-byte position groups b[kt]; BF: the values are bfloat16
template <bool BF>
__device__ __forceinline__ void h128_mfma_pair(const H128Signs& s, const u32x4v (&b)[8], int mb0,
                                               int mb1, float16v& a0, float16v& a1) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    a0[e] = 0.f;
    a1[e] = 0.f;
  }
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) {
    const u32x4v k0 = h128_block(s, mb0, kt), k1 = h128_block(s, mb1, kt);
    if constexpr (BF) {
      a0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, k0),
                                                   __builtin_bit_cast(bf16x8v, b[kt]), a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, k1),
                                                   __builtin_bit_cast(bf16x8v, b[kt]), a1, 0, 0, 0);
    } else {
      a0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8v, k0),
                                                  __builtin_bit_cast(half8v, b[kt]), a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8v, k1),
                                                  __builtin_bit_cast(half8v, b[kt]), a1, 0, 0, 0);
    }
  }
}

// Pair-f16 store of one 128-block held by a 16-lane group (lane q holds
// elements 8q..8q+7): dword p of the block's 64 dwords at `blk` is
// (x[p], x[p + 64]). Lanes q < 8 write dwords 8q..8q+3, lanes q >= 8 dwords
// 8(q-8)+4..8(q-8)+7, each as one 16-byte store. Every lane of the group must
// take part (cross-lane exchange); only `live` lanes store.
__device__ __forceinline__ void store_pair_block(const float v[8], int q, uint32_t* blk, bool live) {
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = lane_xor<8>(v[i]);
  if (!live) return;
  u32x4v w;
  int p0;
  if (q < 8) {
    p0 = 8 * q;
    w = u32x4v{pack_h2(v[0], o[0]), pack_h2(v[1], o[1]), pack_h2(v[2], o[2]), pack_h2(v[3], o[3])};
  } else {
    p0 = 8 * (q - 8) + 4;
    w = u32x4v{pack_h2(o[4], v[4]), pack_h2(o[5], v[5]), pack_h2(o[6], v[6]), pack_h2(o[7], v[7])};
  }
  *reinterpret_cast<u32x4v*>(blk + p0) = w;
}

// ---------------------------------------------------------------------------
// Per-lane replicated codebook table in LDS: dword e*64 + lane holds entry e.
//   TBL_NIB_H2: entry e = half2(ct[e & 15], ct[e >> 4]) (nibble byte e)
//   TBL_F16   : entry e = fp16 bits of ct[e] in the low half
//   TBL_F32   : entry e = ct[e]
// Lane j first loads ct[j + 64 i] (one global load per lane); each thread then
// writes four lane copies of one entry per ds_write_b128, the entry value
// fetched from the owning lane with ds_bpermute.
// ---------------------------------------------------------------------------
enum { TBL_NIB_H2 = 0, TBL_F16 = 1, TBL_F32 = 2 };

// Lane j keeps ct[j + 64 i] (i < 4; zero past n_levels).
__device__ __forceinline__ void codebook_regs(float (&c)[4], const float* __restrict__ ct,
                                              int n_levels) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = (lane + 64 * i) < n_levels ? ct[lane + 64 * i] : 0.f;
}

template <int KIND>
__device__ __forceinline__ void fill_codebook_from(uint32_t tbl_off, const float (&c)[4],
                                                   int entries, int nwaves) {
  const int nthreads = nwaves * 64;
  const int total16 = entries * 16;  // 16-byte stores: 16 per entry (64 lanes x 4 B)
  // wave-uniform trip count: every lane of the wave takes part in ds_bpermute
  // (a source lane must be active), only the store is predicated
  for (int d0 = threadIdx.x & ~63; d0 < total16; d0 += nthreads) {
    const int d = d0 + (threadIdx.x & 63);
    const int e = d >> 4;
    uint32_t v;
    if constexpr (KIND == TBL_NIB_H2) {
      const int lo = e & 15, hi = e >> 4;  // n_levels <= 16: both held in c[0]
      const int c0 = __builtin_bit_cast(int, c[0]);
      v = pack_h2(__builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(lo << 2, c0)),
                  __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(hi << 2, c0)));
    } else {
      const int q = e >> 6, r = e & 63;
      const float src = q == 0 ? c[0] : q == 1 ? c[1] : q == 2 ? c[2] : c[3];
      const float val = __builtin_bit_cast(
          float, __builtin_amdgcn_ds_bpermute(r << 2, __builtin_bit_cast(int, src)));
      v = KIND == TBL_F16 ? (uint32_t)f2h_bits(val) : __builtin_bit_cast(uint32_t, val);
    }
    if (d < total16) lds_st128(tbl_off + (uint32_t)d * 16u, u32x4v{v, v, v, v});
  }
}

template <int KIND>
__device__ __forceinline__ void fill_codebook(uint32_t tbl_off, const float* __restrict__ ct,
                                              int n_levels, int entries, int nwaves) {
  float c[4];
  codebook_regs(c, ct, n_levels);
  fill_codebook_from<KIND>(tbl_off, c, entries, nwaves);
}

// Load 8 consecutive activations as float from a dtype-tagged pointer.
template <int DT>
__device__ __forceinline__ void load8(const void* p, float v[8]) {
  if constexpr (DT == PE_DTYPE_F32) {
    const float4* q = reinterpret_cast<const float4*>(p);
    float4 a = q[0], b = q[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    uint4 a = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == PE_DTYPE_F16) {
        v[2 * i] = h2f((uint16_t)(w[i] & 0xffff));
        v[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
      } else {
        v[2 * i] = bf2f((uint16_t)(w[i] & 0xffff));
        v[2 * i + 1] = bf2f((uint16_t)(w[i] >> 16));
      }
    }
  }
}


}  // namespace pe

// ---------------------------------------------------------------------------
// host-side helpers (defined in pe_api.hip)
// ---------------------------------------------------------------------------
namespace pe {
int num_cus();                         // CUs of the current device (cached)
int launch_status();                   // PE_OK or PE_ERR_LAUNCH
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
// 16-bit activation dtype code -> bf16 flag; -1 for anything else
inline int bf16_flag(int dtype) {
  return dtype == PE_DTYPE_F16 ? 0 : dtype == PE_DTYPE_BF16 ? 1 : -1;
}
inline int table_entries(bool nibble, int n_levels) {
  // nibble: entries 0..mask where mask = (n_levels-1) * 0x11; int8: n_levels.
  return nibble ? (n_levels - 1) * 0x11 + 1 : n_levels;
}
}  // namespace pe
