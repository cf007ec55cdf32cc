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

__device__ __forceinline__ uint32_t as_u32(half2v h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

__device__ __forceinline__ float h2f(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}
__device__ __forceinline__ uint16_t f2h_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
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

// LDS table address for code byte `b` (0..3) of dword `w`: (byte << 8) | lane4.
// v_perm_b32 picks byte 0 from src1 (= lane4 < 256) and byte 1 from byte b of
// src0 (= w); bytes 2-3 are zero (selector 0x0c).
template <int B>
__device__ __forceinline__ uint32_t tbl_addr(uint32_t w, uint32_t lane4) {
  return __builtin_amdgcn_perm(w, lane4, 0x0c0c0000u | ((4u + B) << 8));
}

// ---------------------------------------------------------------------------
// wave-level reductions (wave64)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------------------
// FWHT-128 on a 16-lane group: each lane holds 8 consecutive values
// (positions 8q..8q+7, q = lane & 15). Stages 1, 2, 4 are in-lane, 8..64 use
// lane xor 1, 2, 4, 8. Result is scaled by 1/sqrt(128).
// ---------------------------------------------------------------------------

__device__ __forceinline__ void fwht128_group16(float v[8], int q) {
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
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    const bool upper = (q & m) != 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float o = __shfl_xor(v[i], m, 64);
      v[i] = upper ? (o - v[i]) : (v[i] + o);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] *= kInvSqrt128;
}

// ---------------------------------------------------------------------------
// Per-lane replicated codebook table in LDS: dword e*64 + lane holds entry e.
// The codebook is read from global memory once per lane (lane j keeps
// ct[j + 64 i]) and broadcast with v_readlane, so filling the table issues
// no dependent global loads.
//   TBL_NIB_H2: entry e = half2(ct[e & 15], ct[e >> 4]) (nibble byte e)
//   TBL_F16   : entry e = fp16 bits of ct[e] in the low half
//   TBL_F32   : entry e = ct[e]
// ---------------------------------------------------------------------------
enum { TBL_NIB_H2 = 0, TBL_F16 = 1, TBL_F32 = 2 };

__device__ __forceinline__ float bcast_lane(float v, int src_lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src_lane));
}

template <int KIND>
__device__ __forceinline__ void fill_codebook(uint32_t* tbl, const float* __restrict__ ct,
                                              int n_levels, int entries, int nwaves) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = (lane + 64 * i) < n_levels ? ct[lane + 64 * i] : 0.f;
  for (int e = wave; e < entries; e += nwaves) {
    uint32_t v;
    if constexpr (KIND == TBL_NIB_H2) {
      const int lo = e & 15, hi = e >> 4;  // n_levels <= 16: both in c[0]
      v = pack_h2(bcast_lane(c[0], lo), bcast_lane(c[0], hi));
    } else {
      const int q = e >> 6, r = e & 63;
      const float src = q == 0 ? c[0] : q == 1 ? c[1] : q == 2 ? c[2] : c[3];
      const float val = bcast_lane(src, r);
      v = KIND == TBL_F16 ? (uint32_t)f2h_bits(val) : __builtin_bit_cast(uint32_t, val);
    }
    tbl[e * 64 + lane] = v;
  }
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
inline int table_entries(bool nibble, int n_levels) {
  // nibble: entries 0..mask where mask = (n_levels-1) * 0x11; int8: n_levels.
  return nibble ? (n_levels - 1) * 0x11 + 1 : n_levels;
}
}  // namespace pe
