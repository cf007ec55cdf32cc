// Decode GEMV (M = 1) for gfx950: y[n] = sum_b norm[n,b] * <ct[codes[n,b,:]], x_tf[b,:]>.
//
// Replaces the reference's M = 1 kernels: polar_gemv / polar_gemv_packed
// (kernels/polar_gemv.py:48-174), the split-K pair that polar_matmul routes
// M = 1 to (kernels/polar_gemv_splitk.py:82-182, 257-328; dispatch
// kernels/polar_gemm.py:485-504) and the unwired CUDA kernels
// (kernels/cuda/polar_gemv_cuda.cu:52-254).
//
// Design (HBM-bound; 16 bytes of codes per lane per row):
//  * persistent grid; a wave streams whole rows: lane l reads the 16-byte
//    chunks l, l+64, ... of the row with one global_load_dwordx4 each, so one
//    wave instruction covers 1 KB of contiguous codes;
//  * the lane's slice of the transformed activation stays in registers for
//    the whole kernel (16 half2 pairs per nibble chunk, 16 floats per int8
//    chunk), staged once per workgroup through LDS -- by an in-kernel
//    FWHT-128 of the raw fp16 activation (fused prologue) or from a given
//    x_tf;
//  * nibble codes: one LDS lookup per byte returns half2(ct[lo], ct[hi]),
//    consumed by one v_dot2_f32_f16 against the pair (x[p], x[p+64]);
//    int8 codes: one fp32 lookup + one FMA per code (the reference's fp32
//    arithmetic);
//  * the LDS table is replicated per lane (entry e of lane l at
//    (e << 8) | (l << 2)) so lookups never conflict and the address is one
//    v_perm_b32 of the code byte;
//  * per-block fp16 norm applied in fp32 to the lane's chunk partial;
//    a wave reduction finishes each row; no split-K, no second pass.

#include "pe_internal.h"

namespace pe {

constexpr int kGemvThreads = 512;

// Stage one transformed 128-block held by a 16-lane group (8 values per lane,
// positions 8q..8q+7) into the kernel's LDS activation layout.
template <bool NIB>
__device__ __forceinline__ void stage_block(char* xs, int b, int q, const float v[8]) {
  if constexpr (NIB) {
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = lane_xor<8>(v[i]);
    uint4 w;
    int p0;
    if (q < 8) {
      p0 = 8 * q;
      w.x = pack_h2(v[0], o[0]); w.y = pack_h2(v[1], o[1]);
      w.z = pack_h2(v[2], o[2]); w.w = pack_h2(v[3], o[3]);
    } else {
      p0 = 8 * (q - 8) + 4;
      w.x = pack_h2(o[4], v[4]); w.y = pack_h2(o[5], v[5]);
      w.z = pack_h2(o[6], v[6]); w.w = pack_h2(o[7], v[7]);
    }
    *reinterpret_cast<uint4*>(xs + (b * 64 + p0) * 4) = w;
  } else {
    float4* d = reinterpret_cast<float4*>(xs + (b * kBlock + 8 * q) * 4);
    d[0] = make_float4(v[0], v[1], v[2], v[3]);
    d[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Dot product of one 16-byte code chunk with the lane's activations: all 16
// table lookups issue before any is consumed; four independent accumulators.
template <bool NIB>
__device__ __forceinline__ float chunk_dot(const uint4& d, uint32_t code_mask, uint32_t lane4,
                                           const uint32_t (&xr)[16]) {
  const uint32_t ws[4] = {d.x & code_mask, d.y & code_mask, d.z & code_mask, d.w & code_mask};
  uint32_t t[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    t[4 * j + 0] = lds_ld32(tbl_addr<0>(ws[j], lane4));
    t[4 * j + 1] = lds_ld32(tbl_addr<1>(ws[j], lane4));
    t[4 * j + 2] = lds_ld32(tbl_addr<2>(ws[j], lane4));
    t[4 * j + 3] = lds_ld32(tbl_addr<3>(ws[j], lane4));
  }
  float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if constexpr (NIB)
        p[b] = __builtin_amdgcn_fdot2(as_h2(t[4 * j + b]), as_h2(xr[4 * j + b]), p[b], false);
      else
        p[b] = fmaf(__uint_as_float(t[4 * j + b]), __uint_as_float(xr[4 * j + b]), p[b]);
    }
  }
  return (p[0] + p[1]) + (p[2] + p[3]);
}

// Issue the loads of one batch of U rows (S chunks each) into registers.
// Straight-line code (no branches), so the compiler can count outstanding
// loads exactly: rows past N re-read the wave's home row (an L2 hit, never a
// shared hot row) and chunks past the row end re-read the last chunk; both
// are masked out at use.
template <bool NIB, int S, int U>
__device__ __forceinline__ void issue_rows(uint4 (&d)[U][S], uint16_t (&nbits)[U][S],
                                           const uint8_t* __restrict__ codes,
                                           const uint16_t* __restrict__ norms, int home, int gw,
                                           int tw, int k0, int pass, int N, int nb, int C,
                                           int lane) {
  const int row_bytes = NIB ? nb * 64 : nb * kBlock;
  constexpr int nshift = NIB ? 2 : 3;  // chunk -> block
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int n = gw + (k0 + u) * tw;
    n = n < N ? n : home;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      int c = (pass * S + s) * 64 + lane;
      c = c < C ? c : C - 1;
      d[u][s] = ld_nt16(codes + (size_t)n * row_bytes + (size_t)c * 16);
      nbits[u][s] = norms[(size_t)n * nb + (c >> nshift)];
    }
  }
}

// XREG: the lane's activation slice lives in registers (S chunks); otherwise
// it is re-read from LDS per chunk (large K, several passes over the row).
template <bool NIB, int S, int U, int XM, int OM, bool XREG = true>
__global__ __launch_bounds__(kGemvThreads) void gemv1_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms,
    const float* __restrict__ ct, int n_levels, uint32_t code_mask, int tbl_entries,
    const void* __restrict__ x, void* __restrict__ y, const uint16_t* __restrict__ bias,
    int N, int nb, int io) {
  const bool xbf = (io & 1) != 0, ybf = (io & 2) != 0;  // raw x / y and bias are bfloat16
  extern __shared__ uint4 smem4[];
  char* smem = reinterpret_cast<char*>(smem4);
  char* xs = smem + tbl_entries * 256;  // the table occupies [0, tbl_entries * 256)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  constexpr int kWaves = kGemvThreads / 64;
  constexpr int kGroups = kGemvThreads / 16;
  const int row_bytes = NIB ? nb * 64 : nb * kBlock;
  const int C = row_bytes >> 4;  // 16-byte chunks per row
  const int gw = blockIdx.x * kWaves + wave;
  const int tw = gridDim.x * kWaves;
  const int g = tid >> 4, q = tid & 15;
  const int npass = XREG ? 1 : (C + 64 * S - 1) / (64 * S);

  // ---- 0. loads, in the order they are needed: the codebook, the activation
  // block of this 16-lane group (FWHT input), then the first batch of weight
  // rows. Loads complete in order, so the prologue below waits only for the
  // first two while the weights stream in.
  float cb[4];
  codebook_regs(cb, ct, n_levels);
  // first FWHT input block of this group, kept raw until after the barrier
  // (block index clamped: groups past nb re-read block 0 and discard it)
  const int gb = g < nb ? g : 0;
  u32x4v xraw[XM == XM_XTF_F32 ? 2 : 1];
  if constexpr (XM == XM_RAW_F16) {
    xraw[0] = *reinterpret_cast<const u32x4v*>(reinterpret_cast<const uint16_t*>(x) + gb * kBlock + q * 8);
  } else if constexpr (XM == XM_XTF_F32) {
    const u32x4v* p = reinterpret_cast<const u32x4v*>(reinterpret_cast<const float*>(x) + gb * kBlock + q * 8);
    xraw[0] = p[0];
    xraw[1] = p[1];
  }
  __builtin_amdgcn_sched_barrier(0);  // codebook and activation loads go first
  const int home = gw < N ? gw : N - 1;
  uint4 d[U][S];
  uint16_t nbits[U][S];
  issue_rows<NIB, S, U>(d, nbits, codes, norms, home, gw, tw, 0, 0, N, nb, C, lane);
  __builtin_amdgcn_sched_barrier(0);

  // ---- 1. codebook table, one copy per lane -------------------------------
  if constexpr (NIB) fill_codebook_from<TBL_NIB_H2>(0, cb, tbl_entries, kWaves);
  else fill_codebook_from<TBL_F32>(0, cb, tbl_entries, kWaves);

  // ---- 2. transformed activation into LDS ----------------------------------
  if constexpr (XM == XM_RAW_F16 || XM == XM_XTF_F32) {
    for (int b = g; b < nb; b += kGroups) {
      float v[8];
      if (b == g) {
        if constexpr (XM == XM_RAW_F16) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[2 * i] = f16or_bf((uint16_t)(xraw[0][i] & 0xffff), xbf);
            v[2 * i + 1] = f16or_bf((uint16_t)(xraw[0][i] >> 16), xbf);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[i] = __uint_as_float(xraw[0][i]);
            v[4 + i] = __uint_as_float(xraw[XM == XM_XTF_F32 ? 1 : 0][i]);
          }
        }
      } else if constexpr (XM == XM_RAW_F16) {
        if (xbf) load8<PE_DTYPE_BF16>(reinterpret_cast<const uint16_t*>(x) + b * kBlock + q * 8, v);
        else load8<PE_DTYPE_F16>(reinterpret_cast<const uint16_t*>(x) + b * kBlock + q * 8, v);
      } else {
        load8<PE_DTYPE_F32>(reinterpret_cast<const float*>(x) + b * kBlock + q * 8, v);
      }
      if constexpr (XM == XM_RAW_F16) fwht128_group16(v, q);
      stage_block<NIB>(xs, b, q, v);
    }
  } else {  // pair f16 input: nb * 64 half2
    const uint4* src = reinterpret_cast<const uint4*>(x);
    if constexpr (NIB) {
      for (int i = tid; i < nb * 16; i += kGemvThreads)
        reinterpret_cast<uint4*>(xs)[i] = src[i];
    } else {
      // pairs p..p+3 of block b -> x[p..p+3] and x[p+64..p+67]
      for (int i = tid; i < nb * 16; i += kGemvThreads) {
        const uint4 w = src[i];
        const int b = i >> 4, p = (i & 15) * 4;
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
        float lo[4], hi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          lo[j] = h2f((uint16_t)(ws[j] & 0xffff));
          hi[j] = h2f((uint16_t)(ws[j] >> 16));
        }
        float* dst = reinterpret_cast<float*>(xs) + b * kBlock + p;
        *reinterpret_cast<float4*>(dst) = make_float4(lo[0], lo[1], lo[2], lo[3]);
        *reinterpret_cast<float4*>(dst + 64) = make_float4(hi[0], hi[1], hi[2], hi[3]);
      }
    }
  }
  __syncthreads();

  // ---- 3. activation slice of this lane ------------------------------------
  // Pass p covers chunks (p*S + s)*64 + lane, s < S. Nibble chunk c: block
  // c>>2, pairs 16*(c&3)..+15; int8 chunk c: block c>>3, positions
  // 16*(c&7)..+15. With XREG there is one pass and the slice is loaded once;
  // otherwise (large K) each pass re-reads its slice from LDS.
  uint32_t xr[S][16];
  auto load_x = [&](int pass) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int c = (pass * S + s) * 64 + lane;
      if (c < C) {
        const int off = NIB ? ((c >> 2) * 64 + (c & 3) * 16) * 4 : ((c >> 3) * kBlock + (c & 7) * 16) * 4;
        const u32x4v* p = reinterpret_cast<const u32x4v*>(xs + off);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x4v w = p[j];
          xr[s][4 * j] = w[0]; xr[s][4 * j + 1] = w[1]; xr[s][4 * j + 2] = w[2]; xr[s][4 * j + 3] = w[3];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) xr[s][j] = 0u;
      }
    }
  };
  if constexpr (XREG) load_x(0);

  // ---- 4. stream rows --------------------------------------------------------
  // rows gw, gw + tw, gw + 2 tw, ... (balanced to +-1 row per wave), U at a
  // time; the first batch (pass 0) was issued before the prologue.
  const uint32_t lane4 = (uint32_t)lane << 2;
  for (int k0 = 0; gw + k0 * tw < N; k0 += U) {
    float acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = 0.f;
    for (int pass = 0; pass < npass; ++pass) {
      if constexpr (!XREG) load_x(pass);
      if (k0 != 0 || pass != 0) {
        issue_rows<NIB, S, U>(d, nbits, codes, norms, home, gw, tw, k0, pass, N, nb, C, lane);
        // keep every load of this batch ahead of the arithmetic: otherwise the
        // scheduler sinks the norm loads to their uses, one round trip each
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (gw + (k0 + u) * tw >= N) continue;  // wave-uniform
        float a = acc[u];
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const bool live = (pass * S + s) * 64 + lane < C;
          const float nrm = live ? h2f(nbits[u][s]) : 0.f;
          a = fmaf(chunk_dot<NIB>(d[u][s], code_mask, lane4, xr[s]), nrm, a);
        }
        acc[u] = a;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int n = gw + (k0 + u) * tw;
      if (n >= N) continue;  // wave-uniform
      const float r = wave_sum_dpp(acc[u]);
      if (lane == 0) {
        if constexpr (OM == OM_F32) {
          reinterpret_cast<float*>(y)[n] = r;
        } else {
          // reference order: fp32 result -> .half() -> + bias.half() (16-bit add)
          reinterpret_cast<uint16_t*>(y)[n] = out16(r, bias, n, ybf);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host launch
// ---------------------------------------------------------------------------

template <bool NIB, int S, int XM, int OM, bool XREG>
static int launch_gemv1_s(const Gemv1Args& a, hipStream_t st) {
  constexpr int U = !XREG ? 2 : (S <= 2 ? 4 : (S <= 6 ? 2 : 1));
  auto kern = gemv1_kernel<NIB, S, U, XM, OM, XREG>;
  const int entries = table_entries(NIB, a.n_levels);
  const size_t lds = (size_t)entries * 256 + (size_t)a.nb * (NIB ? 256 : 512);
  if (lds > 160 * 1024) return PE_ERR_DIMS;
  static const bool attr_ok = [&] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  const int per_cu = lds <= 80 * 1024 ? 2 : 1;
  // enough waves for one row each, capped at what stays resident
  constexpr int kWaves = kGemvThreads / 64;
  int grid = (a.N + kWaves - 1) / kWaves;
  const int cap = num_cus() * per_cu;
  if (grid > cap) grid = cap;
  const uint8_t mb = NIB ? (uint8_t)((a.n_levels - 1) * 0x11) : (uint8_t)(a.n_levels - 1);
  const uint32_t mask = 0x01010101u * mb;
  kern<<<dim3(grid), dim3(kGemvThreads), lds, st>>>(a.codes, a.norms, a.ct, a.n_levels, mask,
                                                   entries, a.x, a.y, a.bias, a.N, a.nb,
                                                   (a.xbf ? 1 : 0) | (a.ybf ? 2 : 0));
  return launch_status();
}

template <bool NIB, int XM, int OM>
static int launch_gemv1(const Gemv1Args& a, hipStream_t st) {
  const int C = (NIB ? a.nb * 64 : a.nb * kBlock) / 16;
  if (C <= 64) return launch_gemv1_s<NIB, 1, XM, OM, true>(a, st);
  if (C <= 128) return launch_gemv1_s<NIB, 2, XM, OM, true>(a, st);
  if (C <= 192) return launch_gemv1_s<NIB, 3, XM, OM, true>(a, st);
  if (C <= 256) return launch_gemv1_s<NIB, 4, XM, OM, true>(a, st);
  if (C <= 512) return launch_gemv1_s<NIB, 8, XM, OM, true>(a, st);
  // large K: activations stay in LDS, four chunks per lane per pass
  return launch_gemv1_s<NIB, 4, XM, OM, false>(a, st);
}

// Largest K (padded) the M = 1 kernel takes: LDS holds the codebook table
// (<= 64 KB) and the activations (256 B per block as pairs, 512 B as fp32).
int gemv1_max_kp(bool nibble) { return nibble ? 96 * 1024 / 256 * 128 : 96 * 1024 / 512 * 128; }

int gemv1(bool nibble, int xmode, int omode, const Gemv1Args& a, hipStream_t st) {
  if (nibble) {
    if (xmode == XM_XTF_F32 && omode == OM_F32) return launch_gemv1<true, XM_XTF_F32, OM_F32>(a, st);
    if (xmode == XM_RAW_F16 && omode == OM_F16) return launch_gemv1<true, XM_RAW_F16, OM_F16>(a, st);
    if (xmode == XM_PAIR_F16 && omode == OM_F16) return launch_gemv1<true, XM_PAIR_F16, OM_F16>(a, st);
  } else {
    if (xmode == XM_XTF_F32 && omode == OM_F32) return launch_gemv1<false, XM_XTF_F32, OM_F32>(a, st);
    if (xmode == XM_RAW_F16 && omode == OM_F16) return launch_gemv1<false, XM_RAW_F16, OM_F16>(a, st);
    if (xmode == XM_PAIR_F16 && omode == OM_F16) return launch_gemv1<false, XM_PAIR_F16, OM_F16>(a, st);
  }
  return PE_ERR_DTYPE;
}

static int check_levels(bool nibble, int n_levels) {
  if (nibble) return (n_levels >= 2 && n_levels <= 16 && (n_levels & (n_levels - 1)) == 0) ? PE_OK : PE_ERR_BITS;
  return (n_levels >= 2 && n_levels <= 256 && (n_levels & (n_levels - 1)) == 0) ? PE_OK : PE_ERR_BITS;
}

int polar_gemv_ref(bool nibble, const void* codes, const float* x_tf, const uint16_t* norms,
                   const float* ct, int n_levels, float* out, int out_f, int kp, int n_blocks,
                   int block_size, hipStream_t st) {
  if (!codes || !x_tf || !norms || !ct || !out) return PE_ERR_NULL;
  if (block_size != kBlock) return PE_ERR_DIMS;
  if (out_f <= 0 || n_blocks <= 0 || kp != n_blocks * kBlock) return PE_ERR_DIMS;
  if (int rc = check_levels(nibble, n_levels)) return rc;
  if (!aligned16(codes) || !aligned16(x_tf)) return PE_ERR_ALIGN;
  Gemv1Args a{reinterpret_cast<const uint8_t*>(codes), norms, ct, n_levels, x_tf, out, nullptr,
              out_f, n_blocks};
  return gemv1(nibble, XM_XTF_F32, OM_F32, a, st);
}

}  // namespace pe

extern "C" int pe_polar_gemv(const int8_t* codes, const float* x_tf, const uint16_t* norms_f16,
                             const float* ct_scaled, int n_levels, float* out, int out_f,
                             int in_f_padded, int n_blocks, int block_size, void* stream) {
  return pe::polar_gemv_ref(false, codes, x_tf, norms_f16, ct_scaled, n_levels, out, out_f,
                            in_f_padded, n_blocks, block_size, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pe_polar_gemv_packed(const uint8_t* packed, const float* x_tf,
                                    const uint16_t* norms_f16, const float* ct_scaled,
                                    int n_levels, float* out, int out_f, int in_f_half,
                                    int n_blocks, int block_size, void* stream) {
  if (in_f_half != n_blocks * 64) return PE_ERR_DIMS;
  return pe::polar_gemv_ref(true, packed, x_tf, norms_f16, ct_scaled, n_levels, out, out_f,
                            n_blocks * pe::kBlock, n_blocks, block_size,
                            reinterpret_cast<hipStream_t>(stream));
}
