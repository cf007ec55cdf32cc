// Small-M quantized matmul for gfx950 (batches M = 2..64 that the decode
// kernel does not take), and the grouped-expert MoE products:
// Y[m, n] = sum_k X_tf[m, k] * W~[n, k].
//
// Replaces the reference's M > 1 path for small batches (polar_gemm /
// polar_gemm_packed, kernels/polar_gemm.py:81-418, autotuned Triton tiles) and
// provides the quantized expert products the reference never had
// (moe_method.py forwards experts to vLLM's bf16 fused MoE).
//
// Structure:
//  * v_mfma_f32_16x16x32_f16 with the activations as the A operand (16 rows
//    per m-tile, rows >= M zero) and the dequantized weights as B
//    (16 weight rows per n-tile);
//  * a 512-lane workgroup owns TN n-tiles and all M (1-2 m-tiles per pass); its 8
//    waves split the K blocks, each reading a contiguous K range, and combine
//    through LDS at the end -- no global workspace, deterministic order;
//  * lane (n = l % 16, g = l / 16) reads 16 contiguous code bytes per row per
//    128-block (one dwordx4 for nibbles); slab t of the block takes dword t,
//    i.e. pairs 16g + 4t + j, and A takes the same pairs from the pair-f16
//    x_tf (16 contiguous bytes per lane per slab);
//  * the per-block fp16 norm multiplies the 4 fp32 MFMA results of each block
//    (fp32, as the reference applies it), not the fp16 operands;
//  * epilogues: fp32 out, or 16-bit out (+ bias).
// The MoE expert products (moe_gemv_kernel, further down) have their own
// kernel: blockIdx.y selects an expert, whose rows are [off[e], off[e+1]) of
// a row list, and the weights advance by per-expert strides.

#include "pe_internal.h"

namespace pe {

constexpr int kSmallThreads = 512;
constexpr int kSmallWaves = kSmallThreads / 64;

template <bool NIB>
__device__ __forceinline__ half8v dequant_slab_raw(const char* tbl, uint32_t wlo, uint32_t whi,
                                                   uint32_t lane4) {
  uint32_t p[4];
  if constexpr (NIB) {
    p[0] = lds_ld32(tbl_addr<0>(wlo, lane4));
    p[1] = lds_ld32(tbl_addr<1>(wlo, lane4));
    p[2] = lds_ld32(tbl_addr<2>(wlo, lane4));
    p[3] = lds_ld32(tbl_addr<3>(wlo, lane4));
  } else {
    const uint32_t a0 = lds_ld32(tbl_addr<0>(wlo, lane4));
    const uint32_t a1 = lds_ld32(tbl_addr<1>(wlo, lane4));
    const uint32_t a2 = lds_ld32(tbl_addr<2>(wlo, lane4));
    const uint32_t a3 = lds_ld32(tbl_addr<3>(wlo, lane4));
    const uint32_t b0 = lds_ld32(tbl_addr<0>(whi, lane4));
    const uint32_t b1 = lds_ld32(tbl_addr<1>(whi, lane4));
    const uint32_t b2 = lds_ld32(tbl_addr<2>(whi, lane4));
    const uint32_t b3 = lds_ld32(tbl_addr<3>(whi, lane4));
    p[0] = __builtin_amdgcn_perm(b0, a0, 0x05040100u);
    p[1] = __builtin_amdgcn_perm(b1, a1, 0x05040100u);
    p[2] = __builtin_amdgcn_perm(b2, a2, 0x05040100u);
    p[3] = __builtin_amdgcn_perm(b3, a3, 0x05040100u);
  }
  u32x4v v = {p[0], p[1], p[2], p[3]};
  return __builtin_bit_cast(half8v, v);
}

// Loads of one 128-block for a wave: codes/norm bits of its NT n-tiles and
// the pair-f16 activations of its (up to MTM) m-tiles.
template <int NT, int MTM>
struct SmallBlk {
  u32x4v lo[NT];
  u32x4v hi[NT];
  uint16_t nbits[NT];
  u32x4v a[MTM][4];
};

template <bool NIB, int NT, int MTM>
__device__ __forceinline__ void load_sblk(SmallBlk<NT, MTM>& k, const uint8_t* const (&brow)[NT],
                                          const uint16_t* const (&nrow)[NT],
                                          const uint32_t* const (&arow)[MTM],
                                          const bool (&alive)[MTM], int b, const WLayout& lay) {
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const uint8_t* pc = brow[j] + b * lay.c_blk;
    k.lo[j] = ld_nt16v(pc);
    if constexpr (!NIB) k.hi[j] = ld_nt16v(pc + 64);
    k.nbits[j] = nrow[j][b * lay.n_blk];
  }
#pragma unroll
  for (int i = 0; i < MTM; ++i) {
    if (alive[i]) {
      const u32x4v* p = reinterpret_cast<const u32x4v*>(arow[i] + b * 64);
#pragma unroll
      for (int t = 0; t < 4; ++t) k.a[i][t] = p[t];
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) k.a[i][t] = u32x4v{0u, 0u, 0u, 0u};
    }
  }
}

template <bool NIB, int NT, int MTM>
__device__ __forceinline__ void compute_sblk(float4v (&acc)[MTM][NT], const SmallBlk<NT, MTM>& k,
                                             const char* tbl, uint32_t lane4, uint32_t code_mask,
                                             int MT) {
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    float4v blk[MTM];
#pragma unroll
    for (int i = 0; i < MTM; ++i) blk[i] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t wl = k.lo[j][t] & code_mask;
      const uint32_t wh = NIB ? 0u : (k.hi[j][t] & code_mask);
      const half8v bf = dequant_slab_raw<NIB>(tbl, wl, wh, lane4);
#pragma unroll
      for (int i = 0; i < MTM; ++i)
        if (i < MT)
          blk[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, k.a[i][t]),
                                                          bf, blk[i], 0, 0, 0);
    }
    // per-block norm applied to the fp32 block partial
    const float nrm = h2f(k.nbits[j]);
#pragma unroll
    for (int i = 0; i < MTM; ++i) acc[i][j] += blk[i] * nrm;
  }
}

// TN: n-tiles of 16 weight rows per workgroup; MTM: m-tiles of 16 rows per
// pass over the weights; EP: SE_F32 or SE_F16.
template <bool NIB, int TN, int EP, int MTM>
__global__ __launch_bounds__(kSmallThreads) void gemm_small_kernel(
    SmallArgs a, uint32_t code_mask, int tbl_entries) {
  static_assert(EP == SE_F32 || EP == SE_F16, "small-M epilogues: fp32 or 16-bit out");
  constexpr int NT = TN;
  extern __shared__ uint4 smem4[];
  char* smem = reinterpret_cast<char*>(smem4);
  char* tbl = smem;
  float* red = reinterpret_cast<float*>(smem);  // after the K loop: [waves][MTM][NT][64][4]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15, g = lane >> 4;
  const uint32_t lane4 = (uint32_t)lane << 2;

  const int M = a.M;
  // ---- this lane's weight rows (clamped; clamped rows are never stored)
  const uint8_t* brow[NT];
  const uint16_t* nrow[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    int n = blockIdx.x * TN * 16 + j * 16 + l16;
    if (n >= a.N) n = a.N - 1;
    brow[j] = a.codes + a.lay.codes_off(n) + 16 * g;
    nrow[j] = a.norms + a.lay.norms_off(n);
  }
  const int64_t xrow = (int64_t)a.nb * 64;
  // K range of this wave
  const int b_begin = (int)((int64_t)a.nb * wave / kSmallWaves);
  const int b_end = (int)((int64_t)a.nb * (wave + 1) / kSmallWaves);

  for (int mbase = 0; mbase < M; mbase += 16 * MTM) {
    const int mrem = M - mbase;
    const int MT = mrem >= 16 * MTM ? MTM : (mrem + 15) >> 4;

    // codebook table (this LDS also holds the previous pass's reduction)
    if constexpr (NIB)
      fill_codebook<TBL_NIB_H2>(0, a.ct, a.n_levels, tbl_entries, kSmallWaves);
    else
      fill_codebook<TBL_F16>(0, a.ct, a.n_levels, tbl_entries, kSmallWaves);
    __syncthreads();

    const uint32_t* arow[MTM];
    bool alive[MTM];
#pragma unroll
    for (int i = 0; i < MTM; ++i) {
      const int m = mbase + i * 16 + l16;
      alive[i] = i < MT && m < M;
      arow[i] = a.xp + (int64_t)(alive[i] ? m : 0) * xrow + 16 * g;
    }

    float4v acc[MTM][NT];
#pragma unroll
    for (int i = 0; i < MTM; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};

    // two-stage pipeline over this wave's blocks: block b+1 loads while b computes
    SmallBlk<NT, MTM> cur, nxt;
    if (b_begin < b_end) load_sblk<NIB, NT, MTM>(cur, brow, nrow, arow, alive, b_begin, a.lay);
    for (int b = b_begin; b < b_end; ++b) {
      if (b + 1 < b_end) load_sblk<NIB, NT, MTM>(nxt, brow, nrow, arow, alive, b + 1, a.lay);
      __builtin_amdgcn_sched_barrier(0);
      compute_sblk<NIB, NT, MTM>(acc, cur, tbl, lane4, code_mask, MT);
      cur = nxt;
    }

    // ---- combine the 8 K-slices through LDS (over the table, now unused):
    // red[wave][i][j][lane][4]
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MTM; ++i) {
      if (i >= MT) continue;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        float4* dst = reinterpret_cast<float4*>(
            red + ((((int64_t)wave * MTM + i) * NT + j) * 64 + lane) * 4);
        *dst = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      }
    }
    __syncthreads();

    // outputs: MT*16 rows x TN*16 columns; D element (lane, e) of tile (i, j)
    // is row i*16 + 4*(lane/16) + e, column j*16 + lane%16
    const int outs = MT * 16 * TN * 16;
    for (int o = tid; o < outs; o += kSmallThreads) {
      const int i = o / (TN * 256);
      const int rem = o - i * TN * 256;
      const int j = rem >> 8;
      const int le = rem & 255;  // lane*4 + e
      const int ln = le >> 2, e = le & 3;
      const int m = mbase + i * 16 + 4 * (ln >> 4) + e;
      const int n = blockIdx.x * TN * 16 + j * 16 + (ln & 15);
      if (m >= M || n >= a.N) continue;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kSmallWaves; ++w) s += red[(((int64_t)w * MTM + i) * NT + j) * 256 + le];
      const int64_t row = m;
      if constexpr (EP == SE_F32)
        reinterpret_cast<float*>(a.y)[row * a.ldy + n] = s;
      else
        reinterpret_cast<uint16_t*>(a.y)[row * a.ldy + n] = out16(s, a.bias, n, a.ybf != 0);
    }
    __syncthreads();  // reduction reads done before the next pass's table fill
  }
}

template <bool NIB, int TN, int EP, int MTM>
static int launch_small_t(const SmallArgs& a, hipStream_t st) {
  constexpr int NT = TN;
  auto kern = gemm_small_kernel<NIB, TN, EP, MTM>;
  const int entries = table_entries(NIB, a.n_levels);
  const size_t red_bytes = (size_t)kSmallWaves * MTM * NT * 64 * 16;
  const size_t lds = (size_t)entries * 256 > red_bytes ? (size_t)entries * 256 : red_bytes;
  if (lds > 160 * 1024) return PE_ERR_DIMS;
  static const bool attr_ok = [&] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  const int tiles = (a.N + TN * 16 - 1) / (TN * 16);
  const uint8_t mb = NIB ? (uint8_t)((a.n_levels - 1) * 0x11) : (uint8_t)(a.n_levels - 1);
  kern<<<dim3(tiles), dim3(kSmallThreads), lds, st>>>(a, 0x01010101u * mb, entries);
  return launch_status();
}

template <bool NIB, int EP>
static int launch_small_ep(const SmallArgs& a, hipStream_t st) {
  // one m-tile per pass when M fits in 16 rows, otherwise two
  const bool one = a.M <= 16;
  // two n-tiles per workgroup when that still leaves >= 1 workgroup per CU
  if ((a.N + 31) / 32 >= num_cus())
    return one ? launch_small_t<NIB, 2, EP, 1>(a, st) : launch_small_t<NIB, 2, EP, 2>(a, st);
  return one ? launch_small_t<NIB, 1, EP, 1>(a, st) : launch_small_t<NIB, 1, EP, 2>(a, st);
}

// ---------------------------------------------------------------------------
// Grouped expert products for the MoE path: one workgroup of 8 waves per
// (expert, 128 weight rows); wave w owns the 16-row n-tile 8 x + w (and, for
// SwiGLU, the matching "up" tile at row n + I) over the WHOLE K range, so its
// accumulators are final: no cross-wave reduction, the epilogue runs in
// registers. The expert's activation rows (up to 32 per pass) are staged one
// 128-block at a time into a two-stage LDS ring shared by the 8 waves (chunk c
// of row r at chunk c ^ (r & 15): the 16 rows one ds_read_b128 phase touches
// hit distinct banks), each block loaded D blocks before it is staged; the
// codes stream through a D-deep register ring.
// ---------------------------------------------------------------------------
constexpr int kMoeWaves = 8;
constexpr int kMoeThreads = 64 * kMoeWaves;
constexpr int kMoeRows = 32;  // activation rows per pass (two 16-row m-tiles)
// Rows per pass for experts with many rows (prefill): four m-tiles, so each
// expert's weights are streamed half as often (at about 27 more VGPRs: one
// workgroup per CU)
constexpr int kMoeRowsWide = 64;
// 16-row tiles per wave of the SE_F32 (w2) kernel with nibble codes; 2 keeps
// two workgroups per CU (4 tiles: one, and slower)
constexpr int kMoeF32Tiles = 2;

template <int NT>
struct MoeBlk {
  u32x4v lo[NT];
  u32x4v hi[NT];
  _Float16 nrm[NT];
};

// Weight source of one lane: buffer resources over this expert's codes and
// norms (a real one and a zero-length one) and the lane's row offsets. A
// block past the end reads through the zero-length resource, which returns
// zeros without touching memory, so every ring slot issues the same loads and
// the compiler's vmcnt waits stay exact.
template <int NT>
struct MoeSrc {
  __amdgpu_buffer_rsrc_t codes, codes_none, norms, norms_none;
  uint32_t voff_codes[NT], voff_norms[NT];
};

constexpr int kMoeBufNT = 2;              // non-temporal: every expert block is read once
constexpr int kMoeBufFlags = 0x00020000;  // raw buffer, 32-bit data format

template <bool NIB, int NT>
__device__ __forceinline__ void moe_load_w(MoeBlk<NT>& k, const MoeSrc<NT>& src, int b, int nb,
                                           const WLayout& lay) {
  const bool valid = b < nb;
  const __amdgpu_buffer_rsrc_t rc = valid ? src.codes : src.codes_none;
  const __amdgpu_buffer_rsrc_t rn = valid ? src.norms : src.norms_none;
  const int cb = (int)(b * lay.c_blk), nbk = (int)(b * lay.n_blk * 2);
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    k.lo[j] = __builtin_bit_cast(
        u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rc, src.voff_codes[j], cb, kMoeBufNT));
    if constexpr (!NIB)
      k.hi[j] = __builtin_bit_cast(
          u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rc, src.voff_codes[j], cb + 64, kMoeBufNT));
    k.nrm[j] = __builtin_bit_cast(
        _Float16, __builtin_amdgcn_raw_buffer_load_b16(rn, src.voff_norms[j], nbk, kMoeBufNT));
  }
}

// first weight row (within the expert) of tile j of `wave`: SwiGLU tiles are
// the gate tile's row 16 (8 x + wave) (the up tile adds I at the use); the
// two-tile SE_F32 workgroup x covers rows 256 x .. 256 x + 255, tile j at
// 128 j + 16 wave
template <bool SWI, int NT>
__device__ __forceinline__ int moe_tile_row(int x, int wave, int j) {
  if constexpr (SWI || NT == 1) return (x * kMoeWaves + wave) * 16;
  else return x * (NT * 16 * kMoeWaves) + j * (16 * kMoeWaves) + wave * 16;
}

template <bool NIB, int EP, int D, int MR>
__global__ __launch_bounds__(kMoeThreads) void moe_gemv_kernel(SmallArgs a, uint32_t code_mask,
                                                               int tbl_entries, uint32_t abuf) {
  constexpr bool SWI = EP == SE_SWIGLU || EP == SE_SWIGLU_XTF;
  constexpr int MTX = MR / 16;  // m-tiles per pass
  constexpr int SR = MR / 32;   // staged rows per thread
  // tiles per wave: gate and up (SwiGLU); SE_F32 with nibble codes: two
  // 16-row tiles 128 rows apart, so the workgroup's table fill, staging and
  // prologue serve 256 weight rows
  constexpr int NT = SWI ? 2 : (NIB ? kMoeF32Tiles : 1);
  constexpr uint32_t kStage = MR * 256;  // bytes per LDS stage
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const uint32_t lane4 = (uint32_t)lane << 2;

  const int row0 = a.group_off[blockIdx.y];
  const int M = a.group_off[blockIdx.y + 1] - row0;
  if (M <= 0) return;  // whole workgroup (uniform)
  const uint8_t* codes = a.codes + (int64_t)blockIdx.y * a.codes_stride;
  const uint16_t* norms = a.norms + (int64_t)blockIdx.y * a.norms_stride;

  // this lane's weight rows (clamped; clamped rows are never stored); the
  // resources cover exactly this expert's codes and norms (< 2 GiB: host check)
  const int nt = blockIdx.x * kMoeWaves + wave;
  const int wrows = SWI ? 2 * a.N : a.N;
  MoeSrc<NT> src;
  src.codes = __builtin_amdgcn_make_buffer_rsrc((void*)codes, (short)0, (int)a.codes_stride, kMoeBufFlags);
  src.codes_none = __builtin_amdgcn_make_buffer_rsrc((void*)codes, (short)0, 0, kMoeBufFlags);
  src.norms = __builtin_amdgcn_make_buffer_rsrc((void*)norms, (short)0, (int)(a.norms_stride * 2), kMoeBufFlags);
  src.norms_none = __builtin_amdgcn_make_buffer_rsrc((void*)norms, (short)0, 0, kMoeBufFlags);
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    int n = moe_tile_row<SWI, NT>(blockIdx.x, wave, j) + l16;
    if (n >= a.N) n = a.N - 1;
    if (SWI && j == 1) n += a.N;
    if (n >= wrows) n = wrows - 1;
    src.voff_codes[j] = (uint32_t)(a.lay.codes_off(n) + 16 * g);
    src.voff_norms[j] = (uint32_t)(a.lay.norms_off(n) * 2);
  }

  // codebook table from wave-uniform loads of ct (scalar loads: they do not
  // queue behind the vector loads); entry (hi << 4) | lo = half2(ct[lo],
  // ct[hi]) for nibbles (wave w writes hi = w, w + 8), fp16(ct[e]) for int8
  // (wave w writes entries 16 w .. 16 w + 15 and 16 (w + 8) ..); every lane
  // its own copy. Entries past n_levels are never read (codes are masked).
  (void)tbl_entries;
  {
    const float* __restrict__ ctp = a.ct;
    const int nl = a.n_levels, last = nl - 1;
    if constexpr (NIB) {
      uint32_t h[16];
#pragma unroll
      for (int lo = 0; lo < 16; ++lo) h[lo] = f2h_bits(ctp[lo < nl ? lo : last]);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int hi = wave + kMoeWaves * hh;
        if (hi < nl) {
          uint32_t chi = h[0];
#pragma unroll
          for (int k = 1; k < 16; ++k) chi = hi == k ? h[k] : chi;
          const uint32_t base = ((uint32_t)hi << 12) | lane4;
#pragma unroll
          for (int lo = 0; lo < 16; ++lo)
            if (lo < nl) lds_st32(base + ((uint32_t)lo << 8), h[lo] | (chi << 16));
        }
      }
    } else {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int chunk = wave + kMoeWaves * hh;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int e = chunk * 16 + k;
          if (e < nl) lds_st32(((uint32_t)e << 8) | lane4, f2h_bits(ctp[e]));
        }
      }
    }
  }

  // staging role of this thread: rows sr + 32 k (k < SR), 16-byte chunk sc of
  // the 256-byte block row
  static_assert(kMoeThreads == 16 * 32, "one 16-byte chunk of 32 staged rows per thread pass");
  const int sr = tid >> 4, sc = tid & 15;
  uint32_t sdst[SR];
#pragma unroll
  for (int k = 0; k < SR; ++k)
    sdst[k] = (uint32_t)(sr + 32 * k) * 256u + ((uint32_t)(sc ^ (sr & 15)) << 4);
  const int64_t xrow = (int64_t)a.nb * 64;  // uint32 per activation row

  for (int mbase = 0; mbase < M; mbase += MR) {
    const int mrem = M - mbase;
    const int MT = mrem >= MR ? MTX : (mrem + 15) >> 4;
    // Rows past M re-read row M - 1 and blocks past the end re-read the last
    // block: every lane issues the same loads on every path, so the
    // compiler's vmcnt waits stay exact (a conditional load made it wait for
    // every outstanding load). Rows past M only feed outputs never stored.
    const uint32_t* ssrc[SR];
#pragma unroll
    for (int k = 0; k < SR; ++k) {
      const int rr = sr + 32 * k;
      int srow = row0 + (mbase + rr < M ? mbase + rr : M - 1);
      if (a.a_rows) srow = a.a_rows[srow];
      ssrc[k] = a.xp + (int64_t)srow * xrow + sc * 4;
    }
    auto lda = [&](int k, int b) -> u32x4v {
      b = b < a.nb ? b : a.nb - 1;
      return *reinterpret_cast<const u32x4v*>(ssrc[k] + (int64_t)b * 64);
    };
    float4v acc[MTX][NT];
#pragma unroll
    for (int i = 0; i < MTX; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};

    // activation FIFO: block q is loaded D blocks before it is staged and
    // waits in sreg[q % D]. Blocks 0 .. D - 1 are loaded before the weight
    // ring, so that staging block 0 waits for its own rows only (loads
    // complete in issue order); block D after block 0 is staged.
    u32x4v sreg[D][SR];
#pragma unroll
    for (int q = 0; q < D; ++q)
#pragma unroll
      for (int k = 0; k < SR; ++k) sreg[q][k] = lda(k, q);
    __builtin_amdgcn_sched_barrier(0);
    MoeBlk<NT> ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      moe_load_w<NIB, NT>(ring[d], src, d, a.nb, a.lay);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int k = 0; k < SR; ++k) {
      lds_st128(abuf + sdst[k], sreg[0][k]);
      sreg[0][k] = lda(k, D);
    }
    __syncthreads();  // codebook table and stage 0 written

    // A row of this lane in m-tile i: activation row 16 i + l16 of the stage.
    // The loop is compiled once per m-tile count, so that no branch on MT
    // splits a block's lookups and MFMAs into separately scheduled pieces (a
    // runtime test there left every lookup's latency exposed).
    auto kloop = [&](auto mt_) {
      constexpr int MTC = decltype(mt_)::value;
      for (int b0 = 0; b0 < a.nb; b0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int b = b0 + d;
          if (b < a.nb) {  // uniform
            const uint32_t st = abuf + (uint32_t)(b & 1) * kStage;
            // the weights are scaled by their block norm (fp16) before the
            // MFMA, which accumulates straight into acc; the slot's norms are
            // then dead once the last slab is dequantized, before the slot's
            // next loads are issued (a value still live there is copied at the
            // loop edge, and the copy waits for the load to arrive)
            half2v nrm2[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) nrm2[j] = half2v{ring[d].nrm[j], ring[d].nrm[j]};
            // each activation fragment is read from LDS once and feeds the
            // gate and up tiles alike
            // software pipeline over the four 32-wide slabs: the activation
            // reads and codebook lookups of slab t + 1 are issued before the
            // MFMAs of slab t
            constexpr int TV = NIB ? 4 : 8;  // lookups per (tile, slab)
            auto issue = [&](auto t_, u32x4v (&af)[MTX], uint32_t (&tv)[NT][TV]) {
              constexpr int t = decltype(t_)::value;
#pragma unroll
              for (int i = 0; i < MTC; ++i) {
                const int r = 16 * i + l16;
                af[i] = lds_ld128(st + (uint32_t)r * 256u + ((uint32_t)((4 * g + t) ^ (r & 15)) << 4));
              }
#pragma unroll
              for (int j = 0; j < NT; ++j) {
                const uint32_t wl = ring[d].lo[j][t] & code_mask;
                tv[j][0] = lds_ld32(tbl_addr<0>(wl, lane4));
                tv[j][1] = lds_ld32(tbl_addr<1>(wl, lane4));
                tv[j][2] = lds_ld32(tbl_addr<2>(wl, lane4));
                tv[j][3] = lds_ld32(tbl_addr<3>(wl, lane4));
                if constexpr (!NIB) {
                  const uint32_t wh = ring[d].hi[j][t] & code_mask;
                  tv[j][TV - 4] = lds_ld32(tbl_addr<0>(wh, lane4));
                  tv[j][TV - 3] = lds_ld32(tbl_addr<1>(wh, lane4));
                  tv[j][TV - 2] = lds_ld32(tbl_addr<2>(wh, lane4));
                  tv[j][TV - 1] = lds_ld32(tbl_addr<3>(wh, lane4));
                }
              }
            };
            auto mma = [&](const u32x4v (&af)[MTX], const uint32_t (&tv)[NT][TV]) {
#pragma unroll
              for (int j = 0; j < NT; ++j) {
                u32x4v bw;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  // int8: (lo16 of the first-position entry, lo16 of the second)
                  const uint32_t p = NIB ? tv[j][q] : __builtin_amdgcn_perm(tv[j][TV - 4 + q], tv[j][q], 0x05040100u);
                  bw[q] = __builtin_bit_cast(uint32_t, as_h2(p) * nrm2[j]);
                }
                const half8v bf = __builtin_bit_cast(half8v, bw);
#pragma unroll
                for (int i = 0; i < MTC; ++i)
                  acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8v, af[i]), bf,
                                                                     acc[i][j], 0, 0, 0);
              }
            };
            u32x4v af0[MTX], af1[MTX];
            uint32_t tv0[NT][TV], tv1[NT][TV];
            issue(std::integral_constant<int, 0>{}, af0, tv0);
            issue(std::integral_constant<int, 1>{}, af1, tv1);
            __builtin_amdgcn_sched_barrier(0);
            mma(af0, tv0);
            issue(std::integral_constant<int, 2>{}, af0, tv0);
            __builtin_amdgcn_sched_barrier(0);
            mma(af1, tv1);
            issue(std::integral_constant<int, 3>{}, af1, tv1);
            __builtin_amdgcn_sched_barrier(0);
            mma(af0, tv0);
            mma(af1, tv1);
            __builtin_amdgcn_sched_barrier(0);
            moe_load_w<NIB, NT>(ring[d], src, b + D, a.nb, a.lay);
            // next stage: block b + 1 into the other buffer (its readers, block
            // b - 1, finished before the previous barrier); load block b + 1 + D
#pragma unroll
            for (int k = 0; k < SR; ++k) {
              if (b + 1 < a.nb) lds_st128(abuf + (uint32_t)((b + 1) & 1) * kStage + sdst[k], sreg[(d + 1) % D][k]);
              sreg[(d + 1) % D][k] = lda(k, b + 1 + D);
            }
            __syncthreads();
          }
        }
      }
    };
    if constexpr (MTX == 4) {
      if (MT == 4) kloop(std::integral_constant<int, 4>{});
      else if (MT == 3) kloop(std::integral_constant<int, 3>{});
      else if (MT == 2) kloop(std::integral_constant<int, 2>{});
      else kloop(std::integral_constant<int, 1>{});
    } else {
      if (MT == 2) kloop(std::integral_constant<int, 2>{});
      else kloop(std::integral_constant<int, 1>{});
    }

    if constexpr (EP == SE_SWIGLU_XTF) {
      // The workgroup's 128 columns are one 128-block of h: silu(gate) * up
      // as fp16 into an LDS tile [MR rows][128] (over the stage buffers; the
      // barrier above ended their reads), then one 16-lane group per row
      // transforms its block and writes pair f16 (x_tf[p], x_tf[p + 64]) at
      // dword p of row (row0 + m), block blockIdx.x. Columns >= N are zero
      // (the padding up to a whole block).
      const int n = nt * 16 + l16;
#pragma unroll
      for (int i = 0; i < MTX; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 16 * i + 4 * g + e;
          const float s = acc[i][0][e], u = acc[i][1][e];
          const _Float16 hv = n < a.N ? (_Float16)(s / (1.f + __expf(-s)) * u) : (_Float16)0.f;
          lds_st16(abuf + (uint32_t)r * 256u + (uint32_t)(wave * 16 + l16) * 2u,
                   __builtin_bit_cast(uint16_t, hv));
        }
      }
      __syncthreads();
      const int q = tid & 15;  // 32 groups of 16 lanes: rows tid / 16 + 32 k
#pragma unroll
      for (int k = 0; k < SR; ++k) {
        const int r = (tid >> 4) + 32 * k;
        float v[8];
        {
          const u32x4v w = lds_ld128(abuf + (uint32_t)r * 256u + (uint32_t)q * 16u);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            v[2 * c] = h2f((uint16_t)(w[c] & 0xffff));
            v[2 * c + 1] = h2f((uint16_t)(w[c] >> 16));
          }
        }
        fwht128_group16(v, q);
        const int m = mbase + r;
        const bool live = r < 16 * MT && m < M;
        const int64_t prow = live ? (int64_t)(row0 + m) : 0;  // no address past the rows
        store_pair_block(v, q, reinterpret_cast<uint32_t*>(a.y) + prow * (a.ldy / 2) + (int64_t)blockIdx.x * 64, live);
      }
    } else {
    // epilogue from registers: D element (lane, e) of m-tile i is row
    // 16 i + 4 (lane / 16) + e, column moe_tile_row + lane % 16
#pragma unroll
    for (int j = 0; j < (SWI ? 1 : NT); ++j) {
      const int n = moe_tile_row<SWI, NT>(blockIdx.x, wave, j) + l16;
      if (n < a.N) {
#pragma unroll
        for (int i = 0; i < MTX; ++i) {
          if (i >= MT) continue;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = mbase + 16 * i + 4 * g + e;
            if (m >= M) continue;
            const int64_t row = row0 + m;
            const float s = acc[i][j][e];
            if constexpr (EP == SE_F32) {
              reinterpret_cast<float*>(a.y)[row * a.ldy + n] = s;
            } else {
              const float u = acc[i][NT - 1][e];
              const float act = s / (1.f + __expf(-s)) * u;
              reinterpret_cast<_Float16*>(a.y)[row * a.ldy + n] = (_Float16)act;
            }
          }
        }
      }
    }
    }
    __syncthreads();  // stage buffers free before the next pass
  }
}

template <bool NIB, int EP, int MR>
static int launch_moe_t(const SmallArgs& a, int groups, hipStream_t st) {
  constexpr int D = 2;  // 2 blocks in flight per wave: measured faster than 3 or 4
  auto kern = moe_gemv_kernel<NIB, EP, D, MR>;
  const int entries = table_entries(NIB, a.n_levels);
  const uint32_t abuf = (uint32_t)round_up((size_t)entries * 256, 256);
  const size_t lds = abuf + 2 * (size_t)MR * 256;
  if (lds > 160 * 1024) return PE_ERR_DIMS;
  static const bool attr_ok = [&] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  constexpr bool SWI = EP == SE_SWIGLU || EP == SE_SWIGLU_XTF;
  const int rows_per_wg = 16 * kMoeWaves * (SWI ? 1 : (NIB ? kMoeF32Tiles : 1));
  const int wgs = (a.N + rows_per_wg - 1) / rows_per_wg;
  const uint8_t mb = NIB ? (uint8_t)((a.n_levels - 1) * 0x11) : (uint8_t)(a.n_levels - 1);
  kern<<<dim3(wgs, groups), dim3(kMoeThreads), lds, st>>>(a, 0x01010101u * mb, entries, abuf);
  return launch_status();
}

// Rows per pass: 64 when the experts hold at least 64 rows on average (a.M:
// the pairs over all experts), else 32 (two workgroups per CU).
template <bool NIB, int EP>
static int launch_moe_mr(const SmallArgs& a, int groups, hipStream_t st) {
  if ((int64_t)a.M >= (int64_t)kMoeRowsWide * groups)
    return launch_moe_t<NIB, EP, kMoeRowsWide>(a, groups, st);
  return launch_moe_t<NIB, EP, kMoeRows>(a, groups, st);
}

int moe_grouped(bool nibble, int epilogue, const SmallArgs& a, int groups, hipStream_t st) {
  if (!a.group_off || a.nb <= 0 || a.N <= 0) return PE_ERR_DIMS;
  // one expert's codes and norms are addressed by 32-bit buffer offsets
  if (a.codes_stride >= ((int64_t)1 << 31) || a.norms_stride * 2 >= ((int64_t)1 << 31))
    return PE_ERR_DIMS;
  switch (epilogue) {
    case SE_F32: return nibble ? launch_moe_mr<true, SE_F32>(a, groups, st) : launch_moe_mr<false, SE_F32>(a, groups, st);
    case SE_SWIGLU: return nibble ? launch_moe_mr<true, SE_SWIGLU>(a, groups, st) : launch_moe_mr<false, SE_SWIGLU>(a, groups, st);
    case SE_SWIGLU_XTF:
      if (a.ldy % 128) return PE_ERR_DIMS;  // rows of whole 128-blocks
      return nibble ? launch_moe_mr<true, SE_SWIGLU_XTF>(a, groups, st) : launch_moe_mr<false, SE_SWIGLU_XTF>(a, groups, st);
    default: return PE_ERR_DTYPE;
  }
}

int gemm_small(bool nibble, int epilogue, const SmallArgs& a, hipStream_t st) {
  if (a.M <= 0 || a.N <= 0 || a.nb <= 0) return PE_ERR_DIMS;
  switch (epilogue) {
    case SE_F32: return nibble ? launch_small_ep<true, SE_F32>(a, st) : launch_small_ep<false, SE_F32>(a, st);
    case SE_F16: return nibble ? launch_small_ep<true, SE_F16>(a, st) : launch_small_ep<false, SE_F16>(a, st);
    default: return PE_ERR_DTYPE;
  }
}

}  // namespace pe
