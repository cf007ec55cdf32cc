// Prefill GEMM for gfx950: Y[M, N] = X_tf[M, K] . W~[N, K]^T with
// W~[n, k] = ct[code[n, k]] * norm[n, k / 128], fp16 operands on MFMA
// (v_mfma_f32_32x32x16_f16), fp32 accumulate.
//
// Replaces polar_gemm / polar_gemm_packed (kernels/polar_gemm.py:81-171,
// 211-418), which gather ct per tile and run tl.dot on fp32 tiles.
//
// Structure (a workgroup of WM x WN waves, wave tile 32*TMW x 32*TNW; the
// dispatcher uses 1 x WN rows of waves, see pick_gemm_tile):
//  * K advances in half-blocks of 64 activations = 32 pairs; pair p of a
//    128-block is (x[p], x[p + 64]), the two positions one nibble byte codes;
//  * the activation tile (BM rows x 32 pairs, pair-f16) is staged global ->
//    registers -> LDS, double-buffered, rows padded to 144 B so the
//    ds_read_b128 of 8 consecutive rows hit distinct banks;
//  * the weight operand never touches LDS as data: every wave loads its own
//    codes (one dwordx4 per row per half-block for nibbles) one half-block
//    ahead, and dequantizes in registers through the per-lane LDS codebook
//    table (one v_perm + one ds_read_b32 per code byte) and a v_pk_mul_f16 by
//    the block norm;
//  * k-order inside an MFMA is the pair order: lane half h of slab t carries
//    pairs 16h + 4t + j, j = 0..3, as (lo, hi) halves, identically for A and B.
//  * workgroup ids are remapped so that each XCD (ids round-robin over 8)
//    walks a contiguous range of tiles (M-tile fastest) and shares A/B in its
//    own L2.

#include <type_traits>

#include "pe_internal.h"

namespace pe {

constexpr int kAStride = 144;  // bytes per A-tile row in LDS (128 + 16 pad)

// OM_F16: 16-bit output, bfloat16 when ybf (bias of the same type)
template <int OM>
__device__ __forceinline__ void store_out(void* y, int64_t ldy, int m, int n, float v,
                                          const uint16_t* bias, bool ybf) {
  if constexpr (OM == 0) {
    reinterpret_cast<float*>(y)[(int64_t)m * ldy + n] = v;
  } else {
    reinterpret_cast<uint16_t*>(y)[(int64_t)m * ldy + n] = out16(v, bias, n, ybf);
  }
}

// Dequantize one slab worth of B for one MFMA n-tile: 4 pair dwords.
template <bool NIB>
__device__ __forceinline__ half8v dequant_slab(const char* tbl, uint32_t wlo, uint32_t whi,
                                               uint32_t lane4, half2v nrm2) {
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
    // (lo16 of a, lo16 of b): bytes a0,a1,b0,b1 -> selector 0x05040100 over {b, a}
    p[0] = __builtin_amdgcn_perm(b0, a0, 0x05040100u);
    p[1] = __builtin_amdgcn_perm(b1, a1, 0x05040100u);
    p[2] = __builtin_amdgcn_perm(b2, a2, 0x05040100u);
    p[3] = __builtin_amdgcn_perm(b3, a3, 0x05040100u);
  }
  half8v r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const half2v v = as_h2(p[j]) * nrm2;
    r[2 * j] = v[0];
    r[2 * j + 1] = v[1];
  }
  return r;
}

// B operand registers of one half-block K-tile for the wave's TNW n-tiles
template <bool NIB, int TNW>
struct BTile {
  u32x4v lo[TNW];
  u32x4v hi[TNW];  // int8 codes only: bytes at +64 (the pair's second position)
  uint16_t nrm[TNW];
};

template <bool NIB, int TNW>
__device__ __forceinline__ void load_btile(BTile<NIB, TNW>& t, const uint8_t* const (&b_row)[TNW],
                                           const uint16_t* const (&n_row)[TNW], int kt,
                                           int64_t c_blk, int64_t n_blk) {
  const int b = kt >> 1, half = kt & 1;
#pragma unroll
  for (int j = 0; j < TNW; ++j) {
    const uint8_t* pc = b_row[j] + b * c_blk + half * 32;
    t.lo[j] = ld_nt16v(pc);
    if constexpr (!NIB) t.hi[j] = ld_nt16v(pc + 64);
    t.nrm[j] = n_row[j][b * n_blk];
  }
}

template <int KA>
__device__ __forceinline__ void load_atile(u32x4v (&r)[KA], const uint32_t* const (&a_src)[KA],
                                           int kt) {
  const int off = (kt >> 1) * 64 + (kt & 1) * 32;
#pragma unroll
  for (int i = 0; i < KA; ++i) r[i] = *reinterpret_cast<const u32x4v*>(a_src[i] + off);
}

template <int KA>
__device__ __forceinline__ void store_atile(char* dst, const u32x4v (&r)[KA],
                                            const int (&a_dst)[KA]) {
#pragma unroll
  for (int i = 0; i < KA; ++i) *reinterpret_cast<u32x4v*>(dst + a_dst[i]) = r[i];
}

// One half-block K-tile of MFMA work on LDS A buffer `abase`.
template <bool NIB, int TMW, int TNW>
__device__ __forceinline__ void mma_ktile(float16v (&acc)[TMW][TNW], const BTile<NIB, TNW>& bt,
                                          const char* abase, const char* tbl, uint32_t lane4,
                                          uint32_t code_mask) {
  half2v nrm2[TNW];
#pragma unroll
  for (int j = 0; j < TNW; ++j) {
    const _Float16 nh = __builtin_bit_cast(_Float16, bt.nrm[j]);
    nrm2[j] = half2v{nh, nh};
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    half8v af[TMW];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
      af[i] = __builtin_bit_cast(half8v, *reinterpret_cast<const u32x4v*>(abase + i * 32 * kAStride + 16 * t));
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
      const uint32_t wl = bt.lo[j][t] & code_mask;
      uint32_t wh = 0;
      if constexpr (!NIB) wh = bt.hi[j][t] & code_mask;
      const half8v bf = dequant_slab<NIB>(tbl, wl, wh, lane4, nrm2[j]);
#pragma unroll
      for (int i = 0; i < TMW; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf, acc[i][j], 0, 0, 0);
    }
  }
}

// WM x WN waves, wave tile 32 TMW x 32 TNW.
template <bool NIB, int TMW, int TNW, int WM, int WN, int OM>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms,
    const float* __restrict__ ct, int n_levels, uint32_t code_mask, int tbl_entries,
    const uint32_t* __restrict__ xp, void* __restrict__ y, const uint16_t* __restrict__ bias,
    int M, int N, int nb, int64_t ldy, int tiles_m, int tiles_total, WLayout lay, int ybf) {
  constexpr int NT = WM * WN * 64;
  constexpr int BM = WM * TMW * 32;
  constexpr int BN = WN * TNW * 32;
  constexpr int KA = BM * 8 / NT;  // uint4 of A per thread per half-block
  static_assert(KA * NT == BM * 8, "A tile must split evenly over the threads");
  extern __shared__ uint4 smem4[];
  char* smem = reinterpret_cast<char*>(smem4);
  char* tbl = smem;
  char* abuf = smem + tbl_entries * 256;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int h = lane >> 5, l32 = lane & 31;
  const uint32_t lane4 = (uint32_t)lane << 2;

  // XCD-aware tile order: ids are dealt round-robin to 8 XCDs; give each XCD a
  // contiguous range of logical tiles.
  int wid = blockIdx.x;
  if ((tiles_total & 7) == 0) wid = (wid & 7) * (tiles_total >> 3) + (wid >> 3);
  const int tm = wid % tiles_m, tn = wid / tiles_m;
  const int m0 = tm * BM, n0 = tn * BN;

  // codebook values now, the table once the first A and B loads are issued
  float cbr[4];
  codebook_regs(cbr, ct, n_levels);

  // K range of this workgroup: gridDim.z groups split the 128-blocks; with
  // more than one, each writes fp32 partial sums to its slab [M][ldy] of y
  // (one group: the whole K range, y itself)
  const int kb0 = (int)((int64_t)nb * blockIdx.z / gridDim.z);
  const int nbz = (int)((int64_t)nb * (blockIdx.z + 1) / gridDim.z) - kb0;
  y = reinterpret_cast<char*>(y) + (int64_t)blockIdx.z * M * ldy * (OM == 0 ? 4 : 2);

  // A loader: thread t moves uint4 q = t + NT i (row q >> 3, 16-byte col q & 7)
  const int64_t xrow_u32 = (int64_t)nb * 64;
  const uint32_t* a_src[KA];
  int a_dst[KA];
#pragma unroll
  for (int i = 0; i < KA; ++i) {
    const int q = tid + NT * i;
    const int r = q >> 3, c = q & 7;
    int m = m0 + r;
    if (m >= M) m = M - 1;  // clamped rows feed discarded outputs only
    a_src[i] = xp + (int64_t)m * xrow_u32 + (int64_t)kb0 * 64 + c * 4;
    a_dst[i] = r * kAStride + c * 16;
  }
  // B rows of this wave
  const uint8_t* b_row[TNW];
  const uint16_t* n_row[TNW];
#pragma unroll
  for (int j = 0; j < TNW; ++j) {
    int n = n0 + wn * TNW * 32 + j * 32 + l32;
    if (n >= N) n = N - 1;
    b_row[j] = codes + lay.codes_off(n) + 16 * h + (int64_t)kb0 * lay.c_blk;
    n_row[j] = norms + lay.norms_off(n) + (int64_t)kb0 * lay.n_blk;
  }

  float16v acc[TMW][TNW];
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int nkt = 2 * nbz;  // half-block K-tiles of this K range (always even)
  const int a_off = (wm * TMW * 32 + l32) * kAStride + 64 * h;
  u32x4v ar[KA];
  BTile<NIB, TNW> b0, b1;

  // prologue: A(0) -> LDS 0, A(1) -> regs, B(0), B(1) -> regs
  load_atile<KA>(ar, a_src, 0);
  load_btile<NIB, TNW>(b0, b_row, n_row, 0, lay.c_blk, lay.n_blk);
  load_btile<NIB, TNW>(b1, b_row, n_row, 1, lay.c_blk, lay.n_blk);
  if constexpr (NIB) fill_codebook_from<TBL_NIB_H2>(0, cbr, tbl_entries, NT / 64);
  else fill_codebook_from<TBL_F16>(0, cbr, tbl_entries, NT / 64);
  store_atile<KA>(abuf, ar, a_dst);
  load_atile<KA>(ar, a_src, 1);
  __syncthreads();

  for (int kt = 0; kt < nkt; kt += 2) {
    // ---- even half-block: B from b0, A from LDS buffer 0
    {
      const BTile<NIB, TNW> cur = b0;
      if (kt + 2 < nkt) load_btile<NIB, TNW>(b0, b_row, n_row, kt + 2, lay.c_blk, lay.n_blk);
      mma_ktile<NIB, TMW, TNW>(acc, cur, abuf + a_off, tbl, lane4, code_mask);
      store_atile<KA>(abuf + BM * kAStride, ar, a_dst);  // A(kt+1) -> LDS 1
      if (kt + 2 < nkt) load_atile<KA>(ar, a_src, kt + 2);
      __syncthreads();
    }
    // ---- odd half-block: B from b1, A from LDS buffer 1
    {
      const BTile<NIB, TNW> cur = b1;
      if (kt + 3 < nkt) load_btile<NIB, TNW>(b1, b_row, n_row, kt + 3, lay.c_blk, lay.n_blk);
      mma_ktile<NIB, TMW, TNW>(acc, cur, abuf + BM * kAStride + a_off, tbl, lane4, code_mask);
      if (kt + 2 < nkt) {
        store_atile<KA>(abuf, ar, a_dst);  // A(kt+2) -> LDS 0
        load_atile<KA>(ar, a_src, kt + 3);
      }
      __syncthreads();
    }
  }

  // ---- epilogue: acc[i][j][e] -> row 8*(e/4) + 4*h + e%4, col l32
#pragma unroll
  for (int i = 0; i < TMW; ++i) {
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
      const int n = n0 + wn * TNW * 32 + j * 32 + l32;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * TMW * 32 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (m < M) store_out<OM>(y, ldy, m, n, acc[i][j][e], bias, ybf != 0);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Four-wave variant: one wave per SIMD, each wave owning BM = 32 TMW rows x
// 32 NTW columns (NTW 32-column n-tiles: 2 or 3), workgroup tile BM x 128 NTW.
// Per MFMA it moves (TMW + NTW) / (NTW TMW) KB of operands through LDS instead
// of (TMW + 1) / TMW, and every weight column is still dequantized by exactly
// one wave; NTW = 3 (384 columns) cuts the LDS reads, A-tile stores and
// barriers per MFMA by a further quarter to a third where its tiles fill the
// CUs in as few rounds.
//  * A half-block tiles sit in a ring of six LDS buffers (96 KB beside the
//    64 KB table), stored four half-blocks ahead, with one barrier per two
//    half-blocks: the tile of half-block kt + 1 is complete before the barrier
//    that precedes kt, so the first slab of kt + 1 is read ahead while kt
//    still computes.
//  * Within a half-block every slab's operands (A fragments and codebook
//    lookups) are issued one slab ahead of its MFMAs.
//  * Codes ride a ring of four half-block slots (issued three half-blocks
//    ahead), activations a ring of two register stages (loaded six ahead,
//    stored four ahead); the loop
//    body covers four half-blocks so every ring index is static. Loads past the
//    end are clamped to the last half-block, so each wait count is static too.
// Requires an even number of 128-blocks.
// ---------------------------------------------------------------------------
// Codes of one half-block for the wave's NTW n-tiles. Norms are kept
// zero-extended to 32 bits: 16-bit members next to vectors made the compiler
// keep the slot in memory.
template <bool NIB, int NTW>
struct BSlot4 {
  u32x4v lo[NTW];
  u32x4v hi[NIB ? 1 : NTW];  // int8 codes only: bytes at +64
  uint32_t nrm[NTW];
};

template <bool NIB, int TMW, int NTW>
struct Frag4 {
  half8v a[TMW];
  uint32_t raw[NTW][NIB ? 4 : 8];
};

// A tiles of the four-wave kernel: 128-byte rows (32 pairs), 16-byte chunk c
// of row r stored at chunk c ^ ((r >> 1) & 7). A ds_read_b128 phase serves 16
// lanes (rows r0..r0+15, one chunk each) from the 64 four-byte banks: a row
// spans half the banks (even rows the low half, odd rows the high half), so
// the eight rows of each parity need eight distinct chunks. The plain
// c ^ (r & 7) repeats after eight rows and made every A read a 2-way conflict.
constexpr int kARow4 = 128;
// A half-block tiles in the four-wave kernel's LDS ring (16 KB each at 128
// rows): A(kt + 4) is stored while A(kt) is read, one barrier per two tiles
constexpr int kA4Ring = 6;
__device__ __forceinline__ uint32_t a4_swz(int r) { return (uint32_t)((r >> 1) & 7); }

// ACT <= TMW: the m-tiles that hold live rows (the others' A fragments are
// not read and their MFMAs not issued; their accumulators stay zero)
template <bool NIB, int TMW, int NTW, bool MASK, int ACT = TMW>
__device__ __forceinline__ void issue_frag4(Frag4<NIB, TMW, NTW>& f, uint32_t aaddr, int t,
                                            const BSlot4<NIB, NTW>& bt, uint32_t lane4,
                                            uint32_t code_mask) {
  // aaddr: this lane's row and swizzled chunk of slab t in m-tile 0
#pragma unroll
  for (int i = 0; i < ACT; ++i)
    f.a[i] = __builtin_bit_cast(half8v, lds_ld128(aaddr + i * 32 * kARow4));
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    uint32_t wl = bt.lo[j][t];
    if constexpr (MASK) wl &= code_mask;
    f.raw[j][0] = lds_ld32(tbl_addr<0>(wl, lane4));
    f.raw[j][1] = lds_ld32(tbl_addr<1>(wl, lane4));
    f.raw[j][2] = lds_ld32(tbl_addr<2>(wl, lane4));
    f.raw[j][3] = lds_ld32(tbl_addr<3>(wl, lane4));
    if constexpr (!NIB) {
      uint32_t wh = bt.hi[j][t];
      if constexpr (MASK) wh &= code_mask;
      f.raw[j][4] = lds_ld32(tbl_addr<0>(wh, lane4));
      f.raw[j][5] = lds_ld32(tbl_addr<1>(wh, lane4));
      f.raw[j][6] = lds_ld32(tbl_addr<2>(wh, lane4));
      f.raw[j][7] = lds_ld32(tbl_addr<3>(wh, lane4));
    }
  }
}

template <bool NIB, int TMW, int NTW, int ACT = TMW>
__device__ __forceinline__ void mma_frag4(float16v (&acc)[TMW][NTW], const Frag4<NIB, TMW, NTW>& f,
                                          const BSlot4<NIB, NTW>& bt) {
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    const _Float16 nh = __builtin_bit_cast(_Float16, (uint16_t)bt.nrm[j]);
    const half2v nrm2{nh, nh};
    half8v bf;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t p = f.raw[j][q];
      // int8: (lo16 of the first-position entry, lo16 of the second)
      if constexpr (!NIB) p = __builtin_amdgcn_perm(f.raw[j][4 + q], p, 0x05040100u);
      const half2v v = as_h2(p) * nrm2;
      bf[2 * q] = v[0];
      bf[2 * q + 1] = v[1];
    }
    // weights as the MFMA's A operand: the accumulator comes out transposed,
    // lane = output row, four consecutive output columns per register group
#pragma unroll
    for (int i = 0; i < ACT; ++i)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf, f.a[i], acc[i][j], 0, 0, 0);
  }
}

// Output tile through LDS: the transposed accumulators (lane = row m, groups
// of four consecutive columns) are written as 8- or 16-byte pieces into a
// row-major staging tile, then copied to y in 16-byte coalesced stores.
template <int TMW, int NTW, int OM>
__device__ __forceinline__ void store_tile4(const float16v (&acc)[TMW][NTW], void* __restrict__ y,
                                            int64_t ldy, const uint16_t* __restrict__ bias, int M,
                                            int N, int m0, int n0, int vec_ok, bool ybf) {
  constexpr int BM = TMW * 32, BN = 128 * NTW;
  constexpr int ES = OM == OM_F16 ? 2 : 4;
  constexpr uint32_t OSTR = BN * ES + 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  __syncthreads();  // every wave is done with the ring and the table
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t addr = (uint32_t)(32 * i + l32) * OSTR +
                              (uint32_t)(wave * 32 * NTW + 32 * j + 8 * g + 4 * h) * ES;
        // element values first: a bit_cast applied to a vector element
        // lvalue reads element 0 of the vector with this compiler
        const float v0 = acc[i][j][4 * g], v1 = acc[i][j][4 * g + 1];
        const float v2 = acc[i][j][4 * g + 2], v3 = acc[i][j][4 * g + 3];
        if constexpr (OM == OM_F16) {
          lds_st64(addr, u32x2v{pack16x2(v0, v1, ybf), pack16x2(v2, v3, ybf)});
        } else {
          lds_st128(addr, u32x4v{__builtin_bit_cast(uint32_t, v0), __builtin_bit_cast(uint32_t, v1),
                                 __builtin_bit_cast(uint32_t, v2), __builtin_bit_cast(uint32_t, v3)});
        }
      }
  __syncthreads();
  constexpr int CPR = BN * ES / 16;  // 16-byte chunks per row
  constexpr int EPC = 16 / ES;       // elements per chunk
  for (int q = tid; q < BM * CPR; q += 256) {
    const int r = q / CPR, c = q % CPR;
    const int m = m0 + r, n = n0 + c * EPC;
    if (m >= M || n >= N) continue;
    u32x4v v = lds_ld128((uint32_t)r * OSTR + (uint32_t)c * 16u);
    if constexpr (OM == OM_F16) {
      if (bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = f16or_bf((uint16_t)(v[e] & 0xffff), ybf);
          const float x1 = f16or_bf((uint16_t)(v[e] >> 16), ybf);
          const int nn = n + 2 * e;
          const float b0 = nn < N ? f16or_bf(bias[nn], ybf) : 0.f;
          const float b1 = nn + 1 < N ? f16or_bf(bias[nn + 1], ybf) : 0.f;
          v[e] = pack16x2(x0 + b0, x1 + b1, ybf);
        }
      }
    }
    char* dst = reinterpret_cast<char*>(y) + ((int64_t)m * ldy + n) * ES;
    if (vec_ok && n + EPC <= N) {
      *reinterpret_cast<u32x4v*>(dst) = v;
    } else {
      const int cnt = N - n < EPC ? N - n : EPC;
      for (int e = 0; e < cnt; ++e) {
        if constexpr (OM == OM_F16)
          reinterpret_cast<uint16_t*>(dst)[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
        else
          reinterpret_cast<uint32_t*>(dst)[e] = v[e];
      }
    }
  }
}

// Grouped form (experts): the row tiles of all groups, in group order, are
// numbered consecutively; tile t of the grid belongs to the group whose tiles
// cover t. A wave finds it from the group offsets with a prefix sum over the
// lanes (64 groups per step). False past the last tile.
template <int BM>
__device__ __forceinline__ bool group_tile(const GemmGroup& g, int t, int lane, int& e_out,
                                           int& mt_out) {
  int base = 0;
  for (int q = 0; q * 64 < g.groups; ++q) {  // uniform
    const int e = q * 64 + lane;
    const int cnt = e < g.groups ? g.offsets[e + 1] - g.offsets[e] : 0;
    const int tiles = (cnt + BM - 1) / BM;
    int incl = tiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    const int first = base + incl - tiles;
    const unsigned long long hit = __ballot(tiles > 0 && t >= first && t < first + tiles);
    if (hit) {
      const int l = __ffsll((long long)hit) - 1;
      e_out = __builtin_amdgcn_readfirstlane(q * 64 + l);
      mt_out = __builtin_amdgcn_readfirstlane(t - __shfl(first, l, 64));
      return true;
    }
    base += __shfl(incl, 63, 64);
  }
  return false;
}

// SwiGLU epilogue of the grouped four-wave kernel: h = silu(gate) * up for
// the tile's 128 columns (one 128-block of h) into an fp16 LDS tile [BM][128],
// then each row through the FWHT-128 (16 lanes per row) into pair-f16 x_tf
// layout at y + (row0 + m) * (ldy / 2) u32, block n0 / 128. Columns >= I are
// zero.
template <int TMW>
__device__ __forceinline__ void swiglu_xtf_tile4(const float16v (&acc)[TMW][2], uint32_t* __restrict__ y,
                                                 int64_t ldy, int M, int I, int64_t row0, int m0, int n0) {
  constexpr int BM = TMW * 32;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  __syncthreads();  // every wave is done with the ring and the table
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int col = wave * 32 + 8 * gq + 4 * h;  // four consecutive columns
      float hv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float s = acc[i][0][4 * gq + e], u = acc[i][1][4 * gq + e];
        hv[e] = n0 + col + e < I ? s / (1.f + __expf(-s)) * u : 0.f;
      }
      const uint32_t addr = (uint32_t)(32 * i + l32) * 256u + (uint32_t)col * 2u;
      lds_st64(addr, u32x2v{pack16x2(hv[0], hv[1], false), pack16x2(hv[2], hv[3], false)});
    }
  __syncthreads();
  const int q = tid & 15;  // 16 groups of 16 lanes: rows tid / 16 + 16 k
#pragma unroll
  for (int k = 0; k < BM / 16; ++k) {
    const int r = (tid >> 4) + 16 * k;
    float v[8];
    {
      const u32x4v w = lds_ld128((uint32_t)r * 256u + (uint32_t)q * 16u);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[2 * c] = h2f((uint16_t)(w[c] & 0xffff));
        v[2 * c + 1] = h2f((uint16_t)(w[c] >> 16));
      }
    }
    fwht128_group16(v, q);
    const int m = m0 + r;
    const bool live = m < M;
    const int64_t prow = live ? row0 + m : row0;  // no address past the expert's rows
    store_pair_block(v, q, y + prow * (ldy / 2) + (int64_t)(n0 / 128) * 64, live);
  }
}

// GRP 0: one matrix. GRP 1 / 2 (grouped experts, GemmGroup g): blockIdx.x is
// a row tile of some expert (group_tile), blockIdx.y the column tile; the
// activation rows are gathered (g.a_rows) and the expert's codes and norms
// start at codes / norms + e * stride. GRP 1 writes fp32 rows of y at the
// expert's pair rows; GRP 2 (SwiGLU, NTW = 2) takes gate rows n and up rows
// I + n for the same 128 columns n of h, and writes silu(gate) * up through
// the FWHT-128 as pair-f16 rows (the next product's activations).
template <bool NIB, int TMW, int NTW, bool MASK, int OM, int GRP>
__global__ __launch_bounds__(256) void gemm4_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ norms,
    const float* __restrict__ ct, int n_levels, uint32_t code_mask, int tbl_entries,
    const uint32_t* __restrict__ xp, void* __restrict__ y, const uint16_t* __restrict__ bias,
    int M, int N, int nb, int64_t ldy, int tiles_m, int tiles_total, WLayout lay, int vec_ok,
    int ybf, GemmGroup g) {
  constexpr int NT = 256;
  constexpr int BM = TMW * 32;
  constexpr int BN = 128 * NTW;
  constexpr int KA = BM * 8 / NT;
  constexpr uint32_t ABUF = BM * kARow4;
  static_assert(KA * NT == BM * 8, "A tile must split evenly over the threads");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const uint32_t lane4 = (uint32_t)lane << 2;

  static_assert(GRP != 2 || NTW == 2, "SwiGLU tiles: one gate and one up n-tile per wave");
  static_assert(GRP == 0 || TMW > 2, "grouped tiles: 1, 2 or TMW live m-tiles");
  int m0, n0;
  int64_t row0 = 0;  // grouped: the expert's first pair row
  if constexpr (GRP == 0) {
    // XCD-aware tile order: ids are dealt round-robin to 8 XCDs; give each
    // XCD a contiguous range of logical tiles (M-tile fastest).
    int wid = blockIdx.x;
    if ((tiles_total & 7) == 0) wid = (wid & 7) * (tiles_total >> 3) + (wid >> 3);
    const int tm = wid % tiles_m, tn = wid / tiles_m;
    m0 = tm * BM;
    n0 = tn * BN;
  } else {
    int e, mt;
    if (!group_tile<BM>(g, blockIdx.x, lane, e, mt)) return;  // uniform
    row0 = g.offsets[e];
    M = g.offsets[e + 1] - (int)row0;  // this expert's rows
    m0 = mt * BM;
    n0 = blockIdx.y * (GRP == 2 ? 128 : BN);
    codes += (int64_t)e * g.codes_stride;
    norms += (int64_t)e * g.norms_stride;
  }

  // codebook values now, the table once the first A and B loads are issued
  // (the values' round trip overlaps theirs)
  float cbr[4];
  codebook_regs(cbr, ct, n_levels);
  const uint32_t abuf = (uint32_t)tbl_entries * 256u;

  // K range of this workgroup, in pairs of 128-blocks (the loop takes four
  // half-blocks per step): gridDim.z groups; with more than one, fp32 partial
  // sums go to slab blockIdx.z [M][ldy] of y
  const int kb0 = GRP ? 0 : 2 * (int)((int64_t)(nb / 2) * blockIdx.z / gridDim.z);
  const int nbz = GRP ? nb : 2 * (int)((int64_t)(nb / 2) * (blockIdx.z + 1) / gridDim.z) - kb0;
  if constexpr (GRP == 0) y = reinterpret_cast<char*>(y) + (int64_t)blockIdx.z * M * ldy * (OM == OM_F16 ? 2 : 4);

  // Loads through buffer resources based at this workgroup's first row of x
  // and first column of the weights: per-lane offsets in VGPRs, the K
  // position in the scalar offset (no 64-bit address arithmetic in the K
  // loop). Every extent is below 2 GiB (host check).
  const int64_t xrow_u32 = (int64_t)nb * 64;
  const int mlast = (m0 + BM <= M ? m0 + BM : M) - 1;
  // grouped: the whole activation matrix (rows gathered per lane)
  const __amdgpu_buffer_rsrc_t ra =
      GRP ? __builtin_amdgcn_make_buffer_rsrc((void*)xp, (short)0, (int)(g.a_total_rows * xrow_u32 * 4), 0x00020000)
          : __builtin_amdgcn_make_buffer_rsrc((void*)(xp + (int64_t)m0 * xrow_u32), (short)0,
                                              (int)((mlast - m0 + 1) * xrow_u32 * 4), 0x00020000);
  uint32_t a_voff[KA];
  uint32_t a_dst[KA];
#pragma unroll
  for (int i = 0; i < KA; ++i) {
    const int q = tid + NT * i;
    const int r = q >> 3, c = q & 7;
    int m = m0 + r;
    if (m >= M) m = M - 1;  // clamped rows feed discarded outputs only
    if constexpr (GRP) {
      const int64_t pr = row0 + m;  // pair row
      const int64_t src = g.a_rows ? (int64_t)g.a_rows[pr] : pr;
      a_voff[i] = (uint32_t)((src * xrow_u32 + c * 4) * 4);
    } else {
      a_voff[i] = (uint32_t)(((int64_t)(m - m0) * xrow_u32 + c * 4) * 4);
    }
    a_dst[i] = (uint32_t)(r * kARow4 + (((uint32_t)c ^ a4_swz(r)) << 4));
  }
  // grouped: resources over the expert's whole codes and norms
  const int nlast = (n0 + BN <= N ? n0 + BN : N) - 1;
  const int64_t cb0 = GRP ? 0 : lay.codes_off(n0), nb0 = GRP ? 0 : lay.norms_off(n0);
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(codes + cb0), (short)0,
      GRP ? (int)g.codes_stride
          : (int)(lay.codes_off(nlast) + (int64_t)(nb - 1) * lay.c_blk + (NIB ? 64 : 128) - cb0), 0x00020000);
  const __amdgpu_buffer_rsrc_t rn = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(norms + nb0), (short)0,
      GRP ? (int)(g.norms_stride * 2)
          : (int)((lay.norms_off(nlast) + (int64_t)(nb - 1) * lay.n_blk + 1 - nb0) * 2),
      0x00020000);
  uint32_t b_voff[NTW], n_voff[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    int n;
    if constexpr (GRP == 2) {
      // gate row (j = 0) or up row (j = 1) of column c of h
      int c = n0 + wave * 32 + l32;
      if (c >= g.I) c = g.I - 1;
      n = j == 0 ? c : g.I + c;
    } else {
      n = n0 + wave * 32 * NTW + j * 32 + l32;
      if (n >= N) n = N - 1;
    }
    b_voff[j] = (uint32_t)(lay.codes_off(n) - cb0) + 16 * h;
    n_voff[j] = (uint32_t)((lay.norms_off(n) - nb0) * 2);
  }
  uint32_t a_off[4];  // lane's row l32, chunk 4h + t, swizzled
#pragma unroll
  for (int t = 0; t < 4; ++t) a_off[t] = (uint32_t)(l32 * kARow4 + (((uint32_t)(4 * h + t) ^ a4_swz(l32)) << 4));

  const int nkt = 2 * nbz;  // half-blocks of this K range, a multiple of 4
  // loads past the last half-block re-read it (in bounds, never used)
  auto ldb = [&](BSlot4<NIB, NTW>& sl, int kt) {
    kt = kt < nkt ? kt : nkt - 1;
    const int bk = kb0 + (kt >> 1), half = kt & 1;
    const int sc = bk * (int)lay.c_blk + half * 32, sn = bk * (int)lay.n_blk * 2;
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      sl.lo[j] = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rc, b_voff[j], sc, 0));
      if constexpr (!NIB)
        sl.hi[j] = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(rc, b_voff[j], sc + 64, 0));
      sl.nrm[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rn, n_voff[j], sn, 0);
    }
  };
  auto lda = [&](u32x4v (&rg)[KA], int kt) {
    kt = kt < nkt ? kt : nkt - 1;
    const int sa = (kb0 * 64 + (kt >> 1) * 64 + (kt & 1) * 32) * 4;
#pragma unroll
    for (int i = 0; i < KA; ++i)
      rg[i] = __builtin_bit_cast(u32x4v, __builtin_amdgcn_raw_buffer_load_b128(ra, a_voff[i], sa, 0));
  };
  auto sta = [&](uint32_t buf, const u32x4v (&rg)[KA]) {
#pragma unroll
    for (int i = 0; i < KA; ++i) lds_st128(buf + a_dst[i], rg[i]);
  };

  float16v acc[TMW][NTW];
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  BSlot4<NIB, NTW> slot[4];
  u32x4v stg[2][KA], pre[2][KA];  // pre: prologue only
  lda(stg[0], 0);
  lda(stg[1], 1);
  lda(pre[0], 2);
  lda(pre[1], 3);
  ldb(slot[0], 0);
  ldb(slot[1], 1);
  ldb(slot[2], 2);
  if constexpr (NIB) fill_codebook_from<TBL_NIB_H2>(0, cbr, tbl_entries, NT / 64);
  else fill_codebook_from<TBL_F16>(0, cbr, tbl_entries, NT / 64);
  __syncthreads();  // codebook table written
  sta(abuf, stg[0]);
  sta(abuf + ABUF, stg[1]);
  sta(abuf + 2 * ABUF, pre[0]);
  sta(abuf + 3 * ABUF, pre[1]);
  lda(stg[0], 4);
  lda(stg[1], 5);
  __syncthreads();

  auto ring_next = [](uint32_t b) { return b == (kA4Ring - 1) * ABUF ? 0u : b + ABUF; };
  // the K loop, computing the first ACT m-tiles
  auto k_loop = [&](auto ACT_) {
    constexpr int ACT = decltype(ACT_)::value;
    Frag4<NIB, TMW, NTW> f;
    issue_frag4<NIB, TMW, NTW, MASK, ACT>(f, abuf + a_off[0], 0, slot[0], lane4, code_mask);
    uint32_t bcur = 0;  // ring offset (bytes) of half-block kt's A buffer

    auto half_step = [&](auto S_, int kt) {
      constexpr int S = decltype(S_)::value;
      const uint32_t bnext = ring_next(bcur);
      const uint32_t bst = ring_next(ring_next(ring_next(bnext)));  // where A(kt - 2) was
      ldb(slot[(S + 3) & 3], kt + 3);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        Frag4<NIB, TMW, NTW> fn;
        // this slab's operands (issued one slab ago) are in: wait for them
        // before the next slab's reads go out
        __builtin_amdgcn_s_waitcnt(0xc07f);
        if (t < 3)
          issue_frag4<NIB, TMW, NTW, MASK, ACT>(fn, abuf + bcur + a_off[t + 1], t + 1, slot[S], lane4, code_mask);
        else
          issue_frag4<NIB, TMW, NTW, MASK, ACT>(fn, abuf + bnext + a_off[0], 0, slot[(S + 1) & 3], lane4, code_mask);
        // keep the next slab's reads ahead of this slab's MFMAs
        __builtin_amdgcn_sched_barrier(0);
        mma_frag4<NIB, TMW, NTW, ACT>(acc, f, slot[S]);
        f = fn;
      }
      sta(abuf + bst, stg[S & 1]);  // A(kt + 4)
      lda(stg[S & 1], kt + 6);
      bcur = bnext;
      // one barrier per 128-block: between two of them the waves read A(kt),
      // A(kt + 1) and the first slab of A(kt + 2) while A(kt + 4), A(kt + 5)
      // go into the buffers of A(kt - 2), A(kt - 1), read before the last one
      if constexpr (S & 1) __syncthreads();
    };
    int kt = 0;
    for (; kt + 4 <= nkt; kt += 4) {
      half_step(std::integral_constant<int, 0>{}, kt);
      half_step(std::integral_constant<int, 1>{}, kt + 1);
      half_step(std::integral_constant<int, 2>{}, kt + 2);
      half_step(std::integral_constant<int, 3>{}, kt + 3);
    }
    if constexpr (GRP != 0) {
      if (kt < nkt) {  // an odd block count: its last block
        half_step(std::integral_constant<int, 0>{}, kt);
        half_step(std::integral_constant<int, 1>{}, kt + 1);
      }
    }
  };
  if constexpr (GRP != 0) {
    // an expert's last row tile often holds a few rows: compute only the
    // m-tiles that hold live rows (uniform: M and m0 are per workgroup)
    const int live = M - m0;
    if (live <= 32) k_loop(std::integral_constant<int, 1>{});
    else if (live <= 64) k_loop(std::integral_constant<int, 2>{});
    else k_loop(std::integral_constant<int, TMW>{});
  } else {
    k_loop(std::integral_constant<int, TMW>{});
  }

  if constexpr (GRP == 2) {
    swiglu_xtf_tile4<TMW>(acc, reinterpret_cast<uint32_t*>(y), ldy, M, g.I, row0, m0, n0);
  } else if constexpr (GRP == 1) {
    store_tile4<TMW, NTW, OM>(acc, reinterpret_cast<char*>(y) + row0 * ldy * (OM == OM_F16 ? 2 : 4), ldy,
                              bias, M, N, m0, n0, vec_ok, ybf != 0);
  } else {
    store_tile4<TMW, NTW, OM>(acc, y, ldy, bias, M, N, m0, n0, vec_ok, ybf != 0);
  }
}

template <bool NIB, int TMW, int NTW, bool MASK, int OM>
static int launch_gemm4_t(const GemmArgs& a, hipStream_t st, int ksplit = 1) {
  constexpr int BM = TMW * 32, BN = 128 * NTW;
  auto kern = gemm4_kernel<NIB, TMW, NTW, MASK, OM, 0>;
  const int entries = table_entries(NIB, a.n_levels);
  constexpr size_t ES = OM == OM_F16 ? 2 : 4;
  const size_t lds_loop = (size_t)entries * 256 + kA4Ring * (size_t)BM * kARow4;
  const size_t lds_out = (size_t)BM * (BN * ES + 16);
  const size_t lds = lds_loop > lds_out ? lds_loop : lds_out;
  if (lds > 160 * 1024) return PE_ERR_DIMS;
  static const bool attr_ok = [&] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  const int tiles_m = (a.M + BM - 1) / BM;
  const int tiles_n = (a.N + BN - 1) / BN;
  const int64_t total = (int64_t)tiles_m * tiles_n;
  if (total > INT32_MAX) return PE_ERR_DIMS;
  // one workgroup's rows of x and columns of codes and norms are addressed by
  // 32-bit buffer offsets
  const int64_t w_span = a.lay.codes_off(BN - 1) + (int64_t)a.nb * a.lay.c_blk + 128;
  if ((int64_t)BM * a.nb * 256 >= ((int64_t)1 << 31) || w_span >= ((int64_t)1 << 31)) return PE_ERR_DIMS;
  const uint8_t mb = NIB ? (uint8_t)((a.n_levels - 1) * 0x11) : (uint8_t)(a.n_levels - 1);
  // 16-byte stores need aligned rows; with a K split, aligned slab starts too
  const int vec_ok = ((uintptr_t)a.y % 16 == 0) && ((a.ldy * (int64_t)ES) % 16 == 0) &&
                     (ksplit == 1 || ((int64_t)a.M * a.ldy * (int64_t)ES) % 16 == 0);
  kern<<<dim3((unsigned)total, 1, (unsigned)ksplit), dim3(256), lds, st>>>(
      a.codes, a.norms, a.ct, a.n_levels, 0x01010101u * mb, entries,
      reinterpret_cast<const uint32_t*>(a.xp), a.y, a.bias, a.M, a.N, a.nb, a.ldy, tiles_m,
      (int)total, a.lay, vec_ok, a.ybf, GemmGroup{});
  return launch_status();
}

// Grouped expert products on the four-wave kernel, 128 x 256 tiles: GRP 1
// (SE_F32 / SE_F16) fp32 or 16-bit rows y[pair][N]; GRP 2 (SE_SWIGLU_XTF) the
// transformed silu(gate) * up as pair-f16 rows of I / 128 blocks.
template <bool NIB, bool MASK, int GRP, int OMX = OM_F32>
static int launch_moe_gemm4_t(const MoeGemmArgs& a, hipStream_t st) {
  constexpr int TMW = 4, NTW = 2, BM = TMW * 32, BN = 128 * NTW;
  constexpr int OM = GRP == 1 ? OMX : OM_F16;
  auto kern = gemm4_kernel<NIB, TMW, NTW, MASK, OM, GRP>;
  const int entries = table_entries(NIB, a.n_levels);
  const size_t lds_loop = (size_t)entries * 256 + kA4Ring * (size_t)BM * kARow4;
  const size_t lds_out = GRP == 1 ? (size_t)BM * (BN * 4 + 16) : (size_t)BM * 256;
  const size_t lds = lds_loop > lds_out ? lds_loop : lds_out;
  if (lds > 160 * 1024) return PE_ERR_DIMS;
  static const bool attr_ok = [&] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  // at least the sum over the groups of ceil(rows / BM); the surplus
  // workgroups find no tile and leave
  const int64_t tiles_m = a.g.groups + (a.P + BM - 1) / BM;
  const int64_t tiles_n = GRP == 2 ? a.g.I / 128 : (a.N + BN - 1) / BN;
  if (tiles_m > INT32_MAX || tiles_n > 65535 || tiles_n < 1) return PE_ERR_DIMS;
  const uint8_t mb = NIB ? (uint8_t)((a.n_levels - 1) * 0x11) : (uint8_t)(a.n_levels - 1);
  const int vec_ok = GRP == 1 && (uintptr_t)a.y % 16 == 0 && (a.ldy * (OM == OM_F16 ? 2 : 4)) % 16 == 0;
  kern<<<dim3((unsigned)tiles_m, (unsigned)tiles_n), dim3(256), lds, st>>>(
      a.codes, a.norms, a.ct, a.n_levels, 0x01010101u * mb, entries,
      reinterpret_cast<const uint32_t*>(a.xp), a.y, nullptr, 0, a.N, a.nb, a.ldy, 0, 0, a.lay, vec_ok,
      GRP == 1 && OM == OM_F16 ? a.ybf : 0, a.g);
  return launch_status();
}

bool moe_gemm4_fits(const MoeGemmArgs& a, int epilogue) {
  const int64_t lim = (int64_t)1 << 31;
  if (epilogue == SE_SWIGLU_XTF && (a.g.I <= 0 || a.g.I % 128 || a.ldy % 128)) return false;
  return a.nb >= 1 && a.g.groups >= 1 && a.g.codes_stride < lim && a.g.norms_stride * 2 < lim &&
         a.g.a_total_rows * a.nb * 256 < lim && a.P < lim;
}

int moe_gemm4(bool nibble, int epilogue, const MoeGemmArgs& a, hipStream_t st) {
  if (!a.g.offsets || !moe_gemm4_fits(a, epilogue)) return PE_ERR_DIMS;
  const bool mask = nibble ? a.n_levels != 16 : a.n_levels != 256;
  if (epilogue == SE_F32) {
    if (nibble) return mask ? launch_moe_gemm4_t<true, true, 1>(a, st) : launch_moe_gemm4_t<true, false, 1>(a, st);
    return mask ? launch_moe_gemm4_t<false, true, 1>(a, st) : launch_moe_gemm4_t<false, false, 1>(a, st);
  }
  if (epilogue == SE_F16) {
    if (nibble)
      return mask ? launch_moe_gemm4_t<true, true, 1, OM_F16>(a, st) : launch_moe_gemm4_t<true, false, 1, OM_F16>(a, st);
    return mask ? launch_moe_gemm4_t<false, true, 1, OM_F16>(a, st) : launch_moe_gemm4_t<false, false, 1, OM_F16>(a, st);
  }
  if (epilogue == SE_SWIGLU_XTF) {
    if (nibble) return mask ? launch_moe_gemm4_t<true, true, 2>(a, st) : launch_moe_gemm4_t<true, false, 2>(a, st);
    return mask ? launch_moe_gemm4_t<false, true, 2>(a, st) : launch_moe_gemm4_t<false, false, 2>(a, st);
  }
  return PE_ERR_DTYPE;
}

template <bool NIB, int TMW, int TNW, int WM, int WN, int OM>
static int launch_gemm_t(const GemmArgs& a, hipStream_t st, int ksplit = 1) {
  constexpr int BM = WM * TMW * 32, BN = WN * TNW * 32;
  auto kern = gemm_kernel<NIB, TMW, TNW, WM, WN, OM>;
  const int entries = table_entries(NIB, a.n_levels);
  const size_t lds = (size_t)entries * 256 + 2 * (size_t)BM * kAStride;
  if (lds > 160 * 1024) return PE_ERR_DIMS;
  static const bool attr_ok = [&] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
  }();
  (void)attr_ok;
  const int tiles_m = (a.M + BM - 1) / BM;
  const int tiles_n = (a.N + BN - 1) / BN;
  const int64_t total = (int64_t)tiles_m * tiles_n;
  if (total > INT32_MAX) return PE_ERR_DIMS;
  const uint8_t mb = NIB ? (uint8_t)((a.n_levels - 1) * 0x11) : (uint8_t)(a.n_levels - 1);
  kern<<<dim3((unsigned)total, 1, (unsigned)ksplit), dim3(WM * WN * 64), lds, st>>>(
      a.codes, a.norms, a.ct, a.n_levels, 0x01010101u * mb, entries,
      reinterpret_cast<const uint32_t*>(a.xp), a.y, a.bias, a.M, a.N, a.nb, a.ldy, tiles_m,
      (int)total, a.lay, a.ybf);
  return launch_status();
}

// Tile shape. Waves sit in one row (1 x WN), each owning 32 TMW rows x 32
// columns, so every weight column is dequantized by exactly one wave and two
// waves share a SIMD (8 waves). A workgroup's time grows with its tile area
// and tiles run in rounds of one workgroup per CU: the cost of a shape is
// rounds x area x a penalty for short tiles (the dequantization is amortised
// over BM rows; measured ~13% per halving of BM) or for 4-wave workgroups
// (one wave per SIMD hides no latency).
struct GemmShape {
  int tmw, wn;
};
static GemmShape pick_gemm_tile(int M, int N) {
  const int cus = num_cus();
  const GemmShape cand[] = {{8, 8}, {4, 8}, {2, 8}, {8, 4}, {4, 4}, {2, 4}};
  GemmShape best = cand[0];
  double best_cost = -1;
  for (const GemmShape& c : cand) {
    const int bm = 32 * c.tmw, bn = 32 * c.wn;
    if (c.tmw > 2 && M <= bm / 2) continue;  // no tile more than twice as tall as needed
    const int64_t tiles = (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int64_t rounds = (tiles + cus - 1) / cus;
    const double pen = (c.tmw == 8 ? 1.0 : c.tmw == 4 ? 1.13 : 1.3) * (c.wn == 8 ? 1.0 : 1.25);
    const double cost = (double)rounds * bm * bn * pen;
    if (best_cost < 0 || cost < best_cost * 0.999) {
      best_cost = cost;
      best = c;
    }
  }
  return best;
}

// n-tiles per wave of the four-wave kernel: the width whose tiles take the
// fewest rounds x columns per CU (M = 2048 on 12288 columns: 768 tiles of 256
// in three rounds or 512 of 384 in two, equal); ties go to the wider tile,
// which reads less through LDS and stores fewer A tiles and passes fewer
// barriers per MFMA. Only for nibble codes with 16-bit output: 384 fp32
// columns would not fit the output staging in LDS, and the int8 variant
// needs more registers than a wave has (it spilled).
static int gemm4_ntw(bool nibble, int M, int N, int om) {
  if (!nibble || om != OM_F16) return 2;
  const int cus = num_cus();
  int best = 2;
  int64_t best_cost = -1;
  for (int ntw = 2; ntw <= 3; ++ntw) {
    const int64_t tiles = (int64_t)((M + 127) / 128) * ((N + 128 * ntw - 1) / (128 * ntw));
    const int64_t cost = (tiles + cus - 1) / cus * ntw;
    if (best_cost < 0 || cost <= best_cost) {
      best = ntw;
      best_cost = cost;
    }
  }
  return best;
}

// 64-row four-wave tiles for 16-bit output when the 128-row ones are too few
// for one round and the 64-row ones fill at least three quarters of it (M =
// 256 on 12288 columns: 192 tiles): one launch without the K split's fp32
// partial sums and reduction (Q4 12288 x 4096 at M = 256: 52.3-52.7 against
// 56.6-57.0 us with the split), at the cost of half the MFMAs per codebook
// lookup.
static bool use_gemm4_short(int M, int N, int nb) {
  const int64_t tiles = (int64_t)((M + 63) / 64) * ((N + 255) / 256);
  return (nb & 1) == 0 && tiles * 4 >= 3 * (int64_t)num_cus() && tiles <= num_cus();
}

// 128 x 128 tiles for 16-bit output where they fill three quarters of a round
// or more but 128 x 256 ones do not fill one, ahead of 64 x 256 tiles: each
// dequantized B fragment feeds four m-tiles instead of two, for twice the A
// reads per MFMA (Q4 12288 x 4096 at M = 256: 41.1-41.7 against 42.0-42.6 us
// for 64 x 256 tiles, Q3 40.4-41.4 against 41.4-42.0; at M = 192, a third of
// their rows empty, 40.1 against 41.4 for 64 x 256 and 50.8 for the
// eight-wave kernel).
static bool use_gemm4_sq(int M, int N, int nb) {
  const int64_t t41 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
  const int64_t t42 = (int64_t)((M + 127) / 128) * ((N + 255) / 256);
  return (nb & 1) == 0 && t42 < num_cus() && t41 * 4 >= 3 * (int64_t)num_cus() && t41 <= num_cus();
}
static bool gemm4_square(int M) { return M % 128 == 0; }

// int8 codes (no 384-column tiles) where 128 x 256 tiles leave most of their
// last round empty: 64 x 128 tiles, whose rounds are each about 0.68 of a
// 128 x 256 round's work rate per tile area, when their total comes out
// lower (int8 6144 x 4096 at M = 1536, 288 tiles of 128 x 256: 142.3 against
// 156.5 us; at M = 2048 the 128 x 256 ones stay, 164.7 against 179.1).
static bool gemm4_int8_narrow(int M, int N) {
  const int64_t cus = num_cus();
  const int64_t t42 = (int64_t)((M + 127) / 128) * ((N + 255) / 256);
  const int64_t t21 = (int64_t)((M + 63) / 64) * ((N + 127) / 128);
  const int64_t r42 = (t42 + cus - 1) / cus, r21 = (t21 + cus - 1) / cus;
  return r21 * 8192 * 100 < r42 * 32768 * 68;
}

static bool use_gemm4(int M, int N, int nb) {
  const int64_t tiles4 = (int64_t)((M + 127) / 128) * ((N + 255) / 256);
  return (nb & 1) == 0 && tiles4 >= num_cus() && tiles4 <= 16 * (int64_t)num_cus();
}

// 64 x 384 four-wave tiles (nibble codes, 16-bit output) where 128 x 256
// tiles do not fill a round, 64 x 256 ones do not fit one, and the 64 x 384
// ones fill at least three quarters of one (M = 384..512 on 12288 columns):
// one launch in place of the eight-wave kernel (Q3 12288 x 4096 at M = 512:
// 65.8-66.1 against 70.6-71.1 us, Q4 65.7-66.0 against 71.2-71.6; M = 384
// 57.5-57.6 against 67.9). 128 x 256 tiles at 192 workgroups measured alike
// at M = 512 (65.5-67.4 us).
static bool use_gemm4_wide_short(int M, int N, int nb) {
  const int64_t t643 = (int64_t)((M + 63) / 64) * ((N + 383) / 384);
  return !use_gemm4(M, N, nb) && !use_gemm4_short(M, N, nb) && (nb & 1) == 0 &&
         t643 * 4 >= 3 * (int64_t)num_cus() && t643 <= num_cus();
}

// 128 x 256 four-wave tiles (128 x 384 where gemm4_ntw picks them) that fill
// half a round or more but less than one, where none of the narrower
// one-round forms above applies: in place of the eight-wave kernel (int8
// 6144 x 4096 at M = 1024, 192 tiles: 78.3 against 117.0 us; at M = 768, 144
// tiles: 77.7 against 115.3).
static bool use_gemm4_part(int M, int N, int nb) {
  const int64_t tiles4 = (int64_t)((M + 127) / 128) * ((N + 255) / 256);
  return (nb & 1) == 0 && tiles4 * 2 >= (int64_t)num_cus() && tiles4 < num_cus();
}

// 64 x 128 four-wave tiles, one launch, in place of the K split for a short K
// (at most 32 blocks) where they fill three quarters of a round or more (M =
// 512 on 4096 x 4096: 39.3-39.5 against 42.3-42.9 us with the split's fp32
// partial sums and reduction, int8 codes; on 4096 x 12288 the split stays
// faster, 77 against 81-82 us). Only above M = 64, where the small-M kernel
// takes the shapes that no K split applies to.
static bool use_gemm4_narrow(int M, int N, int nb) {
  const int64_t t21 = (int64_t)((M + 63) / 64) * ((N + 127) / 128);
  return M > 64 && nb <= 32 && (nb & 1) == 0 && !use_gemm4(M, N, nb) && !use_gemm4_short(M, N, nb) &&
         !use_gemm4_part(M, N, nb) && t21 * 4 >= 3 * (int64_t)num_cus() && t21 <= num_cus();
}

// K split of the four-wave kernel for M > 32 whose tiles are too few for one
// round (M = 33..512 on the 4096 x 12288 down projection: 16-64 tiles):
// groups of at least four 128-blocks (an even count each), about one
// workgroup per CU in all. 1 = no split.
// Tile rows of that split: 64 up to M = 256 (half the fp32 partial sums of
// 128-row tiles at the same grid size; measured against the eight-wave
// kernel's split at M = 128: 31.9 against 43.7 us on the 4096 x 12288 down
// projection, 33.3 against 45.5 on Q4 12288 x 4096; M = 256 on the down
// projection 47.1 against 48.5 with 128-row tiles), 128 above (M = 512: 79.1
// against 82.4 us with 64-row ones). At M = 256, 128 x 128 tiles instead of
// 64 x 256 ones (the same tile count; Q3 down projection 44.6-45.1 against
// 45.0-45.4 us); at M = 128 they measured slightly slower (31.3-31.7 against
// 31.1-31.5 us), above M = 256 slower (M = 512: 75.9 against 72.8 us).
// Up to M = 128, 64 x 128 tiles (twice the tiles, so a smaller split and
// fewer fp32 partial sums; Q4 12288 x 4096 at M = 64: 23.0 against 24.7 us,
// 4096 x 12288 21.7-21.8 against 24.1-24.2, int8 6144 x 4096 18.6 against
// 20.4; M = 128: 4096 x 12288 30.0 against 30.6, int8 4096 x 4096 22.1
// against 22.9; at M = 192 slower, 43.3 against 38.7).
static bool gemm4_split_square(int M) { return M > 128 && M <= 256 && gemm4_square(M); }
static int gemm4_split_rows(int M) { return M <= 256 && !gemm4_split_square(M) ? 64 : 128; }
static int gemm4_split_cols(int M) { return gemm4_split_square(M) || M <= 128 ? 128 : 256; }

static int gemm4_ksplit(int M, int N, int nb) {
  if (M <= 32 || (nb & 1) || use_gemm4(M, N, nb) || use_gemm4_sq(M, N, nb) || use_gemm4_short(M, N, nb) ||
      use_gemm4_part(M, N, nb) || use_gemm4_narrow(M, N, nb))
    return 1;
  const int rows = gemm4_split_rows(M), cols = gemm4_split_cols(M);
  const int64_t tiles4 = (int64_t)((M + rows - 1) / rows) * ((N + cols - 1) / cols);
  int z = (int)(num_cus() / tiles4);
  if (z > nb / 4) z = nb / 4;
  return z < 2 ? 1 : z;
}

// K split of the eight-wave kernel where the four-wave one takes none (an
// odd block count, or too many 64-row tiles for a split) and its tiles would
// leave more than half the CUs idle (few output tiles over a long K):
// gemm_ksplit groups of at least two 128-blocks, fp32 partial sums in the
// workspace, then the ordered reduction shared with the decode path. 1 = no
// split.
static int gemm_ksplit(int M, int N, int nb) {
  if (use_gemm4(M, N, nb) || use_gemm4_sq(M, N, nb) || use_gemm4_short(M, N, nb) || use_gemm4_part(M, N, nb) ||
      use_gemm4_narrow(M, N, nb) || gemm4_ksplit(M, N, nb) > 1)
    return 1;
  const GemmShape g = pick_gemm_tile(M, N);
  const int bm = 32 * g.tmw, bn = 32 * g.wn;
  const int64_t tiles = (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
  const int cus = num_cus();
  if (tiles * 2 > cus) return 1;
  int z = (int)(cus / tiles);
  if (z > nb / 2) z = nb / 2;
  return z < 2 ? 1 : z;
}

// The four-wave kernel (128 x 256 or 128 x 384 tiles) is the faster one when
// its tiles fill the CUs for one to sixteen rounds (measured on the C3
// prefill shapes: 6-18% ahead at M = 2048, 2.5-4% at M = 8192 on 12288
// columns); with fewer tiles the eight-wave kernel's narrower tiles spread
// wider.
template <bool NIB, int OM>
static int launch_gemm_eight(const GemmArgs& a, hipStream_t st, int ksplit) {
  const GemmShape g = pick_gemm_tile(a.M, a.N);
  switch (g.tmw * 16 + g.wn) {
    case 8 * 16 + 8: return launch_gemm_t<NIB, 8, 1, 1, 8, OM>(a, st, ksplit);
    case 4 * 16 + 8: return launch_gemm_t<NIB, 4, 1, 1, 8, OM>(a, st, ksplit);
    case 2 * 16 + 8: return launch_gemm_t<NIB, 2, 1, 1, 8, OM>(a, st, ksplit);
    case 8 * 16 + 4: return launch_gemm_t<NIB, 8, 1, 1, 4, OM>(a, st, ksplit);
    case 4 * 16 + 4: return launch_gemm_t<NIB, 4, 1, 1, 4, OM>(a, st, ksplit);
    default: return launch_gemm_t<NIB, 2, 1, 1, 4, OM>(a, st, ksplit);
  }
}

// the four-wave kernel with the code mask its codebook size needs
template <bool NIB, int TMW, int NTW, int OM>
static int launch_gemm4_m(const GemmArgs& a, hipStream_t st, int ksplit = 1) {
  const bool mask = NIB ? a.n_levels != 16 : a.n_levels != 256;
  return mask ? launch_gemm4_t<NIB, TMW, NTW, true, OM>(a, st, ksplit)
              : launch_gemm4_t<NIB, TMW, NTW, false, OM>(a, st, ksplit);
}

template <bool NIB, int OM>
static int launch_gemm_shape(const GemmArgs& a, hipStream_t st, void* ws, size_t ws_bytes) {
  // 128 x 256 or 128 x 384 tiles for one round or more (int8: 64 x 128 where
  // those rounds cost less)
  if (use_gemm4(a.M, a.N, a.nb)) {
    if constexpr (NIB && OM == OM_F16) {
      if (gemm4_ntw(NIB, a.M, a.N, OM) == 3) return launch_gemm4_m<NIB, 4, 3, OM>(a, st);
    }
    if constexpr (!NIB && OM == OM_F16) {
      if (gemm4_int8_narrow(a.M, a.N)) return launch_gemm4_m<NIB, 2, 1, OM>(a, st);
    }
    return launch_gemm4_m<NIB, 4, 2, OM>(a, st);
  }
  // fewer tiles than a round: the one-round forms, widest dequantization first
  if constexpr (NIB && OM == OM_F16) {
    if (use_gemm4_wide_short(a.M, a.N, a.nb)) return launch_gemm4_m<NIB, 2, 3, OM>(a, st);
  }
  if constexpr (OM == OM_F16) {
    if (use_gemm4_sq(a.M, a.N, a.nb)) return launch_gemm4_m<NIB, 4, 1, OM>(a, st);
    if (use_gemm4_short(a.M, a.N, a.nb)) return launch_gemm4_m<NIB, 2, 2, OM>(a, st);
  }
  if (use_gemm4_part(a.M, a.N, a.nb)) {
    if constexpr (NIB && OM == OM_F16) {
      if (gemm4_ntw(NIB, a.M, a.N, OM) == 3) return launch_gemm4_m<NIB, 4, 3, OM>(a, st);
    }
    return launch_gemm4_m<NIB, 4, 2, OM>(a, st);
  }
  if constexpr (OM == OM_F16) {
    if (use_gemm4_narrow(a.M, a.N, a.nb)) return launch_gemm4_m<NIB, 2, 1, OM>(a, st);
  }
  // fp16 out (the linear entry points): split K when the tiles are few and
  // the workspace holds the partial sums; otherwise one launch
  const int z4 = OM == OM_F16 ? gemm4_ksplit(a.M, a.N, a.nb) : 1;
  if (z4 > 1 && ws && aligned16(ws) && ws_bytes >= (size_t)z4 * a.M * a.N * 4) {
    GemmArgs p = a;
    p.y = ws;
    p.ldy = a.N;
    p.bias = nullptr;
    const bool rows64 = gemm4_split_rows(a.M) == 64, cols128 = gemm4_split_cols(a.M) == 128;
    const int rc = rows64 ? (cols128 ? launch_gemm4_m<NIB, 2, 1, OM_F32>(p, st, z4)
                                     : launch_gemm4_m<NIB, 2, 2, OM_F32>(p, st, z4))
                          : (cols128 ? launch_gemm4_m<NIB, 4, 1, OM_F32>(p, st, z4)
                                     : launch_gemm4_m<NIB, 4, 2, OM_F32>(p, st, z4));
    if (rc) return rc;
    return split_reduce(reinterpret_cast<const float*>(ws), z4, a.M, a.N, a.bias, a.y, a.ldy, st,
                        a.ybf != 0);
  }
  const int z = OM == OM_F16 ? gemm_ksplit(a.M, a.N, a.nb) : 1;
  if (z > 1 && ws && aligned16(ws) && ws_bytes >= (size_t)z * a.M * a.N * 4) {
    GemmArgs p = a;
    p.y = ws;
    p.ldy = a.N;
    p.bias = nullptr;
    if (int rc = launch_gemm_eight<NIB, OM_F32>(p, st, z)) return rc;
    return split_reduce(reinterpret_cast<const float*>(ws), z, a.M, a.N, a.bias, a.y, a.ldy, st,
                        a.ybf != 0);
  }
  return launch_gemm_eight<NIB, OM>(a, st, 1);
}

int gemm(bool nibble, int omode, const GemmArgs& a, hipStream_t st, void* ws, size_t ws_bytes) {
  if (nibble) return omode == 0 ? launch_gemm_shape<true, 0>(a, st, ws, ws_bytes) : launch_gemm_shape<true, 1>(a, st, ws, ws_bytes);
  return omode == 0 ? launch_gemm_shape<false, 0>(a, st, ws, ws_bytes) : launch_gemm_shape<false, 1>(a, st, ws, ws_bytes);
}

// Matmul on a pair-f16 x_tf, used by the linear entry points for M > 1: the
// fp32 partial sums of the K split, if it applies.
// M = 33..64 with fp16 out takes the GEMM when a K split applies (the
// four-wave kernel's with 64 x 128 tiles: 23.0 us at M = 64 on Q4 12288 x
// 4096, against 31.5 us for the eight-wave kernel's split and 57 us for the
// small-M kernel)
static bool mm_small(int64_t M, int N, int nb, int out_mode) {
  if (M <= 32) return true;
  if (M > kSmallMaxRows) return false;
  return out_mode != OM_F16 || (gemm4_ksplit((int)M, N, nb) <= 1 && gemm_ksplit((int)M, N, nb) <= 1);
}

size_t mm_xtf_workspace(bool nibble, int64_t M, int N, int nb) {
  (void)nibble;
  if (M > INT32_MAX || mm_small(M, N, nb, OM_F16)) return 0;
  const int z4 = gemm4_ksplit((int)M, N, nb);
  const int z = z4 > 1 ? z4 : gemm_ksplit((int)M, N, nb);
  return z > 1 ? (size_t)z * (size_t)M * (size_t)N * 4 : 0;
}

int mm_xtf(bool nibble, bool tiled, const void* codes, const uint16_t* norms, const float* ct,
           int n_levels, const void* x_pair, int64_t M, int N, int nb, void* y, int out_mode,
           int64_t ldy, const uint16_t* bias, void* ws, size_t ws_bytes, hipStream_t st,
           bool ybf) {
  if (M > INT32_MAX) return PE_ERR_DIMS;
  const WLayout lay = wlayout(nibble, tiled, nb);
  if (mm_small(M, N, nb, out_mode)) {
    SmallArgs s{reinterpret_cast<const uint8_t*>(codes), norms, ct, n_levels,
                reinterpret_cast<const uint32_t*>(x_pair), nullptr, nullptr, 0, 0, y, ldy, bias,
                (int)M, N, nb, lay, ybf ? 1 : 0};
    return gemm_small(nibble, out_mode == OM_F32 ? SE_F32 : SE_F16, s, st);
  }
  GemmArgs a{reinterpret_cast<const uint8_t*>(codes), norms, ct, n_levels, x_pair, y, bias,
             (int)M, N, nb, ldy, lay, ybf ? 1 : 0};
  return gemm(nibble, out_mode, a, st, ws, ws_bytes);
}

}  // namespace pe
