// Internal (C++) interfaces shared by the translation units of the library.
#pragma once

#include "pe_common.h"

namespace pe {

// Weight layout of one quantized matrix (nb 128-blocks per row, bpb code
// bytes per block: 64 nibble-packed, 128 int8). Byte offset of (row n, block b)
// in the codes: (n >> 4) * c_tile + (n & 15) * c_row + b * c_blk; norms alike,
// in elements.
//   row-major (the reference layout): c_tile = 16 row_bytes, c_row = row_bytes,
//     c_blk = bpb;
//   tiled-16 (PE_LAYOUT_TILE16): the 16 rows x bpb bytes of one (16-row tile,
//     block) are contiguous, c_tile = 16 nb bpb, c_row = bpb, c_blk = 16 bpb;
//     rows are padded to a multiple of 16.
struct WLayout {
  int64_t c_tile, c_row, c_blk;
  int64_t n_tile, n_row, n_blk;
  __host__ __device__ int64_t codes_off(int n) const {
    return (int64_t)(n >> 4) * c_tile + (int64_t)(n & 15) * c_row;
  }
  __host__ __device__ int64_t norms_off(int n) const {
    return (int64_t)(n >> 4) * n_tile + (int64_t)(n & 15) * n_row;
  }
};
inline WLayout wlayout(bool nibble, bool tiled, int nb) {
  const int64_t bpb = nibble ? 64 : 128;
  if (tiled) return WLayout{16 * nb * bpb, bpb, 16 * bpb, 16 * (int64_t)nb, 1, 16};
  return WLayout{16 * nb * bpb, nb * bpb, bpb, 16 * (int64_t)nb, nb, 1};
}

// activation source of the M = 1 GEMV
enum { XM_RAW_F16 = 0, XM_XTF_F32 = 1, XM_PAIR_F16 = 2 };
// output element type of GEMV/GEMM epilogues
enum { OM_F32 = 0, OM_F16 = 1 };

struct Gemv1Args {
  const uint8_t* codes;
  const uint16_t* norms;
  const float* ct;
  int n_levels;
  const void* x;
  void* y;
  const uint16_t* bias;
  int N;
  int nb;
  int xbf = 0;  // XM_RAW_F16 input is bfloat16
  int ybf = 0;  // OM_F16 output (and bias) is bfloat16
};

struct GemmArgs {
  const uint8_t* codes;
  const uint16_t* norms;
  const float* ct;
  int n_levels;
  const void* xp;  // pair-f16 x_tf [M][nb][64]
  void* y;
  const uint16_t* bias;
  int M, N, nb;
  int64_t ldy;
  WLayout lay;
  int ybf = 0;  // 16-bit output (and bias) is bfloat16
};

// Grouped form of the four-wave prefill kernel (expert products): row tiles
// of every group in group order, activation rows gathered per pair row.
struct GemmGroup {
  const int32_t* offsets;  // [groups + 1]: first pair row of each group
  const int32_t* a_rows;   // activation row of each pair row (null: the pair row)
  int64_t codes_stride;    // bytes of one group's codes
  int64_t norms_stride;    // fp16 norms of one group
  int64_t a_total_rows;    // rows of the activation matrix
  int groups;
  int I;  // SwiGLU: columns of h (gate rows 0..I-1, up rows I..2I-1)
};
struct MoeGemmArgs {
  const uint8_t* codes;
  const uint16_t* norms;
  const float* ct;
  int n_levels;
  WLayout lay;
  int nb;          // 128-blocks of K (any count)
  const void* xp;  // pair-f16 activations [a_total_rows][nb][64]
  void* y;         // SE_F32 / SE_F16: [pairs][ldy]; SE_SWIGLU_XTF: pair-f16 rows of ldy halves
  int64_t ldy;
  int N;      // SE_F32 / SE_F16: output columns; SE_SWIGLU_XTF: weight rows (2 I)
  int64_t P;  // pair rows over all groups
  GemmGroup g;
  int ybf = 0;  // SE_F16: the 16-bit rows are bfloat16
};
bool moe_gemm4_fits(const MoeGemmArgs& a, int epilogue);
int moe_gemm4(bool nibble, int epilogue, const MoeGemmArgs& a, hipStream_t st);

// pe_gemv.hip
int gemv1(bool nibble, int xmode, int omode, const Gemv1Args& a, hipStream_t st);
int gemv1_max_kp(bool nibble);

// small-M epilogues
// SE_SWIGLU_XTF (grouped experts only): the SwiGLU output of a 128-column
// block goes straight through the FWHT-128 into pair-f16 rows (the next
// product's activation operand) instead of fp16 h
enum { SE_F32 = 0, SE_F16 = 1, SE_SWIGLU = 2, SE_SWIGLU_XTF = 3 };

struct SmallArgs {
  const uint8_t* codes;
  const uint16_t* norms;
  const float* ct;
  int n_levels;
  const uint32_t* xp;        // pair-f16 activations, rows of nb*64 uint32
  const int32_t* a_rows;     // nullable (MoE): A row m reads xp row a_rows[m]
  const int32_t* group_off;  // MoE: expert e owns rows [off[e], off[e+1]), gridDim.y experts
  int64_t codes_stride;      // bytes between experts' codes (MoE)
  int64_t norms_stride;      // uint16 between experts' norms (MoE)
  void* y;
  int64_t ldy;
  const uint16_t* bias;
  int M;                     // rows (small-M matmul); MoE: all pairs over the experts
  int N;                     // output columns (SwiGLU: I; the weights hold 2I rows)
  int nb;
  WLayout lay;               // per-expert layout (row-major for the MoE path)
  int ybf = 0;               // SE_F16 output (and bias) is bfloat16
};

// pe_gemm_small.hip: M <= kSmallMaxRows per pass is cheapest (larger M loops)
constexpr int kSmallMaxRows = 64;
// small-M matmul: M rows of xp, epilogue SE_F32 or SE_F16 (+ bias); the
// MoE fields of SmallArgs are ignored
int gemm_small(bool nibble, int epilogue, const SmallArgs& a, hipStream_t st);
// grouped expert products (group_off required; epilogue SE_F32, SE_SWIGLU or
// SE_SWIGLU_XTF)
int moe_grouped(bool nibble, int epilogue, const SmallArgs& a, int groups, hipStream_t st);

// pe_gemv_mfma.hip: decode GEMV, 1 <= M <= kDecMaxRows (M > 16 through the K
// split with two m-tiles; at M = 33..64 the prefill GEMM's K split measured
// faster: 25 against 44 us at M = 64), fp16 out (+ fp16 bias)
constexpr int kDecMaxRows = 32;
struct DecArgs {
  const uint8_t* codes;
  const uint16_t* norms;
  const float* ct;
  int n_levels;
  const void* x;   // raw fp16 rows (xraw) or pair-f16 x_tf rows
  int64_t ldx;     // row stride of x in fp16 elements
  void* y;
  int64_t ldy;     // row stride of y in fp16 elements
  const uint16_t* bias;
  int M, N, nb;
  WLayout lay;
  const float* ct_host;  // nullable host copy of ct (n_levels floats): codebook by value
  void* ws;              // fp32 partial sums of the K-split path (gemv_mfma_workspace bytes)
  size_t ws_bytes;
  int xbf = 0;           // raw x is bfloat16 (else fp16)
  int ybf = 0;           // y and bias are bfloat16 (else fp16)
  uint32_t* cnt = nullptr;  // K split: completion counters (zero; left zero)
};
bool gemv_mfma_fits(bool nibble, int M, int N, int nb, int n_levels);
// y[m, n] = fp16(sum over g = 0.. G-1 in order of part[g][m][n]) (+ fp16 bias)
int split_reduce(const float* part, int G, int M, int N, const uint16_t* bias, void* y, int64_t ldy,
                 hipStream_t st, bool ybf = false);
// bytes of fp32 partial sums of the K-split path (0 when it does not split);
// the counters come on top (kWsCounterBytes, see above)
size_t gemv_mfma_workspace(bool nibble, int M, int N, int nb, int n_levels);
int gemv_mfma(bool nibble, bool xraw, const DecArgs& a, hipStream_t st);

// pe_gemm.hip (ws: fp32 partial sums of the K split for fp16 output; may be null)
int gemm(bool nibble, int omode, const GemmArgs& a, hipStream_t st, void* ws = nullptr,
         size_t ws_bytes = 0);
size_t mm_xtf_workspace(bool nibble, int64_t M, int N, int nb);
int mm_xtf(bool nibble, bool tiled, const void* codes, const uint16_t* norms, const float* ct,
           int n_levels, const void* x_pair, int64_t M, int N, int nb, void* y, int out_mode,
           int64_t ldy, const uint16_t* bias, void* ws, size_t ws_bytes, hipStream_t st,
           bool ybf = false);

// pe_fwht.hip
int fwht128(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ldx, void* y,
            int y_layout, hipStream_t st);
int repack_pair(const float* x, int64_t rows, int64_t cols, void* y, hipStream_t st);

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Every workspace of this library starts with a block of completion counters
// (one 32-bit word per group of workgroups that meet in a K split: the last
// one to finish adds the partial sums). The block must be zero before the
// workspace's first use; every call leaves it zero again, and no entry point
// writes anything else into it, so one buffer can serve every entry point.
constexpr size_t kWsCounterBytes = 4096;
constexpr int kWsCounters = (int)(kWsCounterBytes / 4);

}  // namespace pe
