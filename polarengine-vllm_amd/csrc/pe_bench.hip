// Measurement helpers: the plain HBM streaming read and copy that the
// benchmark times next to the quantized linear, as the measured bandwidth
// ceiling of the part (no counterpart in the reference).
//
// Read: each workgroup of 256 lanes reads one contiguous 8 KB run, two 16-byte
// non-temporal loads per lane (the decode GEMV's weight stream has the same
// shape: 1-2 KB per wave, 128-bit loads). The loaded words are folded into one
// value per lane that is stored only when it equals a value passed in at run
// time, so the loads cannot be removed and (almost) nothing is written.
// Copy: each lane moves four 16-byte words, all four loads in flight before
// the stores.

#include "pe_internal.h"
#include "../../include/polarengine_amd_bench.h"

namespace pe {

constexpr int kReadLaneBytes = 32;
constexpr int kReadWgBytes = 256 * kReadLaneBytes;
constexpr int kCopyLaneBytes = 64;

__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* src, int64_t bytes,
                                                          uint32_t* sink, uint32_t magic) {
  const int64_t off = (int64_t)blockIdx.x * kReadWgBytes + (int64_t)threadIdx.x * 16;
  u32x4v a = {0, 0, 0, 0}, b = {0, 0, 0, 0};
  if (off + 16 <= bytes) a = ld_nt16v(src + off);
  if (off + 256 * 16 + 16 <= bytes) b = ld_nt16v(src + off + 256 * 16);
  const uint32_t v = a[0] ^ a[1] ^ a[2] ^ a[3] ^ b[0] ^ b[1] ^ b[2] ^ b[3];
  if (v == magic) sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = v;
}

__global__ __launch_bounds__(256) void copy_kernel(const uint8_t* src, uint8_t* dst,
                                                   int64_t bytes) {
  const int64_t base = (int64_t)blockIdx.x * 256 * kCopyLaneBytes + (int64_t)threadIdx.x * 16;
  u32x4v v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t o = base + (int64_t)i * 256 * 16;
    v[i] = o + 16 <= bytes ? ld_nt16v(src + o) : u32x4v{0, 0, 0, 0};
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t o = base + (int64_t)i * 256 * 16;
    if (o + 16 <= bytes) __builtin_nontemporal_store(v[i], reinterpret_cast<u32x4v*>(dst + o));
  }
}

}  // namespace pe

using namespace pe;

extern "C" size_t pe_stream_read_sink_bytes(int64_t bytes) {
  if (bytes <= 0) return 0;
  return (size_t)((bytes + kReadWgBytes - 1) / kReadWgBytes) * 256 * 4;
}

extern "C" int pe_stream_read(const void* src, int64_t bytes, void* sink, uint32_t magic,
                              void* stream) {
  if (!src || !sink) return PE_ERR_NULL;
  if (bytes <= 0 || bytes % 16) return PE_ERR_DIMS;
  if (!aligned16(src) || !aligned16(sink)) return PE_ERR_ALIGN;
  const int64_t grid = (bytes + kReadWgBytes - 1) / kReadWgBytes;
  if (grid > INT32_MAX) return PE_ERR_DIMS;
  stream_read_kernel<<<dim3((unsigned)grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint8_t*>(src), bytes, reinterpret_cast<uint32_t*>(sink), magic);
  return launch_status();
}

extern "C" int pe_copy(void* dst, const void* src, int64_t bytes, void* stream) {
  if (!src || !dst) return PE_ERR_NULL;
  if (bytes <= 0 || bytes % 16) return PE_ERR_DIMS;
  if (!aligned16(src) || !aligned16(dst)) return PE_ERR_ALIGN;
  const int64_t grid = (bytes + 256 * kCopyLaneBytes - 1) / (256 * kCopyLaneBytes);
  if (grid > INT32_MAX) return PE_ERR_DIMS;
  copy_kernel<<<dim3((unsigned)grid), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint8_t*>(src), reinterpret_cast<uint8_t*>(dst), bytes);
  return launch_status();
}
