/*
 * Measurement helpers of libpolarengine_amd.so (no counterpart in the
 * reference): the plain HBM streaming read and copy that bench.py times beside
 * the quantized linear, as the measured bandwidth ceiling of the part.
 * Same conventions as polarengine_amd.h: device pointers, byte sizes, a
 * hipStream_t, int status; nothing is allocated and nothing synchronises.
 */
#ifndef POLARENGINE_AMD_BENCH_H
#define POLARENGINE_AMD_BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of the sink buffer pe_stream_read needs for `bytes` of input. */
size_t pe_stream_read_sink_bytes(int64_t bytes);

/*
 * Read `bytes` (a multiple of 16, 16-byte aligned) of device memory with
 * 128-bit non-temporal loads, 8 KB per 256-lane workgroup. A lane writes its
 * folded word to `sink` only if it equals `magic` (pass a value the data does
 * not produce): the loads stay, the writes are (almost) none.
 */
int pe_stream_read(const void* src, int64_t bytes, void* sink, uint32_t magic, void* stream);

/* dst[0:bytes] = src[0:bytes] (a multiple of 16; both 16-byte aligned). */
int pe_copy(void* dst, const void* src, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif
