/*
 * fln_stream.h -- C ABI of libfln_stream.so: streaming reference kernels for gfx950.
 *
 * Not part of the drop-in: these kernels have no counterpart in the reference's operator API.
 * They move the byte pattern of one normalization call (reads and writes of 16-byte vectors,
 * nothing computed) with the normalization kernels' own access idioms, so that bench.py can
 * state the HBM ceiling those kernels are judged against.  The reference reports bandwidth the
 * same way, as bytes moved per call against the device peak
 * (tests/publication_validation.py:367-418).
 *
 * Streams are device pointers of `in_bytes` bytes each (a multiple of 16, below 2 GiB); the
 * half-width output of FLN_STREAM_1R_HALF_W has in_bytes / 2 bytes.  Calls are asynchronous on
 * `stream` (a hipStream_t, NULL = the null stream) and return 0 or FLN_STREAM_ERR_INVALID / a
 * hipError_t value.
 */
#ifndef FLN_STREAM_H
#define FLN_STREAM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLN_STREAM_ERR_INVALID 1

/* Access patterns: out0 = in0 (1R1W); out0 = in0 ^ in1 (2R1W); out0 = in0 ^ in1 and
 * out1 = in0 + in1 per 32-bit word (2R2W); out0 = the XOR of each 16-byte vector's two 8-byte
 * halves (1R + half-width W). */
#define FLN_STREAM_1R1W 0
#define FLN_STREAM_2R1W 1
#define FLN_STREAM_2R2W 2
#define FLN_STREAM_1R_HALF_W 3

/* One streaming pass.  threads: 256, 512 or 1024 per block; blocks: the persistent grid (tiles
 * are dealt grid-stride); unroll: 16-byte vectors per thread per tile (1, 2, 4); depth: tiles of
 * loads in flight ahead of the current one (1-4); load_policy / store_policy: 0 default, 2
 * non-temporal (the CPol bits of the buffer instructions). */
int fln_stream_run(int pattern, const void* in0, const void* in1, void* out0, void* out1,
                   int64_t in_bytes, int threads, int blocks, int unroll, int depth,
                   int load_policy, int store_policy, void* stream);

/* Resident blocks per CU of that instantiation (hipOccupancyMaxActiveBlocksPerMultiprocessor),
 * or -1 for an invalid combination. */
int fln_stream_blocks_per_cu(int pattern, int threads, int unroll, int depth, int load_policy,
                             int store_policy);

/* Compute units of the current device, or -1. */
int fln_stream_cu_count(void);

#ifdef __cplusplus
}
#endif

#endif /* FLN_STREAM_H */
