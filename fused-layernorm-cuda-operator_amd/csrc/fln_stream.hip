// fln_stream.hip -- streaming reference kernels for gfx950: the HBM ceiling that the
// normalization kernels are measured against (libfln_stream.so, include/fln_stream.h).
//
// Each kernel moves the byte pattern of one normalization call with nothing else in the way:
//   pattern 0  1 read  + 1 write  (the forward: x -> y)
//   pattern 1  2 reads + 1 write  (the backward: x, dy -> dx)
//   pattern 2  2 reads + 2 writes (residual add + norm: x, r -> h, y)
//   pattern 3  1 read  + 1 half-width write (norm -> fp8: bf16 x -> one byte per element)
// with the idioms of the normalization kernels: raw buffer loads / stores through buffer
// resources (out-of-range offsets read zeros and drop stores), a persistent grid that deals
// tiles grid-stride so every block walks one window of adjacent memory, a static ring of PD
// tiles of loads in flight, the current tile's stores issued after the next tile's loads (loads
// and stores share the vmcnt counter on gfx9-family GPUs), and selectable cache policies.  A tile
// is U 16-byte vectors per thread.  The arithmetic is a bitwise combine of the inputs, so the
// outputs depend on every input byte and the kernels are bound by memory traffic alone.
//
// The reference measures its bandwidth as bytes moved per call against the device's peak
// (tests/publication_validation.py:367-418); these kernels give the same figure for plain
// streams on this device, which is what an HBM-bound kernel can reach at best.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fln_stream.h"
#include "fln_device.h"

namespace fln {
namespace {

struct StreamArgs {
  const void* in[2];
  void* out[2];
  uint32_t nvec;  // 16-byte vectors per input stream
};

template <int PAT> struct StreamShape {
  static constexpr int NR = (PAT == 1 || PAT == 2) ? 2 : 1;  // input streams
  static constexpr int NW = PAT == 2 ? 2 : 1;                // output streams
  static constexpr bool HALF = PAT == 3;                     // 8-byte output vectors
};

template <int PAT, int U, int PD, int LPOL, int SPOL>
__global__ __launch_bounds__(1024) void stream_kernel(const StreamArgs a) {
  using S = StreamShape<PAT>;
  const uint32_t B = blockDim.x;
  const uint32_t tile_vecs = B * U;
  const uint32_t ntiles = (a.nvec + tile_vecs - 1) / tile_vecs;
  const uint32_t in_bytes = a.nvec * 16u;
  const uint32_t out_bytes = a.nvec * (S::HALF ? 8u : 16u);
  const rsrc_t r0 = make_rsrc(a.in[0], in_bytes);
  const rsrc_t r1 = make_rsrc(S::NR > 1 ? a.in[1] : nullptr, in_bytes);
  const rsrc_t w0 = make_rsrc(a.out[0], out_bytes);
  const rsrc_t w1 = make_rsrc(S::NW > 1 ? a.out[1] : nullptr, out_bytes);
  const uint32_t G = gridDim.x;
  const uint32_t my_tiles = ntiles > blockIdx.x ? (ntiles - 1 - blockIdx.x) / G + 1 : 0u;

  // Vector index of slot u of `tile` for this thread, or an index no resource reaches.
  auto vec_of = [&](uint32_t tile, int u) -> uint32_t {
    return tile < ntiles ? tile * tile_vecs + static_cast<uint32_t>(u) * B + threadIdx.x
                         : (kOutOfRange >> 4);
  };
  u32x4 v0[PD][U], v1[PD][U];
  auto load = [&](uint32_t tile, int slot) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t off = vec_of(tile, u) * 16u;
      v0[slot][u] = __builtin_amdgcn_raw_buffer_load_b128(r0, off, 0, LPOL);
      if constexpr (S::NR > 1)
        v1[slot][u] = __builtin_amdgcn_raw_buffer_load_b128(r1, off, 0, LPOL);
    }
  };

  // The loop runs whole rounds of PD tiles; tiles past the end read zeros and store nothing.
  // (An early exit from the unrolled round would make the compiler wait for every load in
  // flight at the top of the loop instead of the one slot it consumes.)
  const uint32_t rounds = (my_tiles + PD - 1) / PD;
  // Prologue: the first PD tiles, in slot order, each followed by as many stores as a loop step
  // issues (zeros to an offset past every resource: dropped by the range check).  The loop top
  // is then reached with the same sequence of outstanding operations from the prologue as from
  // the previous step, so the compiler's wait there covers only the slot it consumes.
#pragma unroll
  for (int k = 0; k < PD; ++k) {
    load(blockIdx.x + static_cast<uint32_t>(k) * G, k);
#pragma unroll
    for (int u = 0; u < U * S::NW; ++u)  // distinct, non-adjacent: none merged away
      __builtin_amdgcn_raw_buffer_store_b32(0u, w0, kOutOfRange + 64u * u, 0, SPOL);
    asm volatile("" ::: "memory");  // keeps the slots in issue order
  }
  for (uint32_t r = 0; r < rounds; ++r) {
#pragma unroll
    for (int s = 0; s < PD; ++s) {
      const uint32_t tile = blockIdx.x + (r * PD + s) * G;
      u32x4 o0[U], o1[U];
      u32x2 h[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (PAT == 0) o0[u] = v0[s][u];
        if constexpr (PAT == 1) o0[u] = v0[s][u] ^ v1[s][u];
        if constexpr (PAT == 2) {
          o0[u] = v0[s][u] ^ v1[s][u];
          o1[u] = v0[s][u] + v1[s][u];
        }
        if constexpr (PAT == 3) {
          h[u].x = v0[s][u].x ^ v0[s][u].y;
          h[u].y = v0[s][u].z ^ v0[s][u].w;
        }
      }
      load(tile + PD * G, s);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t vi = vec_of(tile, u);
        if constexpr (S::HALF) {
          __builtin_amdgcn_raw_buffer_store_b64(h[u], w0, vi * 8u, 0, SPOL);
        } else {
          __builtin_amdgcn_raw_buffer_store_b128(o0[u], w0, vi * 16u, 0, SPOL);
          if constexpr (S::NW > 1)
            __builtin_amdgcn_raw_buffer_store_b128(o1[u], w1, vi * 16u, 0, SPOL);
        }
      }
      // Keep the scheduler from hoisting the next slot's (cheap) combine above this slot's
      // loads and stores: that would make the wait at its top cover every slot in flight.
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

template <int PAT, int U, int PD, int LP, int SP>
int run_k(const StreamArgs& a, int threads, int blocks, hipStream_t s, int* occupancy) {
  auto k = stream_kernel<PAT, U, PD, LP, SP>;
  if (occupancy) {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, k, threads, 0) != hipSuccess) return -1;
    *occupancy = v;
    return 0;
  }
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(blocks)), dim3(static_cast<unsigned>(threads)),
                     0, s, a);
  return static_cast<int>(hipGetLastError());
}

template <int PAT, int U, int PD>
int by_policy(const StreamArgs& a, int threads, int blocks, int lp, int sp, hipStream_t s,
              int* occ) {
  if (lp == 0 && sp == 0) return run_k<PAT, U, PD, 0, 0>(a, threads, blocks, s, occ);
  if (lp == 0 && sp == 2) return run_k<PAT, U, PD, 0, 2>(a, threads, blocks, s, occ);
  if (lp == 2 && sp == 0) return run_k<PAT, U, PD, 2, 0>(a, threads, blocks, s, occ);
  if (lp == 2 && sp == 2) return run_k<PAT, U, PD, 2, 2>(a, threads, blocks, s, occ);
  return FLN_STREAM_ERR_INVALID;
}

template <int PAT, int U>
int by_depth(const StreamArgs& a, int threads, int blocks, int pd, int lp, int sp, hipStream_t s,
             int* occ) {
  switch (pd) {
    case 1: return by_policy<PAT, U, 1>(a, threads, blocks, lp, sp, s, occ);
    case 2: return by_policy<PAT, U, 2>(a, threads, blocks, lp, sp, s, occ);
    case 3: return by_policy<PAT, U, 3>(a, threads, blocks, lp, sp, s, occ);
    case 4: return by_policy<PAT, U, 4>(a, threads, blocks, lp, sp, s, occ);
    default: return FLN_STREAM_ERR_INVALID;
  }
}

template <int PAT>
int by_unroll(const StreamArgs& a, int threads, int blocks, int u, int pd, int lp, int sp,
              hipStream_t s, int* occ) {
  switch (u) {
    case 1: return by_depth<PAT, 1>(a, threads, blocks, pd, lp, sp, s, occ);
    case 2: return by_depth<PAT, 2>(a, threads, blocks, pd, lp, sp, s, occ);
    case 4: return by_depth<PAT, 4>(a, threads, blocks, pd, lp, sp, s, occ);
    default: return FLN_STREAM_ERR_INVALID;
  }
}

int dispatch(int pattern, const StreamArgs& a, int threads, int blocks, int u, int pd, int lp,
             int sp, hipStream_t s, int* occ) {
  if (threads != 256 && threads != 512 && threads != 1024) return FLN_STREAM_ERR_INVALID;
  switch (pattern) {
    case FLN_STREAM_1R1W: return by_unroll<0>(a, threads, blocks, u, pd, lp, sp, s, occ);
    case FLN_STREAM_2R1W: return by_unroll<1>(a, threads, blocks, u, pd, lp, sp, s, occ);
    case FLN_STREAM_2R2W: return by_unroll<2>(a, threads, blocks, u, pd, lp, sp, s, occ);
    case FLN_STREAM_1R_HALF_W: return by_unroll<3>(a, threads, blocks, u, pd, lp, sp, s, occ);
    default: return FLN_STREAM_ERR_INVALID;
  }
}

}  // namespace
}  // namespace fln

extern "C" int fln_stream_run(int pattern, const void* in0, const void* in1, void* out0,
                              void* out1, int64_t in_bytes, int threads, int blocks, int unroll,
                              int depth, int load_policy, int store_policy, void* stream) {
  // Byte offsets are 32-bit and kOutOfRange (2^31) must lie past every stream.
  if (in_bytes <= 0 || in_bytes % 16 != 0 || in_bytes >= (int64_t(1) << 31) || blocks < 1)
    return FLN_STREAM_ERR_INVALID;
  const bool two_in = pattern == FLN_STREAM_2R1W || pattern == FLN_STREAM_2R2W;
  if (!in0 || !out0 || (two_in && !in1) || (pattern == FLN_STREAM_2R2W && !out1))
    return FLN_STREAM_ERR_INVALID;
  fln::StreamArgs a{};
  a.in[0] = in0;
  a.in[1] = in1;
  a.out[0] = out0;
  a.out[1] = out1;
  a.nvec = static_cast<uint32_t>(in_bytes / 16);
  return fln::dispatch(pattern, a, threads, blocks, unroll, depth, load_policy, store_policy,
                       static_cast<hipStream_t>(stream), nullptr);
}

extern "C" int fln_stream_blocks_per_cu(int pattern, int threads, int unroll, int depth,
                                        int load_policy, int store_policy) {
  fln::StreamArgs a{};
  int occ = 0;
  const int rc = fln::dispatch(pattern, a, threads, 1, unroll, depth, load_policy, store_policy,
                               nullptr, &occ);
  return rc == 0 ? occ : -1;
}

extern "C" int fln_stream_cu_count(void) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  return cus;
}
