// fln_forward_impl.h -- forward kernel templates and the per-dtype dispatch.  Included by the
// per-dtype translation units (fln_forward_f32.hip, ...) so the instantiations compile in parallel.
#pragma once
#include <stdio.h>
#include <stdlib.h>

#include "fln_device.h"
#include "fln_internal.h"

namespace fln {

// Cross-lane reduction over a row group of `wpr` waves.  The wave step is register-only; with
// several waves per row each wave publishes its partial in LDS slot[wave] and every wave sums
// its group's partials in the same fixed order (deterministic, identical in every lane).
template <class Op>
__device__ __forceinline__ float row_allreduce(float v, float* slot, int wpr, int rg, int wave,
                                               int lane) {
  v = wave_allreduce<Op>(v);
  if (wpr == 1) return v;
  if (lane == 0) slot[wave] = v;
  __syncthreads();
  float r = slot[rg * wpr];
  for (int k = 1; k < wpr; ++k) r = Op::apply(r, slot[rg * wpr + k]);
  return r;
}

template <int VEC>
__device__ __forceinline__ void store_fp8(uint8_t* q, int v, const float (&a)[VEC], float inv) {
  if constexpr (VEC == 8) {
    uint2 w;
    w.x = fp8x4(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
    w.y = fp8x4(a[4] * inv, a[5] * inv, a[6] * inv, a[7] * inv);
    *reinterpret_cast<uint2*>(q + (int64_t)v * 8) = w;
  } else if constexpr (VEC == 4) {
    *reinterpret_cast<uint32_t*>(q + (int64_t)v * 4) =
        fp8x4(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
  } else {
    static_assert(VEC == 1, "fp8 store supports 1, 4 or 8 elements");
    q[v] = fp8x1(a[0] * inv);
  }
}

// ---------------------------------------------------------------------------------------------
// Register-resident forward.  Block = rows_per_block row groups of `wpr` waves; thread t of a
// row group owns vectors t, t + 64*wpr, ... (VPL of them) -- consecutive lanes read consecutive
// 16-byte vectors, so each wave-wide load is one fully coalesced 1 KiB transaction.
// ---------------------------------------------------------------------------------------------
template <class T, bool FP8, bool RES, int VEC, int VPL, int MAXT>
__global__ __launch_bounds__(MAXT) void fwd_reg_kernel(const FwdParams p, int64_t row_blocks) {
  __shared__ float red[3][MAXT / kWave];
  using P = Pack<T, VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int wpr = p.wpr;
  const int rg = wave / wpr;
  const int t = (wave - rg * wpr) * kWave + lane;
  const int tpr = kWave * wpr;
  const int rows_per_block = blockDim.x / tpr;
  const int64_t N = p.cols;
  const int nvec = static_cast<int>(N / VEC);
  const float inv_n = 1.0f / static_cast<float>(N);

  for (int64_t rb = blockIdx.x; rb < row_blocks; rb += gridDim.x) {
    const int64_t row = rb * rows_per_block + rg;
    const bool row_ok = row < p.rows;
    float xf[VPL][VEC];
    {
      const P* xr = reinterpret_cast<const P*>(static_cast<const T*>(p.x) + row * N);
      P xv[VPL];
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int v = t + i * tpr;
        xv[i] = (row_ok && v < nvec) ? xr[v] : zero_pack<T, VEC>();
      }
      if constexpr (RES) {
        const P* rr = reinterpret_cast<const P*>(static_cast<const T*>(p.res) + row * N);
        P* hr = p.h ? reinterpret_cast<P*>(static_cast<T*>(p.h) + row * N) : nullptr;
        P rv[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          const int v = t + i * tpr;
          rv[i] = (row_ok && v < nvec) ? rr[v] : zero_pack<T, VEC>();
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          P hv;
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            hv.v[e] = from_f32<T>(to_f32(xv[i].v[e]) + to_f32(rv[i].v[e]));
            xf[i][e] = to_f32(hv.v[e]);
          }
          const int v = t + i * tpr;
          if (hr && row_ok && v < nvec) hr[v] = hv;
        }
      } else {
#pragma unroll
        for (int i = 0; i < VPL; ++i)
#pragma unroll
          for (int e = 0; e < VEC; ++e) xf[i][e] = to_f32(xv[i].v[e]);
      }
    }

    // Statistics: two passes over registers (mean, then centred sum of squares).
    float mean = 0.0f;
    if (!p.rms) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) s += xf[i][e];
      mean = row_allreduce<SumOp>(s, red[0], wpr, rg, wave, lane) * inv_n;
    }
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const bool ok = (t + i * tpr) < nvec;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float d = xf[i][e] - mean;
        q += ok ? d * d : 0.0f;
      }
    }
    q = row_allreduce<SumOp>(q, red[1], wpr, rg, wave, lane);
    const float rstd = 1.0f / sqrtf(q * inv_n + p.eps);
    if (row_ok && t == 0) {
      if (p.mean) p.mean[row] = mean;
      if (p.rstd) p.rstd[row] = rstd;
    }

    // Normalize + affine + epilogue, in place.
    const P* gr = static_cast<const P*>(p.gamma);
    const P* br = static_cast<const P*>(p.beta);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int v = t + i * tpr;
      const bool ok = v < nvec;
      P gv, bv;
      if (gr) gv = ok ? gr[v] : zero_pack<T, VEC>();
      if (br) bv = ok ? br[v] : zero_pack<T, VEC>();
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float a = (xf[i][e] - mean) * rstd;
        if (gr) a *= to_f32(gv.v[e]);
        if (br) a += to_f32(bv.v[e]);
        xf[i][e] = apply_gelu(a, p.gelu);
      }
    }

    if constexpr (!FP8) {
      P* yr = reinterpret_cast<P*>(static_cast<T*>(p.y) + row * N);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int v = t + i * tpr;
        if (row_ok && v < nvec) {
          P o;
#pragma unroll
          for (int e = 0; e < VEC; ++e) o.v[e] = from_f32<T>(xf[i][e]);
          yr[v] = o;
        }
      }
    } else {
      float am = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const bool ok = (t + i * tpr) < nvec;
#pragma unroll
        for (int e = 0; e < VEC; ++e) am = fmaxf(am, ok ? fabsf(xf[i][e]) : 0.0f);
      }
      am = row_allreduce<MaxOp>(am, red[2], wpr, rg, wave, lane);
      const float inv = am > 0.0f ? 448.0f / am : 0.0f;
      if (row_ok && t == 0) p.scale[row] = am / 448.0f;
      uint8_t* qr = static_cast<uint8_t*>(p.y) + row * N;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int v = t + i * tpr;
        if (row_ok && v < nvec) store_fp8<VEC>(qr, v, xf[i], inv);
      }
    }
    if (wpr > 1) __syncthreads();  // LDS slots are reused by the next row block
  }
}

// ---------------------------------------------------------------------------------------------
// Looped fallback: one block per row, any length, any alignment; A is the accumulation type
// (fp32, or fp64 for fp64 I/O).  Same two-pass statistics as the register path.
// ---------------------------------------------------------------------------------------------
template <class A, bool MAX>
__device__ __forceinline__ A block_allreduce(A v, A* slot) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const A o = __shfl_xor(v, m, kWave);
    v = MAX ? (o > v ? o : v) : v + o;
  }
  if (lane == 0) slot[wave] = v;
  __syncthreads();
  A r = slot[0];
  for (int k = 1; k < nw; ++k) r = MAX ? (slot[k] > r ? slot[k] : r) : r + slot[k];
  return r;
}

template <class T, class A, bool FP8>
__global__ __launch_bounds__(1024) void fwd_loop_kernel(const FwdParams p) {
  __shared__ A red[3][16];
  const int64_t N = p.cols;
  const T* x = static_cast<const T*>(p.x);
  const T* r = static_cast<const T*>(p.res);
  T* h = static_cast<T*>(p.h);
  const T* g = static_cast<const T*>(p.gamma);
  const T* b = static_cast<const T*>(p.beta);
  for (int64_t row = blockIdx.x; row < p.rows; row += gridDim.x) {
    const int64_t base = row * N;
    auto in = [&](int64_t j) -> A {
      if (r) return static_cast<A>(static_cast<T>(static_cast<A>(x[base + j]) +
                                                  static_cast<A>(r[base + j])));
      return static_cast<A>(x[base + j]);
    };
    A mean = 0;
    if (!p.rms) {
      A s = 0;
      for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
        const A v = in(j);
        if (h) h[base + j] = static_cast<T>(v);
        s += v;
      }
      mean = block_allreduce<A, false>(s, red[0]) / static_cast<A>(N);
    } else if (h) {
      for (int64_t j = threadIdx.x; j < N; j += blockDim.x) h[base + j] = static_cast<T>(in(j));
    }
    A q = 0;
    for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
      const A d = in(j) - mean;
      q += d * d;
    }
    q = block_allreduce<A, false>(q, red[1]);
    const A rstd = static_cast<A>(1) / sqrt(q / static_cast<A>(N) + static_cast<A>(p.eps));
    if (threadIdx.x == 0) {
      if (p.mean) p.mean[row] = static_cast<float>(mean);
      if (p.rstd) p.rstd[row] = static_cast<float>(rstd);
    }
    auto outv = [&](int64_t j) -> A {
      A a = (in(j) - mean) * rstd;
      if (g) a *= static_cast<A>(g[j]);
      if (b) a += static_cast<A>(b[j]);
      return apply_gelu(a, p.gelu);
    };
    if constexpr (!FP8) {
      T* y = static_cast<T*>(p.y);
      for (int64_t j = threadIdx.x; j < N; j += blockDim.x) y[base + j] = static_cast<T>(outv(j));
    } else {
      A am = 0;
      for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
        const A a = outv(j);
        const A m = a < 0 ? -a : a;
        am = m > am ? m : am;
      }
      am = block_allreduce<A, true>(am, red[2]);
      const float amf = static_cast<float>(am);
      const float inv = amf > 0.0f ? 448.0f / amf : 0.0f;
      if (threadIdx.x == 0) p.scale[row] = amf / 448.0f;
      uint8_t* q8 = static_cast<uint8_t*>(p.y);
      for (int64_t j = threadIdx.x; j < N; j += blockDim.x)
        q8[base + j] = fp8x1(static_cast<float>(outv(j)) * inv);
    }
    __syncthreads();  // slots are reused by the next row
  }
}

// ---------------------------------------------------------------------------------------------
// Host side: geometry selection and dispatch.
// ---------------------------------------------------------------------------------------------
namespace detail {

constexpr int64_t kMaxGrid = int64_t(1) << 20;

inline int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

inline int env_int(const char* name, int dflt) {
  const char* s = getenv(name);
  return (s && *s) ? atoi(s) : dflt;
}

template <class T, bool FP8, bool RES, int VEC, int VPL>
int launch_reg(const FwdParams& p, int threads, hipStream_t s) {
  const int rows_per_block = threads / (kWave * p.wpr);
  const int64_t row_blocks = (p.rows + rows_per_block - 1) / rows_per_block;
  const int64_t grid = row_blocks < kMaxGrid ? row_blocks : kMaxGrid;
  if (threads <= 256)
    hipLaunchKernelGGL((fwd_reg_kernel<T, FP8, RES, VEC, VPL, 256>), dim3(grid), dim3(threads), 0,
                       s, p, row_blocks);
  else
    hipLaunchKernelGGL((fwd_reg_kernel<T, FP8, RES, VEC, VPL, 1024>), dim3(grid), dim3(threads),
                       0, s, p, row_blocks);
  return static_cast<int>(hipGetLastError());
}

// Largest vectors-per-lane instantiated: 32 elements per lane for 16-byte vectors (keeps a
// LayerNorm row slice, its fp32 copy and the affine parameters within ~120 VGPRs), 16 for the
// scalar path.
template <int VEC> constexpr int max_vpl() { return VEC == 1 ? 16 : 32 / VEC; }

template <class T, bool FP8, bool RES, int VEC>
int launch_reg_vpl(const FwdParams& p, int vpl, int threads, hipStream_t s) {
  constexpr int CAP = max_vpl<VEC>();
  switch (vpl) {
    case 1: return launch_reg<T, FP8, RES, VEC, 1>(p, threads, s);
    case 2: return launch_reg<T, FP8, RES, VEC, 2>(p, threads, s);
    case 4: return launch_reg<T, FP8, RES, VEC, 4>(p, threads, s);
    case 8:
      if constexpr (CAP >= 8) return launch_reg<T, FP8, RES, VEC, 8>(p, threads, s);
      return FLN_ERR_INVALID;
    case 16:
      if constexpr (CAP >= 16) return launch_reg<T, FP8, RES, VEC, 16>(p, threads, s);
      return FLN_ERR_INVALID;
    default: return FLN_ERR_INVALID;
  }
}

template <class T, class A, bool FP8>
int launch_loop(const FwdParams& p, hipStream_t s) {
  const int threads = p.cols >= 4096 ? 1024 : 256;
  const int64_t grid = p.rows < kMaxGrid ? p.rows : kMaxGrid;
  hipLaunchKernelGGL((fwd_loop_kernel<T, A, FP8>), dim3(grid), dim3(threads), 0, s, p);
  return static_cast<int>(hipGetLastError());
}

template <class T, bool FP8>
int dispatch_typed(FwdParams p, hipStream_t s) {
  constexpr int VV = 16 / sizeof(T);  // elements per 16-byte vector
  const int64_t N = p.cols;
  bool vec_ok = (N % VV == 0) && aligned16(p.x) && aligned16(p.gamma) && aligned16(p.beta) &&
                aligned16(p.res) && aligned16(p.h);
  if (FP8)
    vec_ok = vec_ok && (reinterpret_cast<uintptr_t>(p.y) % VV == 0);
  else
    vec_ok = vec_ok && aligned16(p.y);
  if (env_int("FLN_FORCE_LOOP", 0)) return launch_loop<T, float, FP8>(p, s);
  const int vec = vec_ok ? VV : 1;
  const int cap = vec_ok ? max_vpl<VV>() : max_vpl<1>();
  const int64_t nvec = N / vec;
  constexpr int max_wpr = 16;
  auto per_lane = [&](int w) { return (nvec + kWave * w - 1) / (kWave * w); };
  int wpr = 1;
  while (per_lane(wpr) > cap && wpr < max_wpr) wpr *= 2;
  if (per_lane(wpr) > cap) return launch_loop<T, float, FP8>(p, s);
  // Few rows: spread each row over more waves so the grid covers more CUs (latency-bound
  // shapes such as 32 x 768 finish in one memory round trip either way, but with fewer serial
  // loads per lane).
  const int64_t target_waves = 4 * static_cast<int64_t>(device_cu_count());
  while (p.rows * wpr < target_waves && wpr < max_wpr && nvec > kWave * wpr * 2) wpr *= 2;
  const int forced = env_int("FLN_FWD_WPR", 0);
  if (forced >= 1 && forced <= max_wpr && (forced & (forced - 1)) == 0 && per_lane(forced) <= cap)
    wpr = forced;
  p.wpr = wpr;
  const int vpl = next_pow2(static_cast<int>(per_lane(wpr)));
  const int threads = wpr <= 4 ? 256 : kWave * wpr;
  const bool res = p.res != nullptr;
  if (vec_ok) {
    return res ? launch_reg_vpl<T, FP8, true, VV>(p, vpl, threads, s)
               : launch_reg_vpl<T, FP8, false, VV>(p, vpl, threads, s);
  }
  return res ? launch_reg_vpl<T, FP8, true, 1>(p, vpl, threads, s)
             : launch_reg_vpl<T, FP8, false, 1>(p, vpl, threads, s);
}

}  // namespace detail

}  // namespace fln
