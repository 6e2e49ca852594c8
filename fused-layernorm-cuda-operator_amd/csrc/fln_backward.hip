// fln_backward.hip -- LayerNorm / RMSNorm backward for gfx950 and its C-ABI entry points.
//
// The reference declares `layernorm_backward_cuda` (csrc/layernorm.h:24-32) and calls it from
// `layernorm_backward` (csrc/layernorm_cuda.cpp:97-141), but never defines it: this file is the
// first implementation of that contract.
//
// Stage 1 (bwd_reg_kernel): row groups of `wpr` waves each take rows grid-stride, with the next
// PD rows of x / dy always in flight (a ring of raw buffer loads; at loaded HBM latency the CU
// needs tens of KiB of reads outstanding).  Per row it computes
//     LayerNorm: xhat = (x - mean) rstd, g = dy gamma,
//                dx = rstd (g - sum(g)/N - xhat sum(g xhat)/N)
//     RMSNorm:   xhat = x rstd,          dx = rstd (g - xhat sum(g xhat)/N)
// and accumulates the column sums dy*xhat (dgamma) and dy (dbeta) for the columns each lane
// owns in fp32 registers.  At the end the block's row groups are combined through LDS in a
// fixed order and written as one fp32 partial row per block.
// Stage 2 (col_reduce_kernel): sums the partial rows per column in a fixed order, spread over
// many small blocks (32 columns each).  Nothing uses atomics, so dgamma/dbeta are bitwise
// reproducible run to run.  (Fusing stage 2 into stage 1 behind a cooperative grid barrier was
// measured at 2x the time of the two launches on gfx950 and is not used.)
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "fln_device.h"
#include "fln_internal.h"

namespace fln {

struct ColReduceArgs {
  const float* part[2];  // [G, ld] partial arrays (dgamma first, then dbeta)
  void* out[2];
  int64_t G;             // partial rows
  int64_t N;             // columns
  int ny;                // arrays to reduce (0, 1 or 2)
  int out_dtype;         // FLN_F32 / FLN_BF16 / FLN_F16
};

// Stage 2.  The partial arrays are [G, ld] fp32 (ld = cols rounded up to 4).  The work is cut
// into "quad blocks": 8 column quads (32 columns) of one array each.  A quad block is reduced by
// 8 * S threads: thread (slice, q) sums partial rows slice, slice + S, ... of quad q with eight
// loads in flight, then the S slices are folded through LDS in fixed steps of 4 (S -> S/4 -> ...
// -> at most 8) and one thread per quad adds the last few.  The order depends only on G and S,
// so the result is bitwise reproducible.
#ifndef FLN_CR_QUADS
#define FLN_CR_QUADS 8
#endif
#ifndef FLN_CR_SLICES
#define FLN_CR_SLICES 32
#endif
constexpr int kCrQuads = FLN_CR_QUADS;

__device__ __forceinline__ void add4(float4& a, const float4& b) {
  a.x += b.x;
  a.y += b.y;
  a.z += b.z;
  a.w += b.w;
}

__device__ __forceinline__ void store_param(void* out, int dtype, int64_t i, float v) {
  if (dtype == FLN_F32)
    static_cast<float*>(out)[i] = v;
  else if (dtype == FLN_BF16)
    static_cast<__bf16*>(out)[i] = from_f32<__bf16>(v);
  else
    static_cast<_Float16*>(out)[i] = from_f32<_Float16>(v);
}

__host__ __device__ inline int64_t quad_blocks(const ColReduceArgs& a) {
  const int64_t ld = (a.N + 3) & ~int64_t(3);
  return a.ny * (((ld >> 2) + kCrQuads - 1) / kCrQuads);
}

// Reduce quad block `qb` with the first 8 * S threads of the block (S a power of two >= 4);
// comb holds 8 * S float4.  Every thread of the block must call this (it contains barriers).
__device__ __forceinline__ void reduce_quad_block(const ColReduceArgs& a, int64_t qb, int S,
                                                  float4* comb) {
  const int tid = threadIdx.x;
  const int q = tid % kCrQuads, slice = tid / kCrQuads;
  const int64_t ld = (a.N + 3) & ~int64_t(3);
  const int64_t nqb = ((ld >> 2) + kCrQuads - 1) / kCrQuads;
  const int y = static_cast<int>(qb / nqb);
  const int64_t c = ((qb - y * nqb) * kCrQuads + q) * 4;
  const bool active = slice < S;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (active && c < ld) {
    const float* col = a.part[y] + c;
    int64_t k = slice;
    for (; k + 7 * S < a.G; k += 8 * S) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const float4*>(col + (k + u * S) * ld);
#pragma unroll
      for (int u = 0; u < 8; ++u) add4(acc, v[u]);
    }
    for (; k < a.G; k += S) add4(acc, *reinterpret_cast<const float4*>(col + k * ld));
  }
  if (active) comb[slice * kCrQuads + q] = acc;
  __syncthreads();
  int n = S;
  while (n > 8) {
    n >>= 2;
    if (slice < n) {
      float4 r = comb[slice * kCrQuads + q];
#pragma unroll
      for (int j = 1; j < 4; ++j) add4(r, comb[(slice + j * n) * kCrQuads + q]);
      comb[slice * kCrQuads + q] = r;  // slice < n reads only slices >= n (none written here)
    }
    __syncthreads();
  }
  if (slice == 0 && c < a.N) {
    float4 r = comb[q];
    for (int j = 1; j < n; ++j) add4(r, comb[j * kCrQuads + q]);
    const float rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c + e < a.N) store_param(a.out[y], a.out_dtype, c + e, rr[e]);
  }
  __syncthreads();  // comb is reused by the caller's next quad block
}

// Rows in flight ahead of the current one.  Measured on MI355X over bf16 / fp16 / fp32 rows of
// 768 to 16384 columns: 2 rows beat 1 and 3 when a lane holds one vector of a row; with two
// vectors per lane (16-bit rows wider than 8192 columns, fp32 wider than 4096) a deeper ring no
// longer fits the 128 VGPRs of a 1024-thread block and spills, so one row is prefetched.
#ifndef FLN_BWD_PREFETCH
#define FLN_BWD_PREFETCH(VPL) ((VPL) == 1 ? 2 : 1)
#endif
// Cache policies of the streamed rows: x / dy / dres loads and dx stores are non-temporal (each
// byte is touched once).  Measured on MI355X with exact ring waits, bf16 backward calls: 8192 x
// 4096 LayerNorm 43.6 -> 41.1 us, 16384 x 8192 RMSNorm 146.3 -> 132.4 us against default-policy
// loads.  gamma, the statistics and the column partials keep the default policy.
#ifndef FLN_BWD_LOAD_POL
#define FLN_BWD_LOAD_POL kStream
#endif
#ifndef FLN_BWD_STORE_POL
#define FLN_BWD_STORE_POL kStream
#endif
// GELU (1 erf, 2 tanh): the backward of GELU(LayerNorm(x) * gamma + beta).  The GELU input
// a = xhat gamma + beta is recomputed from the saved statistics, and dy is replaced by
// dy GELU'(a) before the LayerNorm algebra (so dgamma / dbeta are sums of dy GELU'(a) xhat and
// of dy GELU'(a)).
template <class T, bool DRES, int GELU, int VEC, int VPL, int MAXT>
__global__ __launch_bounds__(MAXT) void bwd_reg_kernel(const BwdParams p) {
  constexpr int MAXW = MAXT / kWave;
  // RAW: 16-bit rows of 18433..24576 columns, 3 vectors per lane in a 1024-thread block.  The
  // row stays in the I/O type and is widened at each use (with GELU, GELU' is looked up at each
  // use too): fp32 copies of x-hat and dy (48 VGPRs) would not fit the 128 a lane has there
  // beside the column sums and the next row in flight.
  constexpr bool RAW = (VPL == 3 || VPL == 4) && MAXT == 1024 && VEC == 8 && sizeof(T) == 2;
  // NOPF: 4 vectors per lane (rows of 24577..32768 columns) leave no room for the next row:
  // each row is loaded at the top of its own step (one block per CU; the row's stores are still
  // in flight while the next row loads).
  constexpr bool NOPF = RAW && VPL == 4;
  static_assert(!NOPF || (GELU == 0 && !DRES), "4-vector raw tiles: LayerNorm / RMSNorm only");
  constexpr int PD = NOPF ? 1 : FLN_BWD_PREFETCH(VPL);  // rows in flight ahead of the current one

  // [double buffer][sum g, sum g*xhat][wave], padded for combine_partials
  __shared__ float red[2][2][MAXW + 16];
  __shared__ float comb[MAXT * VEC];         // row-group combine, one vector slot at a time
  __shared__ float4 gelu_tab[GELU != 0 ? kGeluTabN : 1];  // GELU epilogue: the GELU' table
  using P = Pack<T, VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wpr = p.wpr;
  const int rg = wave / wpr;
  const int t = (wave - rg * wpr) * kWave + lane;
  const int tpr = kWave * wpr;
  const int rgs = p.rgs;
  const int64_t N = p.cols;
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  const float inv_n = 1.0f / static_cast<float>(N);
  // Rows are dealt out grid-stride: iteration `it` of block b handles row group
  // (it * gridDim.x + b), i.e. rows (it * gridDim.x + b) * rgs + rg.  At any moment all blocks
  // work on one window of adjacent rows, which keeps HBM page locality like a streaming copy;
  // each block still accumulates its column partials in a fixed order (deterministic).
  const int64_t group_stride = static_cast<int64_t>(gridDim.x);
  const int iters = static_cast<int>(
      ((p.rows + rgs - 1) / rgs + group_stride - 1 - blockIdx.x) / group_stride);
  const T* X = static_cast<const T*>(p.x);
  const T* DY = static_cast<const T*>(p.dy);
  const T* DR = static_cast<const T*>(p.dres);
  T* DX = static_cast<T*>(p.dx);

  // gamma (and, with GELU, beta) stay in registers in the I/O type and are widened at each use
  // (gamma ones when absent; zeros past the row): half the VGPRs of fp32 copies for 16-bit types.
  // The 16-bit GELU and residual-gradient flavours with two vectors per lane in 1024-thread
  // blocks (three in 768-thread blocks) park them in LDS instead, each thread its own copy
  // (64-72 KiB, no barrier): in registers
  // they made those flavours spill 84-132 B per lane (4096 x 16384 bf16: GELU tanh 132.4 ->
  // 102.6 us, erf 153.2 -> 96.5 us; with a residual gradient 97.8 us on the LDS-staged kernel
  // -> 90.8 us here).
  constexpr bool PARAMS_IN_LDS =
      ((GELU != 0 || DRES) && ((VPL == 2 && MAXT == 1024) || (VPL == 3 && MAXT == 768)) &&
       sizeof(T) == 2) || RAW;
  __shared__ P gsh[PARAMS_IN_LDS ? VPL * MAXT : 1], bsh[PARAMS_IN_LDS ? VPL * MAXT : 1];
  P gmr[PARAMS_IN_LDS ? 1 : VPL];
  P btr[GELU && !PARAMS_IN_LDS ? VPL : 1];
  {
    const rsrc_t gr = make_rsrc(p.gamma, row_bytes);
    const bool has_g = p.gamma != nullptr;
    const T one = from_f32<T>(1.0f);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      P gv = buf_load<P>(gr, t + i * tpr);
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if (!has_g) gv.v[e] = one;
      if constexpr (PARAMS_IN_LDS)
        gsh[i * MAXT + threadIdx.x] = gv;
      else
        gmr[i] = gv;
    }
    if constexpr (GELU != 0) {
      const rsrc_t br = make_rsrc(p.beta, row_bytes);  // absent beta reads as zeros
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        if constexpr (PARAMS_IN_LDS)
          bsh[i * MAXT + threadIdx.x] = buf_load<P>(br, t + i * tpr);
        else
          btr[i] = buf_load<P>(br, t + i * tpr);
      }
    }
  }
  auto gam = [&](int i, int e) {
    if constexpr (PARAMS_IN_LDS)
      return to_f32(gsh[i * MAXT + threadIdx.x].v[e]);
    else
      return to_f32(gmr[i].v[e]);
  };
  auto bet = [&](int i, int e) {
    if constexpr (PARAMS_IN_LDS)
      return to_f32(bsh[i * MAXT + threadIdx.x].v[e]);
    else
      return to_f32(btr[GELU ? i : 0].v[e]);
  };
  float acc_g[VPL][VEC], acc_b[VPL][VEC];
#pragma unroll
  for (int i = 0; i < VPL; ++i)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc_g[i][e] = acc_b[i][e] = 0.0f;

  auto row_of = [&](int it) {
    return (static_cast<int64_t>(it) * group_stride + blockIdx.x) * rgs + rg;
  };
  auto bytes_of = [&](int it) -> uint32_t {
    return (it < iters && row_of(it) < p.rows) ? row_bytes : 0u;
  };

  // Ring of raw loads (x, dy, dres, mean, rstd) for the PD rows after the current one; rows
  // past the block's range have zero-byte resources and read as zeros.
  P xn[PD][VPL], dn[PD][VPL], rn[PD][VPL];
  float mun[PD], rsn[PD];
  auto load_row = [&](int it, int slot) {
    const int64_t row = row_of(it);
    const uint32_t nb = bytes_of(it);
    const rsrc_t xr = make_rsrc(X + row * N, nb);
    const rsrc_t dr = make_rsrc(DY + row * N, nb);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      xn[slot][i] = buf_load<P, FLN_BWD_LOAD_POL>(xr, t + i * tpr);
      dn[slot][i] = buf_load<P, FLN_BWD_LOAD_POL>(dr, t + i * tpr);
    }
    if constexpr (DRES) {
      const rsrc_t rr = make_rsrc(DR + row * N, nb);
#pragma unroll
      for (int i = 0; i < VPL; ++i) rn[slot][i] = buf_load<P, FLN_BWD_LOAD_POL>(rr, t + i * tpr);
    }
    const uint32_t sb = nb ? 4u : 0u;
    mun[slot] = __builtin_bit_cast(
        float, BufIO<4>::load(make_rsrc(p.rms ? nullptr : p.mean + row, sb), 0));
    rsn[slot] = __builtin_bit_cast(float, BufIO<4>::load(make_rsrc(p.rstd + row, sb), 0));
  };

  // The row being processed, widened once: xhat and dy in fp32 (g = dy * gamma is formed in the
  // row sums and kept for dx only by lanes with 8 columns: see KEEP_G).  With a GELU
  // epilogue, dd holds twice the gradient at the LayerNorm output; kInvD takes the factor out once
  // per row (rstd and the row-sum coefficients) and once per block (the column partials), exactly.
  constexpr float kInvD = GELU != 0 ? 0.5f : 1.0f;
  float xh[RAW ? 1 : VPL][VEC], dd[RAW ? 1 : VPL][VEC];
  P xc[RAW ? VPL : 1], dc[RAW ? VPL : 1];  // RAW: the row's x and dy in the I/O type
  P rv[VPL];
  float rs = 0.0f, mu_c = 0.0f;
  // The statistics are the same in every lane of a wave (a wave works on one row), so they are
  // taken into scalar registers: the ring's VGPRs are free again as soon as the row is widened,
  // and the next load into the slot needs no register copy at the loop latch (such a copy would
  // wait for that load and drain the ring).
  auto uniform = [](float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
  };
  auto widen = [&](int slot) {
    rs = uniform(rsn[slot]);
    const float mu = uniform(mun[slot]);
    if constexpr (RAW) {
      mu_c = mu;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        xc[i] = xn[slot][i];
        dc[i] = dn[slot][i];
        if constexpr (DRES) rv[i] = rn[slot][i];
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        xh[i][e] = (to_f32(xn[slot][i].v[e]) - mu) * rs;
        dd[i][e] = to_f32(dn[slot][i].v[e]);
        if constexpr (GELU != 0) {
          // GELU' from the block's table: the GELU input comes as table coordinates u = a / h
          // (gamma and beta scaled once, out of the loop, when they sit in registers), and dd
          // becomes 2 dy GELU'(a) in one FMA.
          const float u = PARAMS_IN_LDS
                              ? kGeluTabInvH * fmaf(xh[i][e], gam(i, e), bet(i, e))
                              : fmaf(xh[i][e], kGeluTabInvH * gam(i, e), kGeluTabInvH * bet(i, e));
          dd[i][e] = fmaf(dd[i][e], gelu_grad2_sign_tab(gelu_tab, u), dd[i][e]);
        }
      }
      if constexpr (DRES) rv[i] = rn[slot][i];
    }
  };

  // Prologue: rows 0 .. PD-1 in slot order, each followed by as many stores as a loop step
  // issues (zero-byte resources: dropped).  The loop top then sees the same sequence of
  // outstanding memory operations whether it comes from here or from the previous step, and the
  // compiler's wait there covers only the slot being consumed: PD rows stay in flight through
  // the row reduction.  (Without the padding the merged wait drains the ring on every step.)
  const rsrc_t none = make_rsrc(nullptr, 0);
  // GELU epilogue: every thread loads one entry of the GELU' table of its form (4 KiB,
  // L2-resident after the first block), ahead of the rows.
  float4 tab_entry;
  if constexpr (GELU != 0) {
    tab_entry = reinterpret_cast<const float4*>(GELU == 1 ? kGeluTabData
                                                          : kGeluTanhTabData)[threadIdx.x % kGeluTabN];
    asm volatile("" ::: "memory");
  }
#pragma unroll
  for (int k = 0; k < (NOPF ? 0 : PD); ++k) {
    load_row(k, k);
#pragma unroll
    for (int i = 0; i < VPL; ++i)  // distinct, non-adjacent: none merged away
      buf_store<P, FLN_BWD_STORE_POL>(zero_pack<T, VEC>(), none, static_cast<uint32_t>(4 * i));
    asm volatile("" ::: "memory");  // keeps the slots in issue order
  }
  // The GELU' table's LDS copy: its load was issued ahead of the rows, so this waits for it
  // alone.
  if constexpr (GELU != 0) {
    if (threadIdx.x < kGeluTabN) gelu_tab[threadIdx.x] = tab_entry;
    __syncthreads();
  }
  // Whole rounds of PD rows: a step past the block's last row reads zeros (its column sums add
  // nothing) and stores nothing.  An early exit from the unrolled round would make the compiler
  // wait for every slot at the loop top.
  const int rounds = (iters + PD - 1) / PD;
  for (int r = 0; r < rounds; ++r) {
#pragma unroll
  for (int sl = 0; sl < PD; ++sl) {
    const int it = r * PD + sl;
    const int64_t row = row_of(it);
    const uint32_t nb = bytes_of(it);
    // Consume slot sl (row it) and put row it + PD in flight in its place.
    if constexpr (NOPF) load_row(it, sl);
    widen(sl);
    if constexpr (!NOPF) load_row(it + PD, sl);
    // Row sums (elements past the row are zero in dy, hence in g).  A lane with 8 columns keeps
    // g = dy gamma for dx below (one multiply per element serves both); with 16 the extra VGPRs
    // would spill, and dx forms dy (rstd gamma) instead.
    constexpr bool KEEP_G = VPL * VEC <= 8;
    // x-hat and dy of element e of vector i: the widened row, or (RAW) widened from the packs
    // at each use.
    auto XH = [&](int i, int e) {
      if constexpr (RAW)
        return (to_f32(xc[i].v[e]) - mu_c) * rs;
      else
        return xh[i][e];
    };
    auto DD = [&](int i, int e) {
      if constexpr (RAW) {
        float d = to_f32(dc[i].v[e]);
        if constexpr (GELU != 0) {
          const float u = kGeluTabInvH * fmaf(XH(i, e), gam(i, e), bet(i, e));
          d = fmaf(d, gelu_grad2_sign_tab(gelu_tab, u), d);
        }
        return d;
      } else {
        return dd[i][e];
      }
    };
    float s1 = 0.0f, s2 = 0.0f;
    float gd[VPL][VEC];
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        gd[i][e] = DD(i, e) * gam(i, e);
        s1 += gd[i][e];
        s2 = fmaf(gd[i][e], XH(i, e), s2);
      }
    // RAW: the packs become opaque here, so that dx widens them again rather than the compiler
    // keeping the fp32 values of the row sums alive across the reduction.
    if constexpr (RAW) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        keep_packed(xc[i]);
        keep_packed(dc[i]);
      }
    }
    s1 = wave_allreduce<SumOp>(s1);
    s2 = wave_allreduce<SumOp>(s2);
    if (wpr > 1) {
      float(*slot)[MAXW + 16] = red[it & 1];
      if (lane == 0) {
        slot[0][wave] = s1;
        slot[1][wave] = s2;
      }
      __syncthreads();
      s1 = combine_partials<SumOp>(slot[0], rg * wpr, wpr, lane, 0.0f);
      s2 = combine_partials<SumOp>(slot[1], rg * wpr, wpr, lane, 0.0f);
    }
    // dx = rstd (g - sum(g)/N - xhat sum(g xhat)/N) = rstd g + cb + cx xhat.
    const float rsd = rs * kInvD;
    const float cb = p.rms ? 0.0f : -rsd * (s1 * inv_n);
    const float cx = -rsd * (s2 * inv_n);
    P o[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float x_h = XH(i, e), d_d = DD(i, e);
        float dxv = KEEP_G ? fmaf(rsd, gd[i][e], fmaf(cx, x_h, cb))
                           : fmaf(d_d, rsd * gam(i, e), fmaf(cx, x_h, cb));
        if constexpr (DRES) dxv += to_f32(rv[i].v[e]);
        o[i].v[e] = from_f32<T>(dxv);
        acc_g[i][e] = fmaf(d_d, x_h, acc_g[i][e]);
        acc_b[i][e] += d_d;
      }
    const rsrc_t xo = make_rsrc(DX ? DX + row * N : nullptr, nb);
#pragma unroll
    for (int i = 0; i < VPL; ++i) buf_store<P, FLN_BWD_STORE_POL>(o[i], xo, t + i * tpr);
    // The next step's (cheap) widening must not be hoisted above this step's loads and stores.
    __builtin_amdgcn_sched_barrier(0);
  }
  }

  // Stage-1 output: one fp32 partial row per block (row stride ld, a multiple of 4).
  const int64_t ld = (N + 3) & ~int64_t(3);
  const int nvec = static_cast<int>(N / VEC);
  float* outs[2] = {p.part_g, p.part_b};
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    float* out = outs[a];
    if (!out) continue;
    out += static_cast<int64_t>(blockIdx.x) * ld;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int v = t + i * tpr;
      float vals[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) vals[e] = (a == 0 ? acc_g[i][e] : acc_b[i][e]) * kInvD;
      if (rgs > 1) {
        __syncthreads();
#pragma unroll
        for (int e = 0; e < VEC; ++e) comb[(rg * tpr + t) * VEC + e] = vals[e];
        __syncthreads();
        if (rg == 0) {
          for (int k = 1; k < rgs; ++k)
#pragma unroll
            for (int e = 0; e < VEC; ++e) vals[e] += comb[(k * tpr + t) * VEC + e];
        }
      }
      if (rg == 0 && v < nvec) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) out[static_cast<int64_t>(v) * VEC + e] = vals[e];
      }
    }
  }
}

// Rows wider than the register kernel holds for their flavour (fp32 rows of 8193..16384 columns;
// fp16 rows of 16385..18432 columns with a residual gradient): one NT-thread block per row at a
// time, thread t owning vectors t + NT i
// (i < CPT) of every row.  Pass A consumes the row's raw loads (issued one row ahead, like the
// register kernel's ring), accumulates the column sums of dy xhat and dy in registers, forms the
// row sums and parks the raw x / dy vectors in LDS; after the row reduction, pass B reads them back
// and writes dx.  A thread reads back only the vectors it parked, so the staging needs no barrier:
// LDS serves as per-thread spill space for the row (128 KiB at CPT 4 and 1024 threads).
// NT = 1024 leaves 128 VGPRs per lane; NT = 768 (12 waves, 3 per SIMD) leaves 168 for the fp32
// column sums and the prefetched row of a 16-bit lane with 3 vectors (gamma in LDS).
constexpr int kLdsThreads = 1024;
constexpr int kLds16Threads = 768;

template <class T, bool DRES, int GELU, int VEC, int CPT, int NT = kLdsThreads>
__global__ __launch_bounds__(NT) void bwd_lds_kernel(const BwdParams p) {
  constexpr int kT = NT;
  constexpr int kW = kT / kWave;
  using P = Pack<T, VEC>;
  // 768-thread blocks (16-bit rows) keep gamma in LDS too, thread-private like the row: 12
  // VGPRs per lane that would otherwise spill.
  constexpr bool PARAMS_IN_LDS = NT == kLds16Threads && CPT >= 3;
  __shared__ P xs[CPT * kT], ds[CPT * kT];
  __shared__ P gs[PARAMS_IN_LDS ? CPT * kT : 1], bs[PARAMS_IN_LDS && GELU ? CPT * kT : 1];
  __shared__ float red[2][2][kW + 16];  // [parity][sum g, sum g*xhat][wave], padded
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int64_t N = p.cols;
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  const float inv_n = 1.0f / static_cast<float>(N);
  const int64_t stride = gridDim.x;
  const int iters = static_cast<int>((p.rows - 1 - blockIdx.x) / stride + 1);  // grid <= rows
  const T* X = static_cast<const T*>(p.x);
  const T* DY = static_cast<const T*>(p.dy);
  const T* DR = static_cast<const T*>(p.dres);
  T* DX = static_cast<T*>(p.dx);

  P gmr[PARAMS_IN_LDS ? 1 : CPT];
  P btr[GELU && !PARAMS_IN_LDS ? CPT : 1];
  {
    const rsrc_t gr = make_rsrc(p.gamma, row_bytes);
    const bool has_g = p.gamma != nullptr;
    const T one = from_f32<T>(1.0f);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      P gv = buf_load<P>(gr, t + i * kT);
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if (!has_g) gv.v[e] = one;
      if constexpr (PARAMS_IN_LDS)
        gs[i * kT + t] = gv;
      else
        gmr[i] = gv;
    }
    if constexpr (GELU != 0) {
      const rsrc_t br = make_rsrc(p.beta, row_bytes);
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        if constexpr (PARAMS_IN_LDS)
          bs[i * kT + t] = buf_load<P>(br, t + i * kT);
        else
          btr[i] = buf_load<P>(br, t + i * kT);
      }
    }
  }
  auto gam = [&](int i, int e) {
    if constexpr (PARAMS_IN_LDS)
      return to_f32(gs[i * kT + t].v[e]);
    else
      return to_f32(gmr[i].v[e]);
  };
  auto bet = [&](int i, int e) {
    if constexpr (PARAMS_IN_LDS)
      return to_f32(bs[i * kT + t].v[e]);
    else
      return to_f32(btr[i].v[e]);
  };
  // Upstream gradient at the LayerNorm output: dy, or dy GELU'(xhat gamma + beta) (GELU rows
  // reach this kernel only in fp32, which is not VALU-bound here: the GELU' formulas).
  auto dln = [&](float d, float xh, int i, int e) {
    if constexpr (GELU == 1) d *= gelu_erf_grad(fmaf(xh, gam(i, e), bet(i, e)));
    if constexpr (GELU == 2) d *= gelu_tanh_grad(fmaf(xh, gam(i, e), bet(i, e)));
    return d;
  };
  float acc_g[CPT][VEC], acc_b[CPT][VEC];
#pragma unroll
  for (int i = 0; i < CPT; ++i)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc_g[i][e] = acc_b[i][e] = 0.0f;

  // Raw loads of the next row (rows past the block's range read as zeros).
  P xr[CPT], dr[CPT], rr[DRES ? CPT : 1];
  float mun = 0.0f, rsn = 0.0f;
  auto load_row = [&](int it) {
    const int64_t row = static_cast<int64_t>(it) * stride + blockIdx.x;
    const uint32_t nb = it < iters ? row_bytes : 0u;
    const rsrc_t xq = make_rsrc(X + row * N, nb);
    const rsrc_t dq = make_rsrc(DY + row * N, nb);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      xr[i] = buf_load<P, FLN_BWD_LOAD_POL>(xq, t + i * kT);
      dr[i] = buf_load<P, FLN_BWD_LOAD_POL>(dq, t + i * kT);
    }
    if constexpr (DRES) {
      const rsrc_t rq = make_rsrc(DR + row * N, nb);
#pragma unroll
      for (int i = 0; i < CPT; ++i) rr[i] = buf_load<P, FLN_BWD_LOAD_POL>(rq, t + i * kT);
    }
    const uint32_t sb = nb ? 4u : 0u;
    mun = __builtin_bit_cast(
        float, BufIO<4>::load(make_rsrc(p.rms ? nullptr : p.mean + row, sb), 0));
    rsn = __builtin_bit_cast(float, BufIO<4>::load(make_rsrc(p.rstd + row, sb), 0));
  };

  load_row(0);
  for (int it = 0; it < iters; ++it) {
    const int64_t row = static_cast<int64_t>(it) * stride + blockIdx.x;
    const float mu = mun, rs = rsn;
    // Pass A: column sums, row sums, park the raw row in LDS.
    P rc[DRES ? CPT : 1];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      xs[i * kT + t] = xr[i];
      ds[i * kT + t] = dr[i];
      if constexpr (DRES) rc[i] = rr[i];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float xh = (to_f32(xr[i].v[e]) - mu) * rs;
        const float d = dln(to_f32(dr[i].v[e]), xh, i, e);
        const float g = d * gam(i, e);
        s1 += g;
        s2 = fmaf(g, xh, s2);
        acc_g[i][e] = fmaf(d, xh, acc_g[i][e]);
        acc_b[i][e] += d;
      }
    }
    load_row(it + 1);  // in flight during the reduction and pass B
    s1 = wave_allreduce<SumOp>(s1);
    s2 = wave_allreduce<SumOp>(s2);
    {
      float(*slot)[kW + 16] = red[it & 1];
      if (lane == 0) {
        slot[0][wave] = s1;
        slot[1][wave] = s2;
      }
      __syncthreads();
      s1 = combine_partials<SumOp>(slot[0], 0, kW, lane, 0.0f);
      s2 = combine_partials<SumOp>(slot[1], 0, kW, lane, 0.0f);
    }
    const float cb = p.rms ? 0.0f : -rs * (s1 * inv_n);
    const float cx = -rs * (s2 * inv_n);
    // Pass B: dx from the parked row.
    const rsrc_t xo = make_rsrc(DX ? DX + row * N : nullptr, row_bytes);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const P xv = xs[i * kT + t];
      const P dv = ds[i * kT + t];
      P o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float xh = (to_f32(xv.v[e]) - mu) * rs;
        const float d = dln(to_f32(dv.v[e]), xh, i, e);
        float dxv = fmaf(d, rs * gam(i, e), fmaf(cx, xh, cb));
        if constexpr (DRES) dxv += to_f32(rc[i].v[e]);
        o.v[e] = from_f32<T>(dxv);
      }
      buf_store<P, FLN_BWD_STORE_POL>(o, xo, t + i * kT);
    }
  }

  // Stage-1 output: one fp32 partial row per block (row stride ld, a multiple of 4).
  const int64_t ld = (N + 3) & ~int64_t(3);
  const int nvec = static_cast<int>(N / VEC);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int v = t + i * kT;
    if (v >= nvec) continue;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int64_t c = static_cast<int64_t>(blockIdx.x) * ld + static_cast<int64_t>(v) * VEC + e;
      if (p.part_g) p.part_g[c] = acc_g[i][e];
      if (p.part_b) p.part_b[c] = acc_b[i][e];
    }
  }
}

// Rows past the register and LDS tiles (16-bit rows of more than 18432 columns, save the rows
// of up to 24576 without a residual gradient (raw tiles); fp32 rows of more than 16384; long
// rows on the scalar path), any width, in two streaming passes:
//   bwd_rowstat_kernel: per row and column split, sum(g) and sum(g xhat) (g = dy' gamma,
//     dy' = dy or dy GELU'(xhat gamma + beta)) into stats[row, split]; one 256-thread block per
//     (row, split) at a time, grid-stride, eight vectors per thread in flight per array.  Few
//     rows split into column chunks so that the pass still has blocks for every CU (64 x
//     1048576 bf16: one 256-thread block per row kept 64 CUs busy);
//   bwd_colpass_kernel: a thread owns one vector column; over every G-th row (G = the blocks
//     per column tile; eight rows in flight) it writes dx from the row's statistics and
//     accumulates dgamma / dbeta in registers, then writes one partial row per block row for
//     col_reduce_kernel.
// 5 streams (x, dy twice, dx once) instead of 3, but every access is a coalesced vector stream
// and no thread holds more than eight vectors per array.
constexpr int kWideThreads = 256;
// Rows (column pass) or vector steps (row statistics) in flight per thread: 8 rather than 4
// measured 2-4% faster with few rows (bf16 backward calls, us: 128 x 131072 43.1 -> 41.2, 512 x
// 131072 122.7 -> 118.3, 64 x 1048576 119.3 -> 115.0, 1024 x 65536 123.4 -> 120.4; 2048 x
// 40960 equal), 169 VGPRs at most in these 256-thread blocks.
constexpr int kWideUnroll = 8;
constexpr int kRowstatBlocksPerCu = 8;
// Few rows: column splits per row for about kRowstatItemsPerCu (row, split) items per CU, at
// most kMaxStatSplits (the column pass sums a row's splits across a 16-lane row).  Fewer,
// longer streams keep DRAM locality (bf16 backward calls, us, splits 1 / 2 / 4 / 8 / 16:
// 64 x 1048576 309.0 / 210.4 / 163.3 / 152.5 / 175.3; 256 x 262144 159.9 / 143.2 / 141.5 /
// 146.5 / 171.6; 16 x 1048576 238.9 / 140.8 / 91.0 / 68.5 / 62.6; with 8 blocks per CU's worth
// of splits, 64 x 1048576 took 257.9).
constexpr int kRowstatItemsPerCu = 2;
constexpr int kMaxStatSplits = 16;
#ifndef FLN_COLPASS_BLOCKS_PER_CU
#define FLN_COLPASS_BLOCKS_PER_CU 2
#endif

template <class T, int GELU, int VEC>
__global__ __launch_bounds__(kWideThreads) void bwd_rowstat_kernel(const BwdParams p,
                                                                   float2* stats) {
  using P = Pack<T, VEC>;
  constexpr int kW = kWideThreads / kWave;
  __shared__ float red[2][2][kW + 16];
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int64_t N = p.cols;
  const int nvec = static_cast<int>(N / VEC);
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  const T* X = static_cast<const T*>(p.x);
  const T* DY = static_cast<const T*>(p.dy);
  const rsrc_t gr = make_rsrc(p.gamma, row_bytes);
  const rsrc_t br = make_rsrc(p.beta, row_bytes);  // GELU only; absent beta reads as zeros
  const bool has_g = p.gamma != nullptr;
  const int S = p.stat_splits;
  const int64_t items = p.rows * S;
  int parity = 0;
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x, parity ^= 1) {
    const int64_t row = item / S;
    const int64_t v_lo = (item - row * S) * p.stat_chunk;
    const int64_t v_hi = v_lo + p.stat_chunk < nvec ? v_lo + p.stat_chunk : nvec;
    // x and dy read as zeros past the split (g = 0 there), gamma / beta over the whole row.
    const uint32_t split_bytes = static_cast<uint32_t>(v_hi * VEC * sizeof(T));
    const rsrc_t xr = make_rsrc(X + row * N, split_bytes);
    const rsrc_t dr = make_rsrc(DY + row * N, split_bytes);
    const float mu = p.rms ? 0.0f : p.mean[row];
    const float rs = p.rstd[row];
    float s1 = 0.0f, s2 = 0.0f;
    for (int v0 = static_cast<int>(v_lo) + t; v0 < v_hi; v0 += kWideUnroll * kWideThreads) {
      P xv[kWideUnroll], dv[kWideUnroll], gv[kWideUnroll], bv[GELU ? kWideUnroll : 1];
#pragma unroll
      for (int u = 0; u < kWideUnroll; ++u) {  // vectors past the row read as zeros
        const int v = v0 + u * kWideThreads;
        xv[u] = buf_load<P, kStream>(xr, v);
        dv[u] = buf_load<P, kStream>(dr, v);
        gv[u] = buf_load<P>(gr, v);
        if constexpr (GELU != 0) bv[u] = buf_load<P>(br, v);
      }
#pragma unroll
      for (int u = 0; u < kWideUnroll; ++u)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float xh = (to_f32(xv[u].v[e]) - mu) * rs;
          const float gam = has_g ? to_f32(gv[u].v[e]) : 1.0f;
          float d = to_f32(dv[u].v[e]);
          if constexpr (GELU == 1) d *= gelu_erf_grad(fmaf(xh, gam, to_f32(bv[u].v[e])));
          if constexpr (GELU == 2) d *= gelu_tanh_grad(fmaf(xh, gam, to_f32(bv[u].v[e])));
          const float g = d * gam;
          s1 += g;
          s2 = fmaf(g, xh, s2);
        }
    }
    s1 = wave_allreduce<SumOp>(s1);
    s2 = wave_allreduce<SumOp>(s2);
    float(*slot)[kW + 16] = red[parity];
    if (lane == 0) {
      slot[0][wave] = s1;
      slot[1][wave] = s2;
    }
    __syncthreads();
    s1 = combine_partials<SumOp>(slot[0], 0, kW, lane, 0.0f);
    s2 = combine_partials<SumOp>(slot[1], 0, kW, lane, 0.0f);
    if (t == 0) stats[item] = make_float2(s1, s2);
  }
}

template <class T, bool DRES, int GELU, int VEC>
__global__ __launch_bounds__(kWideThreads) void bwd_colpass_kernel(const BwdParams p,
                                                                   const float2* stats) {
  using P = Pack<T, VEC>;
  const int v = blockIdx.x * kWideThreads + threadIdx.x;  // this thread's vector column
  const int64_t N = p.cols;
  const int nvec = static_cast<int>(N / VEC);
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  const float inv_n = 1.0f / static_cast<float>(N);
  // Block y takes rows y, y + G, y + 2G, ... (G = gridDim.y): all blocks stream through one
  // window of adjacent rows at a time, which keeps DRAM page locality (contiguous row chunks
  // per block had every block in a different part of the tensors at once).
  const int64_t G = gridDim.y;
  const T* X = static_cast<const T*>(p.x);
  const T* DY = static_cast<const T*>(p.dy);
  const T* DR = static_cast<const T*>(p.dres);
  T* DX = static_cast<T*>(p.dx);
  P gv = buf_load<P>(make_rsrc(p.gamma, row_bytes), v);
  if (p.gamma == nullptr)
#pragma unroll
    for (int e = 0; e < VEC; ++e) gv.v[e] = from_f32<T>(1.0f);
  P bv{};
  if constexpr (GELU != 0) bv = buf_load<P>(make_rsrc(p.beta, row_bytes), v);
  float acc_g[VEC], acc_b[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc_g[e] = acc_b[e] = 0.0f;
  const int split = threadIdx.x & 15;
  for (int64_t row = blockIdx.y; row < p.rows; row += kWideUnroll * G) {
    P xv[kWideUnroll], dv[kWideUnroll], rv[DRES ? kWideUnroll : 1];
    float mu[kWideUnroll], rs[kWideUnroll], cb[kWideUnroll], cx[kWideUnroll];
    float2 sp[kWideUnroll];
#pragma unroll
    for (int u = 0; u < kWideUnroll; ++u) {
      const bool in = row + u * G < p.rows;  // uniform
      const int64_t r = in ? row + u * G : row;
      const uint32_t nb = in ? row_bytes : 0u;
      xv[u] = buf_load<P, kStream>(make_rsrc(X + r * N, nb), v);
      dv[u] = buf_load<P, kStream>(make_rsrc(DY + r * N, nb), v);
      if constexpr (DRES) rv[u] = buf_load<P, kStream>(make_rsrc(DR + r * N, nb), v);
      mu[u] = p.rms ? 0.0f : p.mean[r];
      rs[u] = p.rstd[r];
      // The row's splits: lane k of each 16-lane row loads split k.
      sp[u] = split < p.stat_splits ? stats[r * p.stat_splits + split] : make_float2(0.0f, 0.0f);
    }
#pragma unroll
    for (int u = 0; u < kWideUnroll; ++u) {  // splits summed in a fixed order (reduce16)
      const float s1 = reduce16<SumOp>(sp[u].x), s2 = reduce16<SumOp>(sp[u].y);
      cb[u] = p.rms ? 0.0f : -rs[u] * (s1 * inv_n);
      cx[u] = -rs[u] * (s2 * inv_n);
    }
#pragma unroll
    for (int u = 0; u < kWideUnroll; ++u) {
      const bool in = row + u * G < p.rows;
      const int64_t r = in ? row + u * G : row;
      P o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float xh = (to_f32(xv[u].v[e]) - mu[u]) * rs[u];
        const float gam = to_f32(gv.v[e]);
        float d = to_f32(dv[u].v[e]);
        if constexpr (GELU == 1) d *= gelu_erf_grad(fmaf(xh, gam, to_f32(bv.v[e])));
        if constexpr (GELU == 2) d *= gelu_tanh_grad(fmaf(xh, gam, to_f32(bv.v[e])));
        float dxv = fmaf(d, rs[u] * gam, fmaf(cx[u], xh, cb[u]));
        if constexpr (DRES) dxv += to_f32(rv[u].v[e]);
        o.v[e] = from_f32<T>(dxv);
        if (in) {  // rows past the tensor were read as zeros: d = 0, but keep the sums exact
          acc_g[e] = fmaf(d, xh, acc_g[e]);
          acc_b[e] += d;
        }
      }
      buf_store<P, kStream>(o, make_rsrc(DX ? DX + r * N : nullptr, in ? row_bytes : 0u), v);
    }
  }
  if (v >= nvec) return;
  if (p.out_g != nullptr || p.out_b != nullptr) {  // one block row: these sums are final
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int64_t j = static_cast<int64_t>(v) * VEC + e;
      if (p.out_g) store_param(p.out_g, p.out_dtype, j, acc_g[e]);
      if (p.out_b) store_param(p.out_b, p.out_dtype, j, acc_b[e]);
    }
    return;
  }
  const int64_t ld = (N + 3) & ~int64_t(3);
  const int64_t c = static_cast<int64_t>(blockIdx.y) * ld + static_cast<int64_t>(v) * VEC;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    if (p.part_g) p.part_g[c + e] = acc_g[e];
    if (p.part_b) p.part_b[c + e] = acc_b[e];
  }
}

// Rows too long for the register path: one block per row chunk, three strided passes per row,
// column partials accumulated in place in the block's partial row (each column is owned by one
// thread of the block, so the read-modify-write is race free).
template <class T>
__global__ __launch_bounds__(1024) void bwd_loop_kernel(const BwdParams p) {
  __shared__ float red[2][2][16];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int64_t N = p.cols;
  const int64_t ld = (N + 3) & ~int64_t(3);
  const T* gm = static_cast<const T*>(p.gamma);
  const T* bt = static_cast<const T*>(p.beta);
  // Upstream gradient at the LayerNorm output: dy, or dy GELU'(xhat gamma + beta).
  auto dln = [&](float d, float xh, int64_t j) {
    if (!p.gelu) return d;
    const float a = fmaf(xh, gm ? to_f32(gm[j]) : 1.0f, bt ? to_f32(bt[j]) : 0.0f);
    return d * gelu_grad(a, p.gelu);
  };
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * p.rows_per_block;
  const int64_t r1 = r0 + p.rows_per_block < p.rows ? r0 + p.rows_per_block : p.rows;
  float* pg = p.part_g ? p.part_g + static_cast<int64_t>(blockIdx.x) * ld : nullptr;
  float* pb = p.part_b ? p.part_b + static_cast<int64_t>(blockIdx.x) * ld : nullptr;
  for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
    if (pg) pg[j] = 0.0f;
    if (pb) pb[j] = 0.0f;
  }
  const float inv_n = 1.0f / static_cast<float>(N);
  int buf = 0;
  for (int64_t row = r0; row < r1; ++row, buf ^= 1) {
    const T* x = static_cast<const T*>(p.x) + row * N;
    const T* dy = static_cast<const T*>(p.dy) + row * N;
    const float mu = p.rms ? 0.0f : p.mean[row];
    const float rs = p.rstd[row];
    float s1 = 0.0f, s2 = 0.0f;
    for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
      const float xh = (to_f32(x[j]) - mu) * rs;
      const float g = dln(to_f32(dy[j]), xh, j) * (gm ? to_f32(gm[j]) : 1.0f);
      s1 += g;
      s2 += g * xh;
    }
    s1 = wave_allreduce<SumOp>(s1);
    s2 = wave_allreduce<SumOp>(s2);
    if (lane == 0) {
      red[buf][0][wave] = s1;
      red[buf][1][wave] = s2;
    }
    __syncthreads();
    s1 = red[buf][0][0];
    s2 = red[buf][1][0];
    for (int k = 1; k < nw; ++k) {
      s1 += red[buf][0][k];
      s2 += red[buf][1][k];
    }
    const float c1 = p.rms ? 0.0f : s1 * inv_n, c2 = s2 * inv_n;
    T* dx = p.dx ? static_cast<T*>(p.dx) + row * N : nullptr;
    const T* dres = p.dres ? static_cast<const T*>(p.dres) + row * N : nullptr;
    for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
      const float xh = (to_f32(x[j]) - mu) * rs;
      const float d = dln(to_f32(dy[j]), xh, j);
      const float g = d * (gm ? to_f32(gm[j]) : 1.0f);
      if (dx) {
        float v = rs * (g - c1 - xh * c2);
        if (dres) v += to_f32(dres[j]);
        dx[j] = from_f32<T>(v);
      }
      if (pg) pg[j] += d * xh;
      if (pb) pb[j] += d;
    }
  }
}

constexpr int kCrSlices = FLN_CR_SLICES;
constexpr int kCrThreads = kCrQuads * kCrSlices;

// Stage 2: one quad block per 256-thread block (32 slices), >= 256 blocks at 4096 columns.
__global__ __launch_bounds__(kCrThreads) void col_reduce_kernel(const ColReduceArgs a) {
  __shared__ float4 comb[kCrThreads];
  reduce_quad_block(a, blockIdx.x, kCrSlices, comb);
}

// Stage 2 for few partial rows (G <= 8: the two-pass backward's column pass over very wide rows,
// tiny batches): every thread owns one column quad of one array and adds its G partial rows in
// order, all loads in flight at once; no LDS, no barrier.  The sliced kernel would idle three
// quarters of its threads at G = 8, over 8192 blocks at 131072 columns (bf16 512 x 131072
// backward call 133.8 -> 129.5 us; at G = 16 the flat grid gets too few threads: 16 x 8192
// 9.4 -> 10.0 us).
constexpr int kCrFlatMaxG = 8;
constexpr int kCrFlatThreads = 256;

__host__ __device__ inline int64_t flat_blocks(const ColReduceArgs& a) {
  const int64_t quads = ((a.N + 3) & ~int64_t(3)) >> 2;
  return a.ny * ((quads + kCrFlatThreads - 1) / kCrFlatThreads);
}

__global__ __launch_bounds__(kCrFlatThreads) void col_reduce_flat_kernel(const ColReduceArgs a) {
  const int64_t ld = (a.N + 3) & ~int64_t(3);
  const int64_t per_array = ((ld >> 2) + kCrFlatThreads - 1) / kCrFlatThreads;
  const int y = static_cast<int>(blockIdx.x / per_array);
  const int64_t c = ((blockIdx.x - y * per_array) * kCrFlatThreads + threadIdx.x) * 4;
  if (c >= a.N) return;
  const float* col = a.part[y] + c;
  float4 v[kCrFlatMaxG];
#pragma unroll
  for (int k = 0; k < kCrFlatMaxG; ++k)
    if (k < a.G) v[k] = *reinterpret_cast<const float4*>(col + k * ld);
  float4 r = v[0];
#pragma unroll
  for (int k = 1; k < kCrFlatMaxG; ++k)
    if (k < a.G) add4(r, v[k]);
  const float rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (c + e < a.N) store_param(a.out[y], a.out_dtype, c + e, rr[e]);
}

namespace {

// Largest vectors per lane instantiated for the backward register path: 2 vectors (16
// elements of a 16-bit type, 8 of fp32) on the vector path, 8 on the scalar path.
constexpr int bwd_max_vpl(int vec, int es) { return vec == 1 ? 8 : 2; }
// 16-bit rows of 16385..18432 columns: one row per 768-thread block, 3 vectors per lane.
constexpr int kReg3Threads = 768;

int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Stage-1 launch (resident == nullptr) or, with `resident`, the number of blocks of that
// instantiation that fit on the device at once (occupancy x CUs, cached per device).
template <class T, bool DRES, int GELU, int VEC, int VPL, int MAXT>
int launch_stage1_k(const BwdParams& p, int64_t blocks, int threads, hipStream_t s,
                    int64_t* resident) {
  auto kernel = bwd_reg_kernel<T, DRES, GELU, VEC, VPL, MAXT>;
  // The GELU kernels fill their LDS table with one entry per thread.
  if (GELU != 0 && threads < kGeluTabN) return FLN_ERR_INVALID;
  if (resident) {
    if (threads < kWave || threads > MAXT || threads % kWave != 0) return FLN_ERR_INVALID;
    static std::atomic<int> per_cu[MAXT / kWave + 1][64];  // [waves per block][device]
    const int dev = current_device();
    std::atomic<int>& slot = per_cu[threads / kWave][dev];
    int v = slot.load(std::memory_order_relaxed);
    if (v == 0) {
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kernel, threads, 0) != hipSuccess ||
          v < 1)
        v = 1;
      slot.store(v, std::memory_order_relaxed);
    }
    *resident = static_cast<int64_t>(v) * device_cu_count();
    return 0;
  }
  static std::atomic<void*> fn_cache[64];
  return launch_cached(kernel, fn_cache, dim3(blocks), dim3(threads), s, p);
}

template <class T, int VEC, int VPL>
int launch_stage1(const BwdParams& p, int64_t blocks, int threads, hipStream_t s,
                  int64_t* resident) {
  if constexpr (VPL == 4 && VEC == 8 && sizeof(T) == 2) {
    // Four vectors per lane on the 16-bit vector path: the raw tiles without a prefetched row
    // (LayerNorm / RMSNorm only).
    if (threads != 1024 || p.gelu != 0 || p.dres) return FLN_ERR_INVALID;
    return launch_stage1_k<T, false, 0, VEC, 4, 1024>(p, blocks, threads, s, resident);
  } else if constexpr ((VPL == 3 || VPL == 4) && sizeof(T) == 4 && VEC == 4) {
    // fp32 rows of 8193..12288 columns (every flavour) and 12289..16384 (LayerNorm / RMSNorm):
    // 1024-thread blocks.
    if (threads != 1024) return FLN_ERR_INVALID;
    if constexpr (VPL == 4) {
      if (p.gelu != 0 || p.dres) return FLN_ERR_INVALID;
    } else {
      if (p.gelu == 1)
        return launch_stage1_k<T, false, 1, VEC, 3, 1024>(p, blocks, threads, s, resident);
      if (p.gelu == 2)
        return launch_stage1_k<T, false, 2, VEC, 3, 1024>(p, blocks, threads, s, resident);
      if (p.dres)
        return launch_stage1_k<T, true, 0, VEC, 3, 1024>(p, blocks, threads, s, resident);
    }
    return launch_stage1_k<T, false, 0, VEC, VPL, 1024>(p, blocks, threads, s, resident);
  } else {
    // Three vectors per lane of 16-bit rows: 768-thread blocks (168 VGPRs per lane), or the raw
    // tiles of 1024-thread blocks (no residual gradient).
    if constexpr (VPL == 3) {
      if (threads == 1024) {
        if (p.dres) return FLN_ERR_INVALID;
        if (p.gelu == 1)
          return launch_stage1_k<T, false, 1, VEC, 3, 1024>(p, blocks, threads, s, resident);
        if (p.gelu == 2)
          return launch_stage1_k<T, false, 2, VEC, 3, 1024>(p, blocks, threads, s, resident);
        return launch_stage1_k<T, false, 0, VEC, 3, 1024>(p, blocks, threads, s, resident);
      }
      if (threads != kReg3Threads) return FLN_ERR_INVALID;
    }
    constexpr int MAXT = VPL == 3 ? kReg3Threads : 1024;
    // GELU is never combined with a residual gradient (no entry point passes both).
    if (p.gelu == 1)
      return launch_stage1_k<T, false, 1, VEC, VPL, MAXT>(p, blocks, threads, s, resident);
    if (p.gelu == 2)
      return launch_stage1_k<T, false, 2, VEC, VPL, MAXT>(p, blocks, threads, s, resident);
    if (p.dres)
      return launch_stage1_k<T, true, 0, VEC, VPL, MAXT>(p, blocks, threads, s, resident);
    return launch_stage1_k<T, false, 0, VEC, VPL, MAXT>(p, blocks, threads, s, resident);
  }
}

template <class T, int VEC>
int launch_stage1_vpl(const BwdParams& p, int vpl, int64_t blocks, int threads, hipStream_t s,
                      int64_t* resident) {
  constexpr int CAP = bwd_max_vpl(VEC, sizeof(T));
  switch (vpl) {
    case 1: return launch_stage1<T, VEC, 1>(p, blocks, threads, s, resident);
    case 2:
      if constexpr (CAP >= 2) return launch_stage1<T, VEC, 2>(p, blocks, threads, s, resident);
      return FLN_ERR_INVALID;
    case 3:  // 16-bit rows of 16385..24576 columns (768 / 1024 threads), fp32 8193..12288
      if constexpr ((sizeof(T) == 2 && VEC == 8) || (sizeof(T) == 4 && VEC == 4))
        return launch_stage1<T, VEC, 3>(p, blocks, threads, s, resident);
      return FLN_ERR_INVALID;
    case 4:
      if constexpr (CAP >= 4 || VEC * sizeof(T) == 16)
        return launch_stage1<T, VEC, 4>(p, blocks, threads, s, resident);
      return FLN_ERR_INVALID;
    case 8:
      if constexpr (CAP >= 8) return launch_stage1<T, VEC, 8>(p, blocks, threads, s, resident);
      return FLN_ERR_INVALID;
    default: return FLN_ERR_INVALID;
  }
}

template <class T, int VEC>
int launch_two_pass(const BwdParams& p, const BwdGeometry& geo, hipStream_t s) {
  float2* stats = reinterpret_cast<float2*>(p.rowstat);
  const int64_t cap = kRowstatBlocksPerCu * static_cast<int64_t>(device_cu_count());
  const int64_t items = p.rows * p.stat_splits;
  const dim3 g1(static_cast<unsigned>(items < cap ? items : cap)), blk(kWideThreads);
  const int64_t nvec = p.cols / VEC;
  const dim3 g2(static_cast<unsigned>((nvec + kWideThreads - 1) / kWideThreads),
                static_cast<unsigned>(geo.blocks));
  if (p.gelu == 1) {
    hipLaunchKernelGGL((bwd_rowstat_kernel<T, 1, VEC>), g1, blk, 0, s, p, stats);
    hipLaunchKernelGGL((bwd_colpass_kernel<T, false, 1, VEC>), g2, blk, 0, s, p, stats);
  } else if (p.gelu == 2) {
    hipLaunchKernelGGL((bwd_rowstat_kernel<T, 2, VEC>), g1, blk, 0, s, p, stats);
    hipLaunchKernelGGL((bwd_colpass_kernel<T, false, 2, VEC>), g2, blk, 0, s, p, stats);
  } else {
    hipLaunchKernelGGL((bwd_rowstat_kernel<T, 0, VEC>), g1, blk, 0, s, p, stats);
    if (p.dres)
      hipLaunchKernelGGL((bwd_colpass_kernel<T, true, 0, VEC>), g2, blk, 0, s, p, stats);
    else
      hipLaunchKernelGGL((bwd_colpass_kernel<T, false, 0, VEC>), g2, blk, 0, s, p, stats);
  }
  return static_cast<int>(hipGetLastError());
}

template <class T, int VEC, int CPT>
int launch_lds(const BwdParams& p, int64_t blocks, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(blocks)), block(kLdsThreads);
  if (p.gelu == 1)
    hipLaunchKernelGGL((bwd_lds_kernel<T, false, 1, VEC, CPT>), grid, block, 0, s, p);
  else if (p.gelu == 2)
    hipLaunchKernelGGL((bwd_lds_kernel<T, false, 2, VEC, CPT>), grid, block, 0, s, p);
  else if (p.dres)
    hipLaunchKernelGGL((bwd_lds_kernel<T, true, 0, VEC, CPT>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((bwd_lds_kernel<T, false, 0, VEC, CPT>), grid, block, 0, s, p);
  return static_cast<int>(hipGetLastError());
}

template <class T>
int dispatch_backward(BwdParams p, const BwdGeometry& geo, hipStream_t s,
                      int64_t* resident = nullptr) {
  p.wpr = geo.wpr;
  p.rgs = geo.rgs;
  p.rows_per_block = geo.rows_per_block;
  constexpr int VV = 16 / sizeof(T);
  if (!resident && tuning().debug_geometry)
    fprintf(stderr, "fln backward: rows=%lld cols=%lld vec=%d -> %s wpr=%d vpl=%d threads=%d "
            "blocks=%lld\n", static_cast<long long>(p.rows), static_cast<long long>(p.cols),
            geo.vec, geo.lds_cpt > 0 ? "lds" : geo.two_pass ? "two-pass"
                     : !geo.reg_path ? "loop" : "registers",
            geo.wpr, geo.vpl, geo.threads, static_cast<long long>(geo.blocks));
  if (geo.lds_cpt > 0) {
    if (resident) {
      *resident = geo.blocks;  // one block per CU (the staged row fills most of the LDS)
      return 0;
    }
    if constexpr (sizeof(T) == 4) {
      if (geo.lds_cpt == 3) return launch_lds<T, VV, 3>(p, geo.blocks, s);
      if (geo.lds_cpt == 4) return launch_lds<T, VV, 4>(p, geo.blocks, s);
    } else {
      if (geo.threads == kLds16Threads) {
        const dim3 grid(static_cast<unsigned>(geo.blocks)), block(kLds16Threads);
        if (geo.lds_cpt == 3 && p.dres && !p.gelu)
          hipLaunchKernelGGL((bwd_lds_kernel<T, true, 0, VV, 3, kLds16Threads>), grid, block, 0,
                             s, p);
        else
          return FLN_ERR_INVALID;
        return static_cast<int>(hipGetLastError());
      }
    }
    return FLN_ERR_INVALID;
  }
  if (geo.two_pass) {
    if (resident) {
      *resident = geo.blocks;  // partial rows = row chunks of the column pass
      return 0;
    }
    if (geo.vec == VV) return launch_two_pass<T, VV>(p, geo, s);
    return launch_two_pass<T, 1>(p, geo, s);
  }
  if (!geo.reg_path) {
    if (resident) {
      *resident = geo.blocks;  // the looped kernel takes any grid
      return 0;
    }
    hipLaunchKernelGGL((bwd_loop_kernel<T>), dim3(geo.blocks), dim3(1024), 0, s, p);
    return static_cast<int>(hipGetLastError());
  }
  if (geo.vec == VV)
    return launch_stage1_vpl<T, VV>(p, geo.vpl, geo.blocks, geo.threads, s, resident);
  return launch_stage1_vpl<T, 1>(p, geo.vpl, geo.blocks, geo.threads, s, resident);
}

}  // namespace

int64_t workspace_partial_rows(int64_t rows) {
  const int64_t g = 4 * static_cast<int64_t>(device_cu_count());
  return rows < g ? rows : g;
}

BwdGeometry backward_geometry(int64_t rows, int64_t cols, int dtype, bool vec_ok, bool dres,
                              bool gelu, bool have_workspace) {
  BwdGeometry g{};
  const int es = element_size(dtype);
  const int vv = es > 0 ? 16 / es : 1;
  g.vec = (vec_ok && cols % vv == 0) ? vv : 1;
  const int64_t nvec = cols / g.vec;
  auto per_lane = [&](int w) { return (nvec + kWave * w - 1) / (kWave * w); };
  // Elements per lane: 8 by default (x-hat, dy, g, gamma, both column accumulators and the
  // prefetched raw rows of a lane's columns stay in registers: 84-98 VGPRs for fp32 rows at 2
  // vectors per lane, one row in flight); more only for rows too wide for 16 waves.  fp32
  // backward calls, us, 4 -> 8 elements per lane: 300 x 768 9.31 -> 8.81, 4096 x 768 13.79 ->
  // 13.19, 16384 x 768 31.46 -> 30.26, 16384 x 1024 38.12 -> 37.68, 8192 x 2048 38.60 ->
  // 38.13, 4096 x 3072 32.62 -> 31.06, 1024 x 4096 17.74 -> 17.14, 8192 x 4096 70.54 -> 69.36
  // (RMSNorm 69.02 -> 67.77); 32 x 768 and 1024 x 1024 tied.  The fp32 scalar path (rows not
  // whole 16-byte vectors) keeps 4.
  const Tuning& tun = tuning();
  const int epl = tun.bwd_epl > 0 ? tun.bwd_epl : (es == 4 && g.vec == 1 ? 4 : 8);
  int cap = (epl >= g.vec ? epl : g.vec) / g.vec;
  if (cap > bwd_max_vpl(g.vec, es)) cap = bwd_max_vpl(g.vec, es);
  int wpr = 1;
  while (per_lane(wpr) > cap && wpr < 16) wpr *= 2;
  if (per_lane(wpr) > cap) cap = bwd_max_vpl(g.vec, es);
  const int forced = tun.bwd_wpr;
  if (forced >= 1 && forced <= 16 && (forced & (forced - 1)) == 0 && per_lane(forced) <= cap)
    wpr = forced;
  // 16-bit rows of 9-12 whole waves of vectors (4608-6144 columns) take a row group of exactly
  // that many waves instead of 16 with 4-7 of them idle.  bf16 backward calls, us, 8192 rows:
  // 4608 49.4 -> 44.8, 5120 50.6 -> 49.0, 5632 56.7 -> 53.4, 6144 59.6 -> 57.1 (16384 rows:
  // 5120 87.9 / 88.1, 6144 105.8 -> 104.1).  Fewer waves than 9 in a power-of-two group lost
  // (16384 x 2560, 5 of 8 waves: 47.8 -> 48.8; 32768 x 1536, 3 of 4: 55.3 -> 55.9), 14 of 16
  // tied (8192 x 7168 66.5 / 66.6).
  if (es == 2 && g.vec == 8 && wpr == 16 && cap == 1 && nvec % kWave == 0 &&
      nvec / kWave >= 9 && nvec / kWave <= 12 && forced <= 0)
    wpr = static_cast<int>(nvec / kWave);
  // 16-bit LayerNorm / RMSNorm rows whose one-vector tile leaves lanes masked (768, 1280, 1536,
  // 2560, 3072, 3584, 7168 columns, ...), with at least 16 rows per CU: 2 vectors per lane over
  // half the waves (one row in flight instead of two).  bf16 backward calls, us: 16384 x 768
  // 20.31 -> 19.79 (RMSNorm 19.59 -> 18.70), 65536 x 768 54.83 -> 54.24, 16384 x 1280 28.12 ->
  // 27.97, 16384 x 1536 31.91 -> 31.37 (fp16 32.20 -> 31.42), 4096 x 2560 20.03 -> 19.43, 8192
  // x 2560 29.28 -> 28.67, 16384 x 3072 55.92 -> 54.63, 16384 x 3584 64.17 -> 63.19, 8192 x
  // 7168 66.31 -> 65.93.  Whole power-of-two tiles keep one vector (16384 x 1024 23.07 / 23.74,
  // 16384 x 2048 38.44 / 38.65, 8192 x 4096 39.84 / 40.50), and so do the GELU flavours, whose
  // 2-vector tiles keep gamma / beta in LDS (16384 x 768 tanh 22.4 -> 25.1, 16384 x 3072 erf
  // 63.4 -> 68.8).
  if (es == 2 && g.vec == 8 && cap == 1 && forced <= 0 && tun.bwd_epl <= 0 && !gelu && !dres &&
      nvec % (static_cast<int64_t>(kWave) * wpr) != 0 && rows >= 16 * device_cu_count()) {
    cap = 2;
    wpr = 1;
    while (per_lane(wpr) > cap && wpr < 16) wpr *= 2;
  }
  g.reg_path = per_lane(wpr) <= cap;
  g.wpr = g.reg_path ? wpr : 16;
  g.vpl = g.reg_path ? next_pow2(static_cast<int>(per_lane(wpr))) : 0;
  int threads = tun.bwd_threads > 0 ? tun.bwd_threads : 1024;
  if (threads != 256 && threads != 512 && threads != 1024) threads = 1024;
  // Blocks per CU (one block per CU leaves one partial row per CU for the column reduction).
  int per_cu = 1;
  bool few_rows = false;
  // Few rows: 1024-thread blocks (1024 / (64 wpr) rows each) would leave CUs idle; take the
  // smallest block that holds a row group and still needs no more blocks than there are CUs
  // (HIP graph latency per call, us: 8 x 4096 bf16 9.21 -> 7.00, 512 x 1024 bf16 9.98 -> 7.84,
  // 32 x 768 fp32 8.26 -> 5.89; past one block per CU, 300 x 4096 bf16 went 12.80 -> 15.09 with
  // twice the column partials, so it keeps 1024).
  if (tun.bwd_threads <= 0 && g.reg_path) {
    for (int t = 256; t < 1024; t *= 2) {
      if (t < kWave * g.wpr) continue;
      const int per_block = t / (kWave * g.wpr);
      if ((rows + per_block - 1) / per_block <= device_cu_count()) {
        threads = t;
        few_rows = true;
        break;
      }
    }
    // Many rows, one block per CU: the smaller block (512 threads, 8 waves) as soon as its row
    // groups move >= 24 KiB per step (x, dy, dx and dres rows; 48 KiB with the GELU epilogue,
    // whose VALU work wants the waves), 1024 threads otherwise.  Fewer rows in progress keep
    // DRAM locality: bf16 backward calls on MI355X, us (1024 -> 512 threads): 8192 x 4096
    // 41.1 -> 40.1, 16384 x 2048 39.9 -> 38.6, 16384 x 1024 24.4 -> 23.4, 65536 x 512 42.0 ->
    // 39.4; 32768 x 768 (18 KiB at 512 threads) 32.6 -> 35.5, so it keeps 1024.
    if (!few_rows) {
      const int64_t moved = cols * es * (dres ? 4 : 3);
      const int64_t target = gelu ? (48 << 10) : (24 << 10);
      threads = 1024;
      if (512 >= kWave * g.wpr && (512 / (kWave * g.wpr)) * moved >= target) threads = 512;
    }
  }
  if (!g.reg_path) threads = 1024;
  if (threads < kWave * g.wpr) threads = kWave * g.wpr;
  if (g.reg_path) threads = threads / (kWave * g.wpr) * (kWave * g.wpr);  // whole row groups
  g.threads = threads;
  g.rgs = g.reg_path ? threads / (kWave * g.wpr) : 1;
  if (few_rows || tun.bwd_threads > 0) per_cu = 1024 / threads;  // 16 waves per CU in total
  if (tun.bwd_grid_mult >= 1 && tun.bwd_grid_mult <= 4) per_cu = tun.bwd_grid_mult;
  const int64_t max_blocks = static_cast<int64_t>(device_cu_count()) * per_cu;
  int64_t blocks = (rows + g.rgs - 1) / g.rgs;
  if (blocks > max_blocks) blocks = max_blocks;
  if (blocks < 1) blocks = 1;
  g.rows_per_block = (rows + blocks - 1) / blocks;
  // The register path deals row groups out grid-stride over `blocks`; the looped fallback
  // gives each block a contiguous chunk of rows_per_block rows.
  g.blocks = g.reg_path ? blocks : (rows + g.rows_per_block - 1) / g.rows_per_block;
  // 16-bit rows of 16385..18432 columns on the vector path: the register kernel with one row
  // per 768-thread block and 3 vectors per lane (xhat, dy, both column sums and the next row in
  // flight fit the 168 VGPRs a lane has at 3 waves per SIMD; the residual-gradient and GELU
  // flavours park gamma / beta in LDS).  Against the LDS-staged kernel below, bf16 4096 x 18432
  // backward calls, us: LN 106.1 -> 90.5, RMSNorm 93.1 -> 84.9, + residual gradient 129.2 ->
  // 115.0, GELU erf 145.8 -> 99.3, tanh 147.9 -> 99.2; 300 x 18432 LN 42.6 -> 26.6.  fp16 with a
  // residual gradient spills there (52 B per lane) and keeps the LDS-staged kernel (130.2
  // against 129.3 us).
  if (!g.reg_path && es == 2 && g.vec == 8 && nvec > 2 * 1024 && nvec <= 3 * kReg3Threads &&
      !(dres && dtype == FLN_F16) && tun.bwd_no_lds == 0) {
    g.reg_path = true;
    g.vpl = 3;
    g.threads = kReg3Threads;
    g.wpr = kReg3Threads / kWave;
    g.rgs = 1;
    g.blocks = rows < device_cu_count() ? rows : device_cu_count();
    g.rows_per_block = (rows + g.blocks - 1) / g.blocks;
  }
  // 16-bit rows of 18433..24576 columns without a residual gradient: the raw tiles (3 vectors
  // per lane of a 1024-thread block, the row kept in the I/O type).  Against the LDS-staged
  // kernel with 4 vectors per thread in 768 threads they replaced, bf16 backward calls, us:
  // 4096 x 20480 LN 146.0 -> 101.4, RMSNorm 129.5 -> 95.8, 4096 x 24576 163.8 -> 118.7 (fp16
  // 161.4 -> 117.5), 2048 x 19000 93.0 -> 63.2, 300 x 24576 56.1 -> 32.5; the GELU flavours
  // against the two passes (68 B of spill left): 4096 x 20480 erf 220.8 -> 184.3, tanh 201.1
  // -> 184.0, 4096 x 24576 erf 243.8 -> 197.3.
  if (!g.reg_path && es == 2 && g.vec == 8 && nvec > 3 * kReg3Threads && nvec <= 3 * 1024 &&
      !dres && tun.bwd_no_lds == 0) {
    g.reg_path = true;
    g.vpl = 3;
    g.threads = 1024;
    g.wpr = 1024 / kWave;
    g.rgs = 1;
    g.blocks = rows < device_cu_count() ? rows : device_cu_count();
    g.rows_per_block = (rows + g.blocks - 1) / g.blocks;
  }
  // fp32 rows of 8193..12288 columns: the register kernel with 3 vectors per lane in 1024-thread
  // blocks (107-128 VGPRs; 28 B spilled with GELU); LayerNorm / RMSNorm rows of 12289..16384: 4
  // vectors per lane (36 B spilled).  Against the LDS-staged kernel, backward calls, us: 4096 x
  // 12288 LN 113.5 -> 108.6, RMSNorm 108.5 -> 105.4, GELU erf 121.4 -> 118.0, + residual 149.4
  // -> 144.3, 2048 x 12288 tanh 71.2 -> 68.2, 300 x 12288 28.9 -> 24.6; 4096 x 16384 LN 153.9
  // -> 147.0, RMSNorm 147.1 -> 142.2, 300 x 16384 33.9 -> 31.2.
  if (!g.reg_path && es == 4 && g.vec == 4 && nvec > 2 * 1024 &&
      (nvec <= 3 * 1024 || (nvec <= 4 * 1024 && !dres && !gelu)) && tun.bwd_no_lds == 0) {
    g.reg_path = true;
    g.vpl = nvec <= 3 * 1024 ? 3 : 4;
    g.threads = 1024;
    g.wpr = 1024 / kWave;
    g.rgs = 1;
    g.blocks = rows < device_cu_count() ? rows : device_cu_count();
    g.rows_per_block = (rows + g.blocks - 1) / g.blocks;
  }
  // 16-bit LayerNorm / RMSNorm rows of 24577..32768 columns without a residual gradient, at
  // least 6 rows per CU: the raw tiles with 4 vectors per lane and no prefetched row (a block's
  // row loads are exposed, so the rows of a block must be many).  Against the two passes, bf16
  // backward calls, us: 2048 x 32768 126.4 -> 110.1, 4096 x 32768 235.1 -> 188.3, 1536 x 32768
  // 99.9 -> 91.8, RMSNorm 2048 x 28672 121.2 -> 92.2, fp16 2048 x 32768 124.5 -> 105.9; with
  // fewer rows the two passes win (1024 x 32768 71.6 against 74.0, 300 x 32768 37.2 against
  // 49.0).
  if (!g.reg_path && es == 2 && g.vec == 8 && nvec > 3 * 1024 && nvec <= 4 * 1024 && !dres &&
      !gelu && rows >= 6 * int64_t(device_cu_count()) && tun.bwd_no_lds == 0) {
    g.reg_path = true;
    g.vpl = 4;
    g.threads = 1024;
    g.wpr = 1024 / kWave;
    g.rgs = 1;
    g.blocks = rows < device_cu_count() ? rows : device_cu_count();
    g.rows_per_block = (rows + g.blocks - 1) / g.blocks;
  }
  // fp32 rows too wide for registers but within 4 vectors per thread of a 1024-thread block
  // (8193..16384 columns): the LDS-staged kernel, one block per CU, rows dealt grid-stride.
  // 16-bit rows of 8193..16384 columns with a residual gradient keep the register kernel
  // (gamma in LDS there), measured faster than 2 vectors per thread here (4096 x 16384 bf16:
  // 90.8 against 97.8 us).  fp16 rows of 16385..18432 columns with a residual gradient take it
  // with 768 threads and 3 vectors per thread (gamma parked in LDS as well), measured faster
  // than the two passes (4096 x 18432 bf16: LN 161 -> 108 us, + residual 164 -> 110 us).
  const int64_t cpt = (nvec + kLdsThreads - 1) / kLdsThreads;
  const int64_t cpt16 = (nvec + kLds16Threads - 1) / kLds16Threads;
  const bool wide_f32 = !g.reg_path && es == 4 && cpt >= 3 && cpt <= 4;
  const bool wide16 = !g.reg_path && es == 2 && !gelu && cpt16 == 3 && dres && dtype == FLN_F16;
  if (g.vec > 1 && (wide_f32 || wide16) && tun.bwd_no_lds == 0) {
    g.reg_path = false;
    g.lds_cpt = wide16 ? static_cast<int>(cpt16) : static_cast<int>(cpt);
    g.threads = wide16 ? kLds16Threads : kLdsThreads;
    g.wpr = g.threads / kWave;
    g.rgs = 1;
    g.blocks = rows < device_cu_count() ? rows : device_cu_count();
    g.rows_per_block = (rows + g.blocks - 1) / g.blocks;
  }
  // Everything else (any width) in two streaming passes, given the workspace for the row
  // statistics; without one (dx alone, no workspace passed) the looped kernel.  Block rows of
  // the column pass (each block takes every G-th row of its column tile): enough that tiles x G
  // gives 2 blocks per CU, at most the workspace's partial rows.  Fewer rows in progress keep
  // DRAM locality, and the column reduction reads fewer partial rows: bf16 backward calls, us,
  // 8 -> 2 blocks per CU: 512 x 131072 145.3 -> 134.5, 2048 x 32768 139.2 -> 124.3, 8192 x 32768
  // -> 448.4 (540.0 with contiguous row chunks), fp32 1024 x 32768 127.4 -> 116.9; one block per
  // CU was slower (178.0 / 165.4 / 625.4 / 155.9).
  // (Buffer resources span at most 4 GiB: rows of 2 GiB or more keep the looped kernel.)
  if (!g.reg_path && g.lds_cpt == 0 && have_workspace && cols * es < (int64_t(1) << 31) &&
      tun.bwd_no_two_pass == 0) {
    const int64_t tiles = (nvec + kWideThreads - 1) / kWideThreads;
    // FLN_BWD_COLPASS_PER_CU overrides the default; re-swept with few rows, 1 / 2 / 4 per CU,
    // bf16 us: 128 x 131072 42.2 / 43.0 / 53.7, 256 x 131072 71.7 / 70.5 / 80.1, 300 x 65536
    // 48.9 / 49.3 / 57.4, 1024 x 65536 129.6 / 123.8 / 129.7.
    const int64_t per_cu =
        tun.bwd_colpass_per_cu > 0 ? tun.bwd_colpass_per_cu : FLN_COLPASS_BLOCKS_PER_CU;
    int64_t chunks = (per_cu * static_cast<int64_t>(device_cu_count()) + tiles - 1) / tiles;
    if (chunks > workspace_partial_rows(rows)) chunks = workspace_partial_rows(rows);
    if (chunks < 1) chunks = 1;
    g.two_pass = true;
    g.threads = kWideThreads;
    g.rows_per_block = (rows + chunks - 1) / chunks;
    g.blocks = (rows + g.rows_per_block - 1) / g.rows_per_block;
  }
  return g;
}

int launch_backward(const BwdParams& p0, int dtype, void* dgamma, void* dbeta, int dparam_dtype,
                    bool have_workspace, size_t workspace_bytes, hipStream_t s) {
  // p0.part_g / p0.part_b carry the workspace base (validated by the caller).
  BwdParams p = p0;
  const bool vec_ok = aligned16(p.x) && aligned16(p.dy) && aligned16(p.dx) &&
                      aligned16(p.gamma) && aligned16(p.dres);
  BwdGeometry geo =
      backward_geometry(p.rows, p.cols, dtype, vec_ok, p.dres != nullptr, p.gelu != 0,
                        have_workspace);
  if (geo.reg_path) {
    // Never more blocks than fit at once: a second round of blocks would only add a tail.
    int64_t resident = geo.blocks;
    int rc = FLN_ERR_INVALID;
    switch (dtype) {
      case FLN_F32: rc = dispatch_backward<float>(p, geo, s, &resident); break;
      case FLN_BF16: rc = dispatch_backward<__bf16>(p, geo, s, &resident); break;
      case FLN_F16: rc = dispatch_backward<_Float16>(p, geo, s, &resident); break;
      default: break;
    }
    if (rc != 0) return rc;
    if (geo.blocks > resident) geo.blocks = resident;
  }
  const int64_t ld = (p.cols + 3) & ~int64_t(3);
  float* ws = p0.part_g;
  // Workspace layout: dgamma partials [blocks, ld] and dbeta partials [blocks, ld] when either
  // gradient is requested, then the row statistics of the two-pass path [rows, splits, 2]
  // (16-byte aligned: ld is a multiple of 4).  At most fln_backward_workspace_bytes() (blocks <=
  // workspace_partial_rows on every path; splits within what that bound leaves).
  const int64_t part = (dgamma || dbeta) ? 2 * geo.blocks * ld : 0;
  // Row statistics of the two-pass path: fewer rows than the statistics pass has blocks split
  // into column chunks of whole steps (kWideUnroll x kWideThreads vectors), as many as the
  // workspace bound (fln_backward_workspace_bytes, not the size passed, so that the split and
  // with it the summation order never depend on the caller's workspace) leaves after the
  // partials.
  int64_t splits = 1;
  const int64_t nvec = p.cols / geo.vec;
  p.stat_chunk = nvec;
  if (geo.two_pass) {
    constexpr int64_t step = int64_t(kWideUnroll) * kWideThreads;
    const int64_t steps = (nvec + step - 1) / step;
    const int forced = tuning().bwd_stat_splits;  // FLN_BWD_STAT_SPLITS
    const int64_t items = kRowstatItemsPerCu * static_cast<int64_t>(device_cu_count());
    splits = forced > 0 ? forced : (items + p.rows - 1) / p.rows;
    if (splits > kMaxStatSplits) splits = kMaxStatSplits;
    const int64_t bound = 2 * workspace_partial_rows(p.rows) * ld + 2 * p.rows;
    const int64_t room = (bound - part) / (2 * p.rows);
    if (splits > room) splits = room;
    if (splits > steps) splits = steps;
    if (splits < 1) splits = 1;
    p.stat_chunk = (steps + splits - 1) / splits * step;
    splits = (nvec + p.stat_chunk - 1) / p.stat_chunk;
  }
  p.stat_splits = static_cast<int>(splits);
  if (have_workspace) {
    const size_t need = (static_cast<size_t>(part) +
                         (geo.two_pass ? 2 * static_cast<size_t>(p.rows * splits) : 0)) *
                        sizeof(float);
    if (need > workspace_bytes) return FLN_ERR_TOO_LARGE;
  }
  p.part_g = dgamma ? ws : nullptr;
  p.part_b = dbeta ? ws + geo.blocks * ld : nullptr;
  p.rowstat = have_workspace ? ws + part : nullptr;
  // The column pass with a single block row (columns >= 2 x CUs column tiles) holds the final
  // column sums: it writes dgamma / dbeta itself and the column reduction is skipped (the same
  // bits: the reduction of one partial row only converts it; 64 x 1048576 bf16: 6.4 us).
  const bool direct = geo.two_pass && geo.blocks == 1;
  if (direct) {
    p.out_g = dgamma;
    p.out_b = dbeta;
    p.out_dtype = dparam_dtype;
    p.part_g = p.part_b = nullptr;
  }
  ColReduceArgs a{};
  if (dgamma) { a.part[a.ny] = p.part_g; a.out[a.ny] = dgamma; ++a.ny; }
  if (dbeta) { a.part[a.ny] = p.part_b; a.out[a.ny] = dbeta; ++a.ny; }
  a.G = geo.blocks;
  a.N = p.cols;
  a.out_dtype = dparam_dtype;
  if (a.ny > 0 && dparam_dtype != FLN_F32 && dparam_dtype != FLN_BF16 &&
      dparam_dtype != FLN_F16)
    return FLN_ERR_INVALID;
  int rc;
  switch (dtype) {
    case FLN_F32: rc = dispatch_backward<float>(p, geo, s); break;
    case FLN_BF16: rc = dispatch_backward<__bf16>(p, geo, s); break;
    case FLN_F16: rc = dispatch_backward<_Float16>(p, geo, s); break;
    default: return FLN_ERR_INVALID;
  }
  if (rc != 0 || a.ny == 0 || direct) return rc;
  if (a.G <= kCrFlatMaxG)
    hipLaunchKernelGGL(col_reduce_flat_kernel, dim3(static_cast<unsigned>(flat_blocks(a))),
                       dim3(kCrFlatThreads), 0, s, a);
  else {
    static std::atomic<void*> fn_cache[64];
    return launch_cached(col_reduce_kernel, fn_cache, dim3(static_cast<unsigned>(quad_blocks(a))),
                         dim3(kCrThreads), s, a);
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace fln

namespace {

// Zeroes the parameter gradients of an empty batch (byte stores: at most 4 x cols bytes, any
// alignment).  A kernel rather than hipMemsetAsync, so that a call captured into a HIP graph
// records a kernel node and no memset node.
__global__ __launch_bounds__(256) void zero_fill_kernel(uint8_t* a, uint8_t* b, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    if (a) a[i] = 0;
    if (b) b[i] = 0;
  }
}

// scratch: the workspace is the device's no-allocation scratch (its size checked against what
// the call's geometry needs, not against the fln_backward_workspace_bytes bound).
int backward_common(fln::BwdParams p, int dtype, void* dgamma, void* dbeta, int dparam_dtype,
                    void* workspace, size_t workspace_bytes, void* stream, bool scratch = false) {
  if (p.rows < 0 || p.cols < 0 || p.rows > INT32_MAX || p.cols > INT32_MAX) return FLN_ERR_INVALID;
  if (dtype != FLN_F32 && dtype != FLN_BF16 && dtype != FLN_F16) return FLN_ERR_INVALID;
  if ((dgamma || dbeta) && dparam_dtype != FLN_F32 && dparam_dtype != dtype) return FLN_ERR_INVALID;
  if (p.rows == 0 || p.cols == 0) {
    // Nothing to reduce: parameter gradients of an empty batch are zero.
    if (p.cols > 0 && (dgamma || dbeta)) {
      const int64_t n = p.cols * fln::element_size(dparam_dtype);
      const int64_t blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
      hipLaunchKernelGGL(zero_fill_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                         static_cast<hipStream_t>(stream), static_cast<uint8_t*>(dgamma),
                         static_cast<uint8_t*>(dbeta), n);
      return static_cast<int>(hipGetLastError());
    }
    return FLN_OK;
  }
  if (!p.dy || !p.x || !p.rstd || (!p.rms && !p.mean)) return FLN_ERR_INVALID;
  if (!p.dx && !dgamma && !dbeta) return FLN_OK;
  const bool have_workspace =
      workspace && fln::aligned16(workspace) &&
      (scratch || workspace_bytes >= fln_backward_workspace_bytes(p.rows, p.cols, dtype));
  if ((dgamma || dbeta) && !have_workspace) return FLN_ERR_INVALID;
  p.part_g = have_workspace ? static_cast<float*>(workspace) : nullptr;
  const fln::CallDevice device_scope;
  return fln::launch_backward(p, dtype, dgamma, dbeta, dparam_dtype, have_workspace,
                              workspace_bytes, static_cast<hipStream_t>(stream));
}

}  // namespace

// Scratch of fln_layernorm_backward_noalloc: the workspace (column partials, row statistics) of
// one call, for callers that cannot allocate.  Every device that runs that entry point holds its
// own copy until the process ends.  Host code never names the array itself (on the host it is
// only a stand-in for the symbol): it uses the device address hipGetSymbolAddress returns, once
// per device, with that device current.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

std::atomic<void*> g_scratch_ptr[64];
std::mutex g_scratch_mu;

// Device address of `scratch` on device `dev` (the current device), or nullptr.
void* scratch_on_device(int dev) {
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr) return ptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  }
  return ptr;
}

}  // namespace

extern "C" size_t fln_backward_workspace_bytes(int64_t rows, int64_t cols, int dtype) {
  (void)dtype;
  if (rows <= 0 || cols <= 0) return 0;
  // Two fp32 partial arrays of up to workspace_partial_rows rows, then the row statistics
  // (2 floats per row) of the two-pass path.
  const int64_t g = fln::workspace_partial_rows(rows);
  const int64_t ld = (cols + 3) & ~int64_t(3);
  return static_cast<size_t>(2 * g * ld + 2 * rows) * sizeof(float);
}

extern "C" int fln_layernorm_backward(const void* dy, const void* x, const float* mean,
                                      const float* rstd, const void* gamma, const void* dres,
                                      void* dx, void* dgamma, void* dbeta, int64_t rows,
                                      int64_t cols, int dtype, int dparam_dtype, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  fln::BwdParams p{};
  p.dy = dy; p.x = x; p.mean = mean; p.rstd = rstd; p.gamma = gamma; p.dres = dres; p.dx = dx;
  p.rows = rows; p.cols = cols; p.rms = 0;
  return backward_common(p, dtype, dgamma, dbeta, dparam_dtype, workspace, workspace_bytes,
                         stream);
}

extern "C" int fln_layernorm_backward_noalloc(const void* dy, const void* x, const float* mean,
                                              const float* rstd, const void* gamma,
                                              const void* dres, void* dx, void* dgamma,
                                              void* dbeta, int64_t rows, int64_t cols, int dtype,
                                              int dparam_dtype, void* stream) {
  // The scratch is per device: the stream must belong to the current device.
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return FLN_ERR_INVALID;
  if (stream) {
    int sdev = -1;
    if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess || sdev != dev)
      return FLN_ERR_INVALID;
  }
  void* ws = scratch_on_device(dev);
  if (!ws) return FLN_ERR_INVALID;
  fln::BwdParams p{};
  p.dy = dy; p.x = x; p.mean = mean; p.rstd = rstd; p.gamma = gamma; p.dres = dres; p.dx = dx;
  p.rows = rows; p.cols = cols; p.rms = 0;
  return backward_common(p, dtype, dgamma, dbeta, dparam_dtype, ws, kScratchBytes, stream,
                         /*scratch=*/true);
}

extern "C" int fln_layernorm_gelu_backward(const void* dy, const void* x, const float* mean,
                                           const float* rstd, const void* gamma,
                                           const void* beta, void* dx, void* dgamma,
                                           void* dbeta, int64_t rows, int64_t cols, int dtype,
                                           int dparam_dtype, int gelu_mode, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  if (gelu_mode != FLN_GELU_ERF && gelu_mode != FLN_GELU_TANH) return FLN_ERR_INVALID;
  fln::BwdParams p{};
  p.dy = dy; p.x = x; p.mean = mean; p.rstd = rstd; p.gamma = gamma; p.beta = beta; p.dx = dx;
  p.rows = rows; p.cols = cols; p.rms = 0; p.gelu = gelu_mode;
  return backward_common(p, dtype, dgamma, dbeta, dparam_dtype, workspace, workspace_bytes,
                         stream);
}

extern "C" int fln_rmsnorm_backward(const void* dy, const void* x, const float* rstd,
                                    const void* weight, const void* dres, void* dx, void* dweight,
                                    int64_t rows, int64_t cols, int dtype, int dweight_dtype,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  fln::BwdParams p{};
  p.dy = dy; p.x = x; p.rstd = rstd; p.gamma = weight; p.dres = dres; p.dx = dx;
  p.rows = rows; p.cols = cols; p.rms = 1;
  return backward_common(p, dtype, dweight, nullptr, dweight_dtype, workspace, workspace_bytes,
                         stream);
}
