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
// The barrier only waits for LDS traffic (lgkmcnt), so global loads issued before it (the next
// row's prefetch) stay in flight across it.
template <class Op>
__device__ __forceinline__ float row_allreduce(float v, float* slot, int wpr, int rg, int wave,
                                               int lane) {
  v = wave_allreduce<Op>(v);
  if (wpr == 1) return v;
  if (lane == 0) slot[wave] = v;
  __syncthreads();
  return combine_partials<Op>(slot, rg * wpr, wpr, lane, 0.0f);  // 0: identity of + and max|.|
}

// ---------------------------------------------------------------------------------------------
// Register-resident forward, persistent over rows.
//
// Block = rows_per_block row groups of `wpr` waves; thread t of a row group owns vectors
// t, t + 64*wpr, ... (VPL of them), so consecutive lanes read consecutive 16-byte vectors and
// every wave-wide access is one coalesced 1 KiB transaction.  The grid holds as many blocks as
// fit on the device at once; each row group walks rows rb*rows_per_block + rg for
// rb = blockIdx.x, blockIdx.x + gridDim.x, ...
//
// Software pipeline, per row group and step (rows i+1 .. i+PD-1 and then i+PD in flight as raw
// packed loads while row i is worked on):
//   1. wait for row i (its ring slot), widen it into registers;
//   2. issue the loads of row i+PD into the freed slot;
//   3. statistics and normalization of row i, outputs packed to the output format;
//   4. issue the stores of row i.
// Loads and stores share one counter (vmcnt) on gfx9-family GPUs, which completes in issue
// order: the wait in step 1 is exact only if every path into it has the same operations
// outstanding, hence whole rounds of PD steps (no early exit) and a prologue padded with dropped
// stores, and scheduling barriers that keep each step's loads and stores in step order.
// All global traffic goes through per-row buffer resources (tails and rows past the end are
// handled by the hardware range check), so the loop body has no divergent branches.
// LDS reduction slots are double-buffered by iteration parity: every iteration of a multi-wave
// row group passes at least one barrier, which separates a slot's reads from its next writes.
// EXACT: the row is exactly VPL vectors per lane (no masking in the statistics); GELU: 0 none,
// 1 erf, 2 tanh (a template parameter so the plain kernels carry no GELU code).
// ---------------------------------------------------------------------------------------------
// Rows in flight ahead of the current one: about 64 bytes of loads per lane.  A lane holding 64
// bytes or more of a row prefetches one row, a smaller slice two (measured with exact ring
// waits, bf16, us: 8192 x 4096 LN 24.9 -> 24.0 and LN + GELU(erf) 31.4 -> 30.0 with one row of
// 64 bytes ahead instead of two; LN -> fp8 32768 x 7168, 32 bytes per lane, 146 with one row
// against 141 with two; three rows ahead were slower everywhere).
// Register budget: a 1024-thread block leaves 128 VGPRs per lane.  There a lane with more than
// 32 bytes of a row prefetches one row (two again for the 16-bit RAW tiles without a residual,
// whose gamma / beta live in LDS), and a lane with 32 elements (RAW) keeps the row in the I/O
// type rather than as an fp32 copy, widening it again in each pass (one VALU op per element).
// Blocks of at most 256 threads have 256 VGPRs and keep the fp32 copy.
#ifndef FLN_FWD_PREFETCH
#define FLN_FWD_PREFETCH(ROW_BYTES, MAXT) \
  (((ROW_BYTES) >= 64 || ((MAXT) > 256 && (ROW_BYTES) > 32)) ? 1 : 2)
#endif
// Cache policies of the streamed rows: loads of x / residual and stores of y / h / q are
// non-temporal (each byte is touched once; measured on MI355X this is 3-10% faster than the
// default policy for every forward flavour, because the streams no longer evict each other's
// lines or the parameters).  The parameters and per-row statistics keep the default policy.
#ifndef FLN_FWD_LOAD_POL
#define FLN_FWD_LOAD_POL kStream
#endif
#ifndef FLN_FWD_STORE_POL
#define FLN_FWD_STORE_POL kStream
#endif
// Rows of raw loads in flight ahead of the current one, per instantiation (the rule above; the
// 16-bit RAW tiles without a residual keep two: their gamma / beta live in LDS; so do the odd
// tiles of LayerNorm / RMSNorm with 5 or 7 vectors per lane, which have the registers for it
// (178-248 VGPRs).  bf16, us, one row ahead -> two: 65536 x 3584 (1 x 7) 160.3 -> 157.3, 16384
// x 5120 (2 x 5) 58.3 -> 56.2, 32768 x 2560 (1 x 5) 55.9 / 55.9.  The fp8 row scale keeps one:
// two gained on one-wave rows (65536 x 3072, 1 x 6: 105.5 -> 97.2; 32768 x 2560, 1 x 5: 44.7 ->
// 41.4) and lost on two-wave rows with the same tile (16384 x 6144, 2 x 6: 53.1 -> 57.0; 16384
// x 5120, 2 x 5: 44.4 -> 51.6; C5, 2 x 7: 121.1 / 121.5), and the depth is fixed per tile.
// Two rows ahead on the 4-vector tiles lost or tied in every flavour (LN 8192 x 4096, 2 x 4:
// 23.9 -> 24.6; 65536 x 2048, 1 x 4: 86.4 -> 87.5; C4's RMSNorm, 4 x 4: 86.8 / 86.8; residual +
// LN 16384 x 8192: 181.8 -> 185.0; LN -> fp8 16384 x 4096: 35.6 -> 47.4) and tied on the
// 3-vector LayerNorm tiles (1536-6144 columns).
template <class T, int FP8, bool RES, int GELU, int VEC, int VPL, int MAXT>
constexpr int fwd_prefetch_depth() {
  constexpr bool raw = MAXT > 256 && VPL * VEC >= 32;
  constexpr bool params_in_lds =
      MAXT == 1024 && ((raw && VEC > 1 && sizeof(T) == 2) || (VEC == 1 && VPL == 16 &&
                                                               sizeof(T) <= 4));
  constexpr bool odd_two =
      VEC == 8 && MAXT == 256 && !RES && GELU == 0 && FP8 == 0 && (VPL == 5 || VPL == 7);
  return (params_in_lds && raw && !RES) || odd_two
             ? 2
             : FLN_FWD_PREFETCH(VPL * VEC * static_cast<int>(sizeof(T)), MAXT);
}

template <class T, int FP8, bool RES, int GELU, int VEC, int VPL, bool EXACT, int MAXT>
__global__ __launch_bounds__(MAXT) void fwd_reg_kernel(const FwdParams p, int64_t row_blocks) {
  constexpr bool RAW = MAXT > 256 && VPL * VEC >= 32;  // row kept in the I/O type
  // gamma / beta parked in LDS, each thread its own copy (no barrier; 64-128 KiB), for the 16-bit
  // RAW tiles and the scalar path's 16 elements per lane in 1024-thread blocks: in registers
  // they made the residual / fp8 flavours spill 16-332 B per lane, and they left room for only
  // one row in flight elsewhere (bf16, us: residual + LN 2048 x 32768 102.7 -> 89.6, residual +
  // RMSNorm -> fp8 111.9 -> 82.3; with two rows in flight LN 2048 x 32768 52.8 -> 48.8, RMSNorm
  // 4096 x 20480 62.6 -> 57.9, LN -> fp8 4096 x 20480 73.5 -> 67.1).
  constexpr bool PARAMS_IN_LDS =
      MAXT == 1024 && ((RAW && VEC > 1 && sizeof(T) == 2) || (VEC == 1 && VPL == 16 &&
                                                                sizeof(T) <= 4));
  // rows in flight ahead of the current one (the residual flavour's second input leaves room for
  // one only)
  constexpr int PD = fwd_prefetch_depth<T, FP8, RES, GELU, VEC, VPL, MAXT>();
  static_assert(PD == 1 || PD == 2, "the ring holds one or two rows ahead");
  constexpr int MAXW = MAXT / kWave;
  __shared__ float red[2][3][MAXW + 16];  // padded: combine_partials reads 16 past the base
  using P = Pack<T, VEC>;
  // fp8 output: VEC codes per vector, held as one 4- or 8-byte word.
  using QW = typename BufIO<(VEC >= 4 ? VEC : 4)>::W;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wpr = p.wpr;
  const int rg = wave / wpr;
  const int t = (wave - rg * wpr) * kWave + lane;
  const int tpr = kWave * wpr;
  const int rows_per_block = blockDim.x / tpr;
  const int64_t N = p.cols;
  const int nvec = static_cast<int>(N / VEC);
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  // mean = sum / N as sum * (1/N) plus one FMA correction step, which returns the exact quotient
  // whenever it is representable (an exactly summed constant row then maps to beta exactly)
  // without the long correctly-rounded division sequence.
  const float fn = static_cast<float>(N);
  const float inv_n = 1.0f / fn;
  const T* X = static_cast<const T*>(p.x);
  const T* R = static_cast<const T*>(p.res);
  const int64_t stride = gridDim.x;

  // Affine parameters, once per row group (vectors past the row read as zero).
  const rsrc_t g_rs = make_rsrc(p.gamma, row_bytes);
  const rsrc_t b_rs = make_rsrc(p.beta, row_bytes);
  __shared__ P gsh[PARAMS_IN_LDS ? VPL * MAXT : 1], bsh[PARAMS_IN_LDS ? VPL * MAXT : 1];
  P gv[PARAMS_IN_LDS ? 1 : VPL], bv[PARAMS_IN_LDS ? 1 : VPL];
  if constexpr (PARAMS_IN_LDS) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      P g0 = buf_load<P>(g_rs, t + i * tpr);
      if (p.gamma == nullptr) {  // absent gamma multiplies by one (uniform)
#pragma unroll
        for (int e = 0; e < VEC; ++e) g0.v[e] = static_cast<T>(1.0f);
      }
      gsh[i * MAXT + threadIdx.x] = g0;
      bsh[i * MAXT + threadIdx.x] = buf_load<P>(b_rs, t + i * tpr);
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {  // unconditional: an absent tensor has a zero-byte resource
      gv[i] = buf_load<P>(g_rs, t + i * tpr);
      bv[i] = buf_load<P>(b_rs, t + i * tpr);  // absent beta reads as zeros: adds nothing
    }
    if (p.gamma == nullptr) {  // absent gamma multiplies by one (uniform, once per kernel)
#pragma unroll
      for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) gv[i].v[e] = static_cast<T>(1.0f);
    }
  }
  // Vector slot i is complete (no lane past the row) when (i + 1) * tpr <= nvec; only the
  // other slots need per-element masks in the centred sums and the fp8 row max.
  auto slot_full = [&](int i) { return EXACT || (i + 1) * tpr <= nvec; };
  // Elements of the row held by wave w of a row group (w < wpr), and this wave's reciprocal.
  auto wave_elems = [&](int w) -> float {
    int n = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int left = nvec - (i * tpr + w * kWave);
      n += left <= 0 ? 0 : (left < kWave ? left : kWave);
    }
    return static_cast<float>(n * VEC);
  };
  const float own_n = wave_elems(wave - rg * wpr);
  const float inv_wave_n = own_n > 0.0f ? 1.0f / own_n : 0.0f;

  auto row_of = [&](int64_t rb) { return rb * rows_per_block + rg; };
  auto bytes_of = [&](int64_t rb) -> uint32_t {
    return (rb < row_blocks && row_of(rb) < p.rows) ? row_bytes : 0u;
  };

  // Ring of raw loads: the PD rows after the current one are in flight.
  P xv[PD][VPL], rv[PD][VPL];
  auto load_row = [&](int64_t rb, int slot) {
    const int64_t row = row_of(rb);
    const uint32_t nb = bytes_of(rb);
    const rsrc_t xr = make_rsrc(X + row * N, nb);
#pragma unroll
    for (int i = 0; i < VPL; ++i) xv[slot][i] = buf_load<P, FLN_FWD_LOAD_POL>(xr, t + i * tpr);
    if constexpr (RES) {
      const rsrc_t rr = make_rsrc(R + row * N, nb);
#pragma unroll
      for (int i = 0; i < VPL; ++i) rv[slot][i] = buf_load<P, FLN_FWD_LOAD_POL>(rr, t + i * tpr);
    }
  };

  float xf[RAW ? 1 : VPL][VEC];  // the row being normalized, fp32 (then its outputs)
  P hv[VPL];  // residual sum of that row (RES), or the row itself (RAW), in the I/O type
  auto widen = [&](int slot) {
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        if constexpr (RES)
          hv[i].v[e] = from_f32<T>(to_f32(xv[slot][i].v[e]) + to_f32(rv[slot][i].v[e]));
        else if constexpr (RAW)
          hv[i].v[e] = xv[slot][i].v[e];
        if constexpr (!RAW) xf[i][e] = to_f32(RES ? hv[i].v[e] : xv[slot][i].v[e]);
      }
  };
  // Element e of vector slot i of the row, fp32.
  auto xin = [&](int i, int e) -> float {
    if constexpr (RAW)
      return to_f32(hv[i].v[e]);
    else
      return xf[i][e];
  };

  // Row k of this row group is rb0 + k * stride; slot k % PD holds its raw loads from step
  // k - PD on.  Prologue: the first PD rows in slot order, each followed by as many stores as a
  // loop step issues (zero-byte resource: dropped), so that the loop top sees the same sequence
  // of outstanding memory operations from here as from the previous step and the compiler's wait
  // there covers only the slot being consumed.  (Without the padding the merged wait also
  // drains the other slots.)
  const int64_t rb0 = blockIdx.x;
  constexpr int kStoresPerRow =
      2 + (RES ? VPL : 0) + (FP8 == 0 ? VPL : (FP8 == 2 ? 2 * VPL : VPL + 1));
  const rsrc_t none = make_rsrc(nullptr, 0);
  // Exact GELU: every thread loads one entry of the GELU table (4 KiB, L2-resident after the
  // first block), ahead of the rows; the LDS copy is written once they are in flight.
  __shared__ float4 gelu_tab[GELU == 1 ? kGeluLogTabN : 1];
  float4 tab_entry;
  if constexpr (GELU == 1) {
    tab_entry = reinterpret_cast<const float4*>(kGeluLogTabData)[threadIdx.x % kGeluLogTabN];
    asm volatile("" ::: "memory");
  }
#pragma unroll
  for (int k = 0; k < PD; ++k) {
    load_row(rb0 + k * stride, k);
#pragma unroll
    for (int j = 0; j < kStoresPerRow; ++j)  // distinct, non-adjacent: none merged away
      BufIO<4>::store(0u, none, 64u * j);
    asm volatile("" ::: "memory");  // keeps the slots in issue order
  }
  if constexpr (GELU == 1) {  // waits for the table's load alone (it was issued first)
    if (threadIdx.x < kGeluLogTabN) gelu_tab[threadIdx.x] = tab_entry;
    __syncthreads();
  }
  // Whole rounds of PD rows (the inner loop is unrolled so every slot index is static): a step
  // past the block's last row reads zeros and stores nothing.  An early exit from the unrolled
  // round would make the compiler wait for every slot at the loop top.
  const int64_t my_rows = rb0 < row_blocks ? (row_blocks - 1 - rb0) / stride + 1 : 0;
  const int64_t rounds = (my_rows + PD - 1) / PD;
  int parity = 0;
  for (int64_t r = 0; r < rounds; ++r) {
#pragma unroll
  for (int s = 0; s < PD; ++s) {
    const int64_t rb = rb0 + (r * PD + s) * stride;
    parity ^= 1;
    const int64_t row = row_of(rb);
    const uint32_t nb = bytes_of(rb);
    float(*slots)[MAXW + 16] = red[parity];
    // Consume slot s (this row) and put the row PD steps ahead in flight in its place.
    widen(s);
    load_row(rb + PD * stride, s);
    if constexpr (MAXT > 256 && !PARAMS_IN_LDS) {  // 128 VGPRs: widen per row, not once
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        keep_packed(gv[i]);
        keep_packed(bv[i]);
      }
    }

    // 1. Statistics over registers: the mean, then the sum of squares centred on it (two
    //    passes over the row, no E[x^2] - mean^2 cancellation).  Vectors past the row were
    //    loaded as zeros, so they drop out of the plain sum.
    auto centred = [&](float c) {  // sum over this lane's elements of (x - c)^2
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        if (slot_full(i)) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float d = xin(i, e) - c;
            acc = fmaf(d, d, acc);
          }
        } else {
          const bool ok = (t + i * tpr) < nvec;
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float d = xin(i, e) - c;
            acc += ok ? d * d : 0.0f;
          }
        }
      }
      return acc;
    };
    float mean = 0.0f, q = 0.0f;
    if (p.rms) {
      q = row_allreduce<SumOp>(centred(0.0f), slots[1], wpr, rg, wave, lane);
    } else {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) s += xin(i, e);
      const float sw = wave_allreduce<SumOp>(s);
      if (wpr == 1) {
        mean = sw * inv_n;
        mean = fmaf(fmaf(-mean, fn, sw), inv_n, mean);
        q = wave_allreduce<SumOp>(centred(mean));
      } else {
        // A row over several waves takes ONE barrier for both statistics: each wave centres its
        // own elements on its own mean c_w = S_w / n_w (wave-uniform, known without the other
        // waves), then the row combines the waves' (S_w, Q_w): mean = sum_w S_w / N (the same
        // fixed-order sum as a plain two-pass mean, bit for bit) and, by the parallel-variance
        // identity, sum (x - mean)^2 = sum_w [Q_w + n_w (c_w - mean)^2 + 2 (c_w - mean) r_w],
        // r_w = S_w - n_w c_w the rounding residue of c_w.
        const float cw = sw * inv_wave_n;
        const float qw = wave_allreduce<SumOp>(centred(cw));
        if (lane == 0) {
          slots[0][wave] = sw;
          slots[1][wave] = qw;
        }
        __syncthreads();
        const int k = lane & 15;  // lane k of every wave reads wave k's pair of this row group
        const bool in = k < wpr;
        const float sk = in ? slots[0][rg * wpr + k] : 0.0f;
        const float qk = in ? slots[1][rg * wpr + k] : 0.0f;
        const float sum = reduce16<SumOp>(sk);
        mean = sum * inv_n;
        mean = fmaf(fmaf(-mean, fn, sum), inv_n, mean);
        const float nk = wave_elems(k);
        const float ck = sk * (nk > 0.0f ? 1.0f / nk : 0.0f);  // == that wave's c_w
        const float dk = ck - mean;
        const float term = in ? qk + dk * fmaf(nk, dk, 2.0f * fmaf(-nk, ck, sk)) : 0.0f;
        q = reduce16<SumOp>(term);
      }
    }
    const float rstd = __builtin_amdgcn_rsqf(q * inv_n + p.eps);  // v_rsq_f32, 1 ulp
    const float poison = FP8 != 0 ? row_poison(mean, rstd) : 0.0f;  // fp8 scales: NaN

    //    Normalize + affine + epilogue, packed to the output format.
    auto affine = [&](int i, int e) -> float {
      float a;
      if constexpr (PARAMS_IN_LDS)
        a = fmaf((xin(i, e) - mean) * rstd, to_f32(gsh[i * MAXT + threadIdx.x].v[e]),
                 to_f32(bsh[i * MAXT + threadIdx.x].v[e]));
      else
        a = fmaf((xin(i, e) - mean) * rstd, to_f32(gv[i].v[e]), to_f32(bv[i].v[e]));
      if constexpr (GELU == 1) a = gelu_erf_tab(gelu_tab, a);
      if constexpr (GELU == 2) a = gelu_tanh(a);
      return a;
    };
    if constexpr (!RAW) {
#pragma unroll
      for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) xf[i][e] = affine(i, e);
    }
    // Output element e of vector slot i (RAW: recomputed at each use).
    auto out = [&](int i, int e) -> float {
      if constexpr (RAW)
        return affine(i, e);
      else
        return xf[i][e];
    };
    P yo[VPL];
    QW qo[VPL];
    P ho[VPL];
    int mxc[FP8 == 2 ? VPL : 1];  // E8M0 codes of the lane's blocks (MX)
    float scale = 0.0f;
    if constexpr (FP8 == 0) {
#pragma unroll
      for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) yo[i].v[e] = from_f32<T>(out(i, e));
    } else if constexpr (FP8 == 2) {
      // OCP MX: each 32-element block is G adjacent lanes' vectors; its maximum needs only
      // DPP steps within the group (blocks never straddle the row end: cols % 32 == 0).
      constexpr int G = 32 / VEC;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float bm = 0.0f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) bm = fmaxf(bm, fabsf(out(i, e)));
        const MxScale ms = mx_scale_e4m3(group_max<G>(bm), mx_poison(poison));
        float a[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) a[e] = out(i, e);
        const float m = ms.mul;  // |a * m| < 512: the saturating conversion clamps to 448
        if constexpr (VEC == 8) {
          qo[i].x = fp8x4(a[0] * m, a[1] * m, a[2] * m, a[3] * m);
          qo[i].y = fp8x4(a[4] * m, a[5] * m, a[6] * m, a[7] * m);
        } else if constexpr (VEC == 4) {
          qo[i] = fp8x4(a[0] * m, a[1] * m, a[2] * m, a[3] * m);
        } else {
          qo[i] = fp8x1(a[0] * m);
        }
        mxc[i] = ms.code;
      }
    } else {
      float am = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        if (slot_full(i)) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) am = fmaxf(am, fabsf(out(i, e)));
        } else {
          const bool ok = (t + i * tpr) < nvec;
#pragma unroll
          for (int e = 0; e < VEC; ++e) am = fmaxf(am, ok ? fabsf(out(i, e)) : 0.0f);
        }
      }
      am = row_allreduce<MaxOp>(am, slots[2], wpr, rg, wave, lane);
      am += poison;
      const float inv = am > 0.0f ? 448.0f * __builtin_amdgcn_rcpf(am) : 0.0f;  // 1 ulp
      scale = am * (1.0f / 448.0f);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float a[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) a[e] = out(i, e);
        // |a * inv| <= 448 (1 + 2^-22) < 464 (1-ulp reciprocal, two roundings): in range for the
        // unclamped conversion.
        if constexpr (VEC == 8) {
          qo[i].x = fp8x4_inrange(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
          qo[i].y = fp8x4_inrange(a[4] * inv, a[5] * inv, a[6] * inv, a[7] * inv);
        } else if constexpr (VEC == 4) {
          qo[i] = fp8x4_inrange(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv);
        } else {
          qo[i] = fp8x1(a[0] * inv);
        }
      }
    }
    if constexpr (RES) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) ho[i] = hv[i];
    }

    // Stores of this row (rows past the end have a zero-byte resource: dropped).
    const uint32_t stat_off = t == 0 ? 0u : kOutOfRange;
    const uint32_t stat_nb = nb ? 4u : 0u;
    buf_store_f32(mean, make_rsrc(p.mean ? p.mean + row : nullptr, stat_nb), stat_off);
    buf_store_f32(rstd, make_rsrc(p.rstd ? p.rstd + row : nullptr, stat_nb), stat_off);
    if constexpr (RES) {
      const rsrc_t hr = make_rsrc(p.h ? static_cast<T*>(p.h) + row * N : nullptr, nb);
#pragma unroll
      for (int i = 0; i < VPL; ++i) buf_store<P, FLN_FWD_STORE_POL>(ho[i], hr, t + i * tpr);
    }
    if constexpr (FP8 == 0) {
      const rsrc_t yr = make_rsrc(static_cast<T*>(p.y) + row * N, nb);
#pragma unroll
      for (int i = 0; i < VPL; ++i) buf_store<P, FLN_FWD_STORE_POL>(yo[i], yr, t + i * tpr);
    } else {
      if constexpr (FP8 == 2) {
        // One E8M0 byte per block, stored by the block's first lane.
        constexpr int G = 32 / VEC;
        const uint32_t nblk = static_cast<uint32_t>(N / 32);
        const rsrc_t br = make_rsrc(p.bscale + row * nblk, nb ? nblk : 0u);
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          const uint32_t v = static_cast<uint32_t>(t + i * tpr);
          __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(mxc[i]), br,
                                               v % G == 0 ? v / G : kOutOfRange, 0, 0);
        }
      } else {
        buf_store_f32(scale, make_rsrc(p.scale + row, stat_nb), stat_off);
      }
      const rsrc_t qr = make_rsrc(static_cast<uint8_t*>(p.y) + row * N,
                                  nb ? static_cast<uint32_t>(N) : 0u);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        if constexpr (VEC >= 4)
          BufIO<VEC, FLN_FWD_STORE_POL>::store(qo[i], qr,
                                               (t + i * tpr) * static_cast<uint32_t>(VEC));
        else
          __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(qo[i]), qr, t + i * tpr,
                                               0, FLN_FWD_STORE_POL);
      }
    }
    // The next step's widening must not be hoisted above this step's loads and stores.
    __builtin_amdgcn_sched_barrier(0);
  }
  }
}

// ---------------------------------------------------------------------------------------------
// Rows past the register tiles on the vector path (16-bit rows of 32769..65536 columns, fp32 rows
// of 16385..32768): one 1024-thread block per row at a time, rows grid-stride, thread t owning
// vectors t + 1024 i (i < CPT) of every row.  The next row's raw loads are in flight in
// registers while the current row is worked on; the row itself (the rounded residual sum with
// RES) is parked in LDS, each thread in its own slots, so reading it back needs no barrier.
// The mean, the centred sum of squares, the fp8 row maximum and the outputs are then passes
// over LDS: x (and the residual) come from HBM once; gamma / beta are re-read per row (L2).
// ---------------------------------------------------------------------------------------------
constexpr int kFwdLdsThreads = 1024;
constexpr int kFwdLdsCpt = 8;  // vectors per thread: 128 KiB of LDS

// CR > 0 (no residual, no fp8 output): rows of up to (8 + CR) vectors per thread, the first
// 8 parked in LDS and the other CR kept in registers (cur).  The next row's LDS half is in
// flight from the start of a row; its register half is loaded into cur once the outputs of the
// current row's register half are written, in flight during the outputs of the LDS half.  (The
// whole next row in flight as well spilled 205 VGPRs.)
template <class T, int FP8, bool RES, int GELU, int VEC, int CR = 0>
__global__ __launch_bounds__(kFwdLdsThreads) void fwd_lds_kernel(const FwdParams p) {
  static_assert(CR == 0 || (FP8 == 0 && !RES), "register-extended rows: no residual or fp8");
  constexpr int kT = kFwdLdsThreads;
  constexpr int CL = kFwdLdsCpt;  // vectors parked in LDS
  constexpr int CPT = CL + CR;    // vectors per thread in all
  constexpr int kW = kT / kWave;
  using P = Pack<T, VEC>;
  using QW = typename BufIO<VEC>::W;  // VEC fp8 codes (VEC is 4 or 8 here)
  __shared__ P xs[CL * kT];
  __shared__ float red[2][3][kW + 16];  // [parity][sum, centred sum of squares, max][wave]
  // Exact GELU of 16-bit rows: the log2 Phi table (4 KiB), one entry per thread, as in the
  // register kernel; fp32 rows keep the polynomial (their kernels are not VALU-bound, and the
  // table reads slowed them: 1024 x 24576 41.2 -> 43.0 us).
  constexpr bool TAB = GELU == 1 && sizeof(T) == 2;
  __shared__ float4 gelu_tab[TAB ? kGeluLogTabN : 1];
  if constexpr (TAB) {
    if (threadIdx.x < kGeluLogTabN)
      gelu_tab[threadIdx.x] = reinterpret_cast<const float4*>(kGeluLogTabData)[threadIdx.x];
    __syncthreads();
  }
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int64_t N = p.cols;
  const int nvec = static_cast<int>(N / VEC);
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  const float fn = static_cast<float>(N);
  const float inv_n = 1.0f / fn;
  const int64_t stride = gridDim.x;
  const int iters = static_cast<int>((p.rows - 1 - blockIdx.x) / stride + 1);  // grid <= rows
  const int cpt = (nvec + kT - 1) / kT;  // vector slots the row needs (uniform; <= CPT)
  const T* X = static_cast<const T*>(p.x);
  const T* R = static_cast<const T*>(p.res);
  const rsrc_t g_rs = make_rsrc(p.gamma, row_bytes);
  const rsrc_t b_rs = make_rsrc(p.beta, row_bytes);  // absent beta reads as zeros
  const bool has_g = p.gamma != nullptr;

  constexpr int CX = CR > 0 ? CL : CPT;  // vectors of the next row loaded by load_row
  P xr[CX], rr[RES ? CPT : 1];
  P cur[CR > 0 ? CR : 1];  // vectors CL.. of the current row (CR > 0)
  // Vector i of the current row, parked (i < CL) or in registers; a register vector is made
  // opaque per use, so that each pass widens it again instead of the compiler keeping fp32
  // copies of the whole register half alive across the passes.
  auto row_vec = [&](int i) -> P {
    if constexpr (CR > 0) {
      if (i >= CL) {
        P v = cur[i - CL];
        keep_packed(v);
        return v;
      }
    }
    return xs[i * kT + threadIdx.x];
  };
  auto load_row = [&](int it) {  // rows past the block's range read as zeros
    const int64_t row = static_cast<int64_t>(it) * stride + blockIdx.x;
    const uint32_t nb = it < iters ? row_bytes : 0u;
    const rsrc_t xq = make_rsrc(X + row * N, nb);
#pragma unroll
    for (int i = 0; i < CX; ++i)
      if (i < cpt) xr[i] = buf_load<P, FLN_FWD_LOAD_POL>(xq, t + i * kT);
    if constexpr (RES) {
      const rsrc_t rq = make_rsrc(R + row * N, nb);
#pragma unroll
      for (int i = 0; i < CPT; ++i)
        if (i < cpt) rr[i] = buf_load<P, FLN_FWD_LOAD_POL>(rq, t + i * kT);
    }
  };

  // The register half of a row (CR > 0).
  auto load_hi = [&](int it) {
    const int64_t row = static_cast<int64_t>(it) * stride + blockIdx.x;
    const rsrc_t xq = make_rsrc(X + row * N, it < iters ? row_bytes : 0u);
#pragma unroll
    for (int j = 0; j < CR; ++j)
      if (CL + j < cpt) cur[j] = buf_load<P, FLN_FWD_LOAD_POL>(xq, t + (CL + j) * kT);
  };

  load_row(0);
  if constexpr (CR > 0) load_hi(0);
  for (int it = 0; it < iters; ++it) {
    const int64_t row = static_cast<int64_t>(it) * stride + blockIdx.x;
    float(*slots)[kW + 16] = red[it & 1];
    // Pass A: park the row in LDS (writing h with RES), plain sum.
    const rsrc_t hr = make_rsrc(RES && p.h ? static_cast<T*>(p.h) + row * N : nullptr, row_bytes);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (i >= cpt) continue;  // uniform
      // (indices clamped so that neither arm names an element past its array)
      P v = i < CX ? xr[i < CX ? i : 0] : cur[i >= CL ? i - CL : 0];
      if constexpr (RES) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          v.v[e] = from_f32<T>(to_f32(xr[i].v[e]) + to_f32(rr[i].v[e]));
        buf_store<P, FLN_FWD_STORE_POL>(v, hr, t + i * kT);
      }
      if (i < CL) xs[i * kT + t] = v;
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += to_f32(v.v[e]);
    }
    load_row(it + 1);  // in flight during the passes over LDS
    float mean = 0.0f;
    if (!p.rms) {
      const float sum = row_allreduce<SumOp>(s, slots[0], kW, 0, wave, lane);
      mean = sum * inv_n;
      mean = fmaf(fmaf(-mean, fn, sum), inv_n, mean);
    }
    // Pass B: centred sum of squares (vectors past the row left out).
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      if (i >= cpt) continue;  // uniform
      const P v = row_vec(i);
      if (t + i * kT < nvec) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float d = to_f32(v.v[e]) - mean;
          q = fmaf(d, d, q);
        }
      }
    }
    q = row_allreduce<SumOp>(q, slots[1], kW, 0, wave, lane);
    const float rstd = __builtin_amdgcn_rsqf(q * inv_n + p.eps);  // v_rsq_f32, 1 ulp
    const float poison = FP8 != 0 ? row_poison(mean, rstd) : 0.0f;  // fp8 scales: NaN

    // Output element e of vector i of the row.
    auto affine = [&](int i, int e, const P& xv, const P& gv, const P& bv) -> float {
      (void)i;
      float a = fmaf((to_f32(xv.v[e]) - mean) * rstd, has_g ? to_f32(gv.v[e]) : 1.0f,
                     to_f32(bv.v[e]));
      if constexpr (GELU == 1) a = TAB ? gelu_erf_tab(gelu_tab, a) : gelu_erf(a);
      if constexpr (GELU == 2) a = gelu_tanh(a);
      return a;
    };
    // Pass C: outputs (CR > 0: the register half first, then the next row's register half is
    // put in flight, then the LDS half).
    if constexpr (FP8 == 0) {
      const rsrc_t yr = make_rsrc(static_cast<T*>(p.y) + row * N, row_bytes);
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const int i = CR > 0 ? (k < CR ? CL + k : k - CR) : k;
        if constexpr (CR > 0)
          if (k == CR) load_hi(it + 1);
        if (i >= cpt) continue;  // uniform
        const int v = t + i * kT;
        const P xv = row_vec(i);
        const P gv = buf_load<P>(g_rs, v);
        const P bv = buf_load<P>(b_rs, v);
        P o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o.v[e] = from_f32<T>(affine(i, e, xv, gv, bv));
        buf_store<P, FLN_FWD_STORE_POL>(o, yr, v);
      }
    } else {
      const rsrc_t qr = make_rsrc(static_cast<uint8_t*>(p.y) + row * N, static_cast<uint32_t>(N));
      auto codes = [&](const float* a, float m, bool in_range) -> QW {
        QW w;
        if constexpr (VEC == 8) {
          w.x = in_range ? fp8x4_inrange(a[0] * m, a[1] * m, a[2] * m, a[3] * m)
                         : fp8x4(a[0] * m, a[1] * m, a[2] * m, a[3] * m);
          w.y = in_range ? fp8x4_inrange(a[4] * m, a[5] * m, a[6] * m, a[7] * m)
                         : fp8x4(a[4] * m, a[5] * m, a[6] * m, a[7] * m);
        } else {
          w = in_range ? fp8x4_inrange(a[0] * m, a[1] * m, a[2] * m, a[3] * m)
                       : fp8x4(a[0] * m, a[1] * m, a[2] * m, a[3] * m);
        }
        return w;
      };
      if constexpr (FP8 == 2) {
        // OCP MX: a 32-element block is G adjacent lanes' vectors (cols % 32 == 0).
        constexpr int G = 32 / VEC;
        const uint32_t nblk = static_cast<uint32_t>(N / 32);
        const rsrc_t br = make_rsrc(p.bscale + row * nblk, nblk);
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          if (i >= cpt) continue;  // uniform
          const int v = t + i * kT;
          const P xv = row_vec(i);
          const P gv = buf_load<P>(g_rs, v);
          const P bv = buf_load<P>(b_rs, v);
          float a[VEC];
          float bm = 0.0f;
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            a[e] = affine(i, e, xv, gv, bv);
            bm = fmaxf(bm, fabsf(a[e]));
          }
          const MxScale ms = mx_scale_e4m3(group_max<G>(bm), mx_poison(poison));
          BufIO<VEC, FLN_FWD_STORE_POL>::store(codes(a, ms.mul, false), qr,
                                               static_cast<uint32_t>(v) * VEC);
          __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(ms.code), br,
                                               v % G == 0 ? v / G : kOutOfRange, 0, 0);
        }
      } else {
        // Per-row scale: the row maximum first (vectors past the row left out), then codes.
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          if (i >= cpt) continue;  // uniform
          const int v = t + i * kT;
          const P xv = row_vec(i);
          const P gv = buf_load<P>(g_rs, v);
          const P bv = buf_load<P>(b_rs, v);
          if (v < nvec) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) am = fmaxf(am, fabsf(affine(i, e, xv, gv, bv)));
          }
        }
        am = row_allreduce<MaxOp>(am, slots[2], kW, 0, wave, lane);
        am += poison;
        const float inv = am > 0.0f ? 448.0f * __builtin_amdgcn_rcpf(am) : 0.0f;  // 1 ulp
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          if (i >= cpt) continue;  // uniform
          const int v = t + i * kT;
          const P xv = row_vec(i);
          const P gv = buf_load<P>(g_rs, v);
          const P bv = buf_load<P>(b_rs, v);
          float a[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) a[e] = affine(i, e, xv, gv, bv);
          // |a * inv| <= 448 (1 + 2^-22) < 464 (1-ulp reciprocal, two roundings): in
          // range for the unclamped conversion.
          BufIO<VEC, FLN_FWD_STORE_POL>::store(codes(a, inv, true), qr,
                                               static_cast<uint32_t>(v) * VEC);
        }
        buf_store_f32(am * (1.0f / 448.0f), make_rsrc(p.scale + row, 4u),
                      t == 0 ? 0u : kOutOfRange);
      }
    }
    const uint32_t stat_off = t == 0 ? 0u : kOutOfRange;
    buf_store_f32(mean, make_rsrc(p.mean ? p.mean + row : nullptr, 4u), stat_off);
    buf_store_f32(rstd, make_rsrc(p.rstd ? p.rstd + row : nullptr, 4u), stat_off);
  }
}

// ---------------------------------------------------------------------------------------------
// Rows past the LDS tile (16-bit rows of more than 65536 columns, fp32 rows of more than 32768)
// and long rows off the vector path: one 1024-thread block per row at a time, rows
// grid-stride, each pass streaming the row in steps of U vectors per thread (64 bytes: 4
// vectors, or 16-32 elements on the scalar path; thread t reads vectors base + t + 1024 u, so
// every wave-wide access is coalesced):
//   pass 1, statistics: per thread, each step's valid elements are reduced to (count, mean,
//     centred sum of squares) and merged into the thread's running triple (the pairwise update
//     of Chan, Golub and LeVeque); the block's mean is then the sum of count x mean over the
//     threads / N, and its centred sum of squares the sum of each thread's M2 plus
//     count (mean_t - mean)^2 -- two block reductions in a fixed order, so the statistics are
//     bitwise reproducible and need no E[x^2] - mean^2 cancellation.  RMSNorm sums squares;
//   pass 2, fp8 with a per-row scale only: the row maximum of the outputs;
//   last pass: outputs (and, with a residual, h = x + r written during pass 1).
// x (and the residual) are read once per pass, the passes walking the row in alternate
// directions so that each starts on the lines the previous one read last, which are still in L2
// (the last pass loads non-temporal).  Most of a later pass still comes from HBM: at 131072
// bf16 columns a block's row is 256 KiB against an L2 share of 64-128 KiB per CU.
// ---------------------------------------------------------------------------------------------
constexpr int kFwdWideThreads = 1024;
constexpr int kFwdWideStepBytes = 64;  // bytes of the row per thread and step (4 vectors)

template <class T, int FP8, bool RES, int GELU, int VEC>
__global__ __launch_bounds__(kFwdWideThreads) void fwd_wide_kernel(const FwdParams p) {
  constexpr int kT = kFwdWideThreads;
  constexpr int kW = kT / kWave;
  constexpr int U = kFwdWideStepBytes / (VEC * static_cast<int>(sizeof(T)));
  using P = Pack<T, VEC>;
  __shared__ float red[2][3][kW + 16];  // [parity][reduction][wave], padded
  // Exact GELU of 16-bit rows: the log2 Phi table (4 KiB), one entry per thread, as in the
  // register kernel; fp32 rows keep the polynomial (their kernels are not VALU-bound, and the
  // table reads slowed them: 1024 x 24576 41.2 -> 43.0 us).
  constexpr bool TAB = GELU == 1 && sizeof(T) == 2;
  __shared__ float4 gelu_tab[TAB ? kGeluLogTabN : 1];
  if constexpr (TAB) {
    if (threadIdx.x < kGeluLogTabN)
      gelu_tab[threadIdx.x] = reinterpret_cast<const float4*>(kGeluLogTabData)[threadIdx.x];
    __syncthreads();
  }
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int64_t N = p.cols;
  const uint32_t nvec = static_cast<uint32_t>(N / VEC);
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  const float fn = static_cast<float>(N);
  const float inv_n = 1.0f / fn;
  const T* X = static_cast<const T*>(p.x);
  const T* R = static_cast<const T*>(p.res);
  const rsrc_t g_rs = make_rsrc(p.gamma, row_bytes);
  const rsrc_t b_rs = make_rsrc(p.beta, row_bytes);  // absent beta reads as zeros
  const bool has_g = p.gamma != nullptr;

  int parity = 0;
  for (int64_t row = blockIdx.x; row < p.rows; row += gridDim.x, parity ^= 1) {
    float(*slots)[kW + 16] = red[parity];
    const rsrc_t xq = make_rsrc(X + row * N, row_bytes);
    const rsrc_t rq = make_rsrc(RES ? R + row * N : nullptr, row_bytes);
    // Step `base`: vectors base + t + kT u of the row (zeros past the row); with a residual,
    // h = x + r rounded to T, as every pass recomputes it.
    auto load_step = [&](uint32_t base, P (&hv)[U], auto pol) {
      constexpr int POL = decltype(pol)::value;
      P rv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        hv[u] = buf_load<P, POL>(xq, base + t + kT * u);
        if constexpr (RES) rv[u] = buf_load<P, POL>(rq, base + t + kT * u);
      }
      if constexpr (RES) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            hv[u].v[e] = from_f32<T>(to_f32(hv[u].v[e]) + to_f32(rv[u].v[e]));
      }
    };
    using Keep = std::integral_constant<int, kDefault>;
    using Last = std::integral_constant<int, kStream>;

    // Pass 1: statistics (and h).
    const rsrc_t hr = make_rsrc(RES && p.h ? static_cast<T*>(p.h) + row * N : nullptr,
                                row_bytes);
    float mean = 0.0f, rstd;
    float cnt = 0.0f, mu = 0.0f, m2 = 0.0f;  // this thread's elements: count, mean, M2
    for (uint32_t base = 0; base < nvec; base += kT * U) {
      P hv[U];
      load_step(base, hv, Keep{});
      if constexpr (RES) {
#pragma unroll
        for (int u = 0; u < U; ++u) buf_store<P, FLN_FWD_STORE_POL>(hv[u], hr, base + t + kT * u);
      }
      if (p.rms) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < VEC; ++e) m2 = fmaf(to_f32(hv[u].v[e]), to_f32(hv[u].v[e]), m2);
        continue;
      }
      float c = 0.0f, s = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (base + t + kT * u < nvec) {
          c += static_cast<float>(VEC);
#pragma unroll
          for (int e = 0; e < VEC; ++e) s += to_f32(hv[u].v[e]);
        }
      }
      if (c > 0.0f) {
        const float mg = s / c;
        float q = 0.0f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (base + t + kT * u < nvec) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
              const float d = to_f32(hv[u].v[e]) - mg;
              q = fmaf(d, d, q);
            }
          }
        }
        const float nn = cnt + c;
        const float d = mg - mu;
        const float w = c / nn;
        mu = fmaf(d, w, mu);
        m2 += fmaf(d * d, cnt * w, q);
        cnt = nn;
      }
    }
    if (p.rms) {
      const float q = row_allreduce<SumOp>(m2, slots[0], kW, 0, wave, lane);
      rstd = __builtin_amdgcn_rsqf(q * inv_n + p.eps);  // v_rsq_f32, 1 ulp
    } else {
      const float sum = row_allreduce<SumOp>(cnt * mu, slots[0], kW, 0, wave, lane);
      mean = sum * inv_n;
      mean = fmaf(fmaf(-mean, fn, sum), inv_n, mean);
      const float dm = mu - mean;
      const float q = row_allreduce<SumOp>(fmaf(cnt * dm, dm, m2), slots[1], kW, 0, wave, lane);
      rstd = __builtin_amdgcn_rsqf(q * inv_n + p.eps);
    }
    const float poison = FP8 != 0 ? row_poison(mean, rstd) : 0.0f;  // fp8 scales: NaN

    auto affine = [&](const P& hv, const P& gv, const P& bv, int e) -> float {
      float a = fmaf((to_f32(hv.v[e]) - mean) * rstd, has_g ? to_f32(gv.v[e]) : 1.0f,
                     to_f32(bv.v[e]));
      if constexpr (GELU == 1) a = TAB ? gelu_erf_tab(gelu_tab, a) : gelu_erf(a);
      if constexpr (GELU == 2) a = gelu_tanh(a);
      return a;
    };

    // Pass 2 (per-row fp8 scale): the row maximum of the outputs.
    float inv = 0.0f, am = 0.0f;
    // Successive passes walk the row in alternate directions, so each pass starts on the part of
    // the row the previous one read last, which is still in L2.
    const uint32_t steps = (nvec + kT * U - 1) / (kT * U);
    if constexpr (FP8 == 1) {
      for (uint32_t st = steps; st-- > 0;) {
        const uint32_t base = st * (kT * U);
        P hv[U];
        load_step(base, hv, Keep{});
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint32_t v = base + t + kT * u;
          const P gv = buf_load<P>(g_rs, v);
          const P bv = buf_load<P>(b_rs, v);
          if (v < nvec) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) am = fmaxf(am, fabsf(affine(hv[u], gv, bv, e)));
          }
        }
      }
      am = row_allreduce<MaxOp>(am, slots[2], kW, 0, wave, lane);
      am += poison;
      inv = am > 0.0f ? 448.0f * __builtin_amdgcn_rcpf(am) : 0.0f;  // v_rcp_f32, 1 ulp
    }

    // Last pass: outputs (backwards after the statistics pass, forwards after the fp8 maximum).
    for (uint32_t k = 0; k < steps; ++k) {
      const uint32_t base = (FP8 == 1 ? k : steps - 1 - k) * (kT * U);
      P hv[U];
      load_step(base, hv, Last{});
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t v = base + t + kT * u;
        const P gv = buf_load<P>(g_rs, v);
        const P bv = buf_load<P>(b_rs, v);
        float a[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) a[e] = affine(hv[u], gv, bv, e);
        if constexpr (FP8 == 0) {
          P o;
#pragma unroll
          for (int e = 0; e < VEC; ++e) o.v[e] = from_f32<T>(a[e]);
          buf_store<P, FLN_FWD_STORE_POL>(o, make_rsrc(static_cast<T*>(p.y) + row * N, row_bytes),
                                          v);
        } else {
          float m = inv;
          if constexpr (FP8 == 2) {
            // OCP MX: a 32-element block is G adjacent lanes' vectors (cols % 32 == 0, and
            // every step starts on a block boundary).
            constexpr int G = 32 / VEC;
            float bm = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) bm = fmaxf(bm, fabsf(a[e]));
            const MxScale ms = mx_scale_e4m3(group_max<G>(bm), mx_poison(poison));
            m = ms.mul;  // |a * m| < 512: the saturating conversion clamps to 448
            const uint32_t nblk = static_cast<uint32_t>(N / 32);
            __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(ms.code),
                                                 make_rsrc(p.bscale + row * nblk, nblk),
                                                 v % G == 0 ? v / G : kOutOfRange, 0, 0);
          }
          // Per-row scale: |a * inv| <= 448 (1 + 2^-22) < 464, but the saturating form is kept
          // (the scalar path converts one element at a time).
          const rsrc_t qr = make_rsrc(static_cast<uint8_t*>(p.y) + row * N,
                                      static_cast<uint32_t>(N));
          if constexpr (VEC == 8) {
            u32x2 w;
            w.x = fp8x4(a[0] * m, a[1] * m, a[2] * m, a[3] * m);
            w.y = fp8x4(a[4] * m, a[5] * m, a[6] * m, a[7] * m);
            BufIO<8, FLN_FWD_STORE_POL>::store(w, qr, v * 8u);
          } else if constexpr (VEC == 4) {
            BufIO<4, FLN_FWD_STORE_POL>::store(fp8x4(a[0] * m, a[1] * m, a[2] * m, a[3] * m), qr,
                                               v * 4u);
          } else {
            __builtin_amdgcn_raw_buffer_store_b8(fp8x1(a[0] * m), qr, v, 0, FLN_FWD_STORE_POL);
          }
        }
      }
    }
    const uint32_t stat_off = t == 0 ? 0u : kOutOfRange;
    if constexpr (FP8 == 1)
      buf_store_f32(am * (1.0f / 448.0f), make_rsrc(p.scale + row, 4u), stat_off);
    buf_store_f32(mean, make_rsrc(p.mean ? p.mean + row : nullptr, 4u), stat_off);
    buf_store_f32(rstd, make_rsrc(p.rstd ? p.rstd + row : nullptr, 4u), stat_off);
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

template <class T, class A, int FP8>
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
    // fp8 scales of a row with unusable statistics (as row_poison): NaN, 0xFF for MX blocks
    const bool bad = !__builtin_isfinite(mean) || !(rstd > 0 && rstd < __builtin_huge_val());
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
    if constexpr (FP8 == 0) {
      T* y = static_cast<T*>(p.y);
      for (int64_t j = threadIdx.x; j < N; j += blockDim.x) y[base + j] = static_cast<T>(outv(j));
    } else {
      if (p.mx) {
        // Blocks of 32 consecutive elements are 32 adjacent lanes here (blockDim is a multiple
        // of 64 and cols % 32 == 0, so a block's lanes are all in or all past the row).
        uint8_t* q8 = static_cast<uint8_t*>(p.y);
        for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
          const float a = static_cast<float>(outv(j));
          const MxScale ms = mx_scale_e4m3(group_max<32>(fabsf(a)), bad ? 0xFF : 0);
          q8[base + j] = fp8x1(a * ms.mul);
          if ((j & 31) == 0)
            p.bscale[row * (N / 32) + j / 32] = static_cast<uint8_t>(ms.code);
        }
        __syncthreads();
        continue;
      }
      A am = 0;
      for (int64_t j = threadIdx.x; j < N; j += blockDim.x) {
        const A a = outv(j);
        const A m = a < 0 ? -a : a;
        am = m > am ? m : am;
      }
      am = block_allreduce<A, true>(am, red[2]);
      const float amf = bad ? __builtin_nanf("") : static_cast<float>(am);
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

// Blocks of `kernel` in `threads`-thread blocks that fit on the current device at once; the
// per-CU count is cached per device in `cache_per_device` (threads may race to fill a slot: they
// store the same value).
template <class K>
int64_t resident_blocks(K kernel, int threads, std::atomic<int>* cache_per_device) {
  const int dev = current_device();
  int per_cu = cache_per_device[dev].load(std::memory_order_relaxed);
  if (per_cu == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    cache_per_device[dev].store(per_cu, std::memory_order_relaxed);
  }
  return static_cast<int64_t>(per_cu) * device_cu_count();
}

template <class T, int FP8, bool RES, int GELU, int VEC, int VPL, bool EXACT, int MAXT>
int launch_reg_t(const FwdParams& p, int threads, hipStream_t s) {
  // The exact-GELU kernels fill their LDS table with one entry per thread.
  if (GELU == 1 && threads < kGeluLogTabN) return FLN_ERR_INVALID;
  if (p.wpr < 1 || threads < kWave * p.wpr || threads > MAXT || threads % kWave != 0)
    return FLN_ERR_INVALID;
  const int rows_per_block = threads / (kWave * p.wpr);
  const int64_t row_blocks = (p.rows + rows_per_block - 1) / rows_per_block;
  auto kernel = fwd_reg_kernel<T, FP8, RES, GELU, VEC, VPL, EXACT, MAXT>;
  // Per instantiation, [waves per block][device]: one instantiation runs with several block
  // sizes (a 1024-thread one with 5-16 waves per row, one row per block).
  static std::atomic<int> occupancy_cache[MAXT / kWave + 1][64];
  const int64_t cus = device_cu_count();
  const int64_t resident = resident_blocks(kernel, threads, occupancy_cache[threads / kWave]);
  // Blocks per CU: the fewest whose rows in flight move enough bytes per CU to cover the per-row
  // latency (loads in flight, reductions, barriers): rows dealt to the CU at once x PD rows of
  // loads ahead x the bytes each row moves >= 32 KiB for one-wave rows (no barrier), 56 KiB for
  // rows over several waves, 7/4 of that with a second dependent row reduction (fp8 row scale)
  // or the exact GELU's VALU work -- except the fp8 row scale in 256-thread blocks (one to four
  // waves per row, no residual), which runs best at 42 KiB.  More concurrent rows than that only
  // cost DRAM locality.  Measured on MI355X (bf16, us, HIP events; blocks per CU in brackets):
  // 8192 x 4096 LN 26.9 [3] 24.4 [1] 23.8 [2]; LN + GELU(erf) 31.1 [2] 30.0 [4]; 32768 x 768 25.5
  // [1] 20.2 [2]; LN -> fp8 32768 x 7168 (7 waves per row) 198 [1] 147 [2] 133 [3], 32768 x 8192
  // 189.5 [1] 136.6 [2] 145.5 [3] 145.0 [4], 65536 x 4096 190.5 [1] 136.9 [2] 146.0 [3] 145.5
  // [4], 262144 x 1024 198.0 [1] 146.1 [2] 153.3 [3]; residual + RMSNorm -> fp8 at 32768 x 7168
  // 283 [1] 300 [2].
  constexpr int PD = fwd_prefetch_depth<T, FP8, RES, GELU, VEC, VPL, MAXT>();
  const int64_t es = static_cast<int64_t>(sizeof(T));
  const int64_t moved_per_row = p.cols * (es * (RES ? 3 : 1) + (FP8 ? 1 : es));
  const int64_t per_block = moved_per_row * rows_per_block * PD;
  int64_t target = p.wpr == 1 ? (32 << 10) : (56 << 10);
  if (FP8 == 1 && !RES && threads == 256)
    target = 42 << 10;
  else if (FP8 == 1 || GELU == 1)
    target = target * 7 / 4;
  int64_t per_cu = per_block > 0 ? (target + per_block - 1) / per_block : 1;
  const int forced = tuning().fwd_grid_mult;
  if (forced > 0) per_cu = forced;
  int64_t grid = per_cu * cus;
  if (grid > resident) grid = resident;
  if (grid > row_blocks) grid = row_blocks;
  if (grid > kMaxGrid) grid = kMaxGrid;
  static std::atomic<void*> fn_cache[64];
  return launch_cached(kernel, fn_cache, dim3(grid), dim3(threads), s, p, row_blocks);
}

template <class T, int FP8, bool RES, int GELU, int VEC, int VPL, bool EXACT>
int launch_reg(const FwdParams& p, int threads, hipStream_t s) {
  if (threads <= 256) return launch_reg_t<T, FP8, RES, GELU, VEC, VPL, EXACT, 256>(p, threads, s);
  return launch_reg_t<T, FP8, RES, GELU, VEC, VPL, EXACT, 1024>(p, threads, s);
}

// Largest vectors-per-lane instantiated: 32 elements per lane for 16-byte vectors (keeps a
// LayerNorm row slice, its fp32 copy and the affine parameters within ~120 VGPRs), 16 for the
// scalar path.
template <int VEC> constexpr int max_vpl() { return VEC == 1 ? 16 : 32 / VEC; }

template <class T, int FP8, bool RES, int GELU, int VEC, int VPL>
int launch_reg_exact(const FwdParams& p, bool exact, int threads, hipStream_t s) {
  // The exact (mask-free) variant is only instantiated for 16-byte vectors.
  if constexpr (VEC > 1)
    if (exact) return launch_reg<T, FP8, RES, GELU, VEC, VPL, true>(p, threads, s);
  return launch_reg<T, FP8, RES, GELU, VEC, VPL, false>(p, threads, s);
}

template <class T, int FP8, bool RES, int GELU, int VEC, int VPL>
int launch_reg_odd(const FwdParams& p, bool exact, int threads, hipStream_t s) {
  // The flavours the plan gives these tiles: GELU only as LN + GELU; with a residual 3 or 5
  // vectors per lane (6 and 7 need AGPRs there); MX outputs only with a residual; 6 vectors for
  // the fp8 row scale and GELU.
  constexpr bool kPlanned =
      VEC == 8 && (GELU == 0 || (FP8 == 0 && !RES)) && (!RES || VPL == 3 || VPL == 5) &&
      (FP8 != 2 || RES) && (VPL != 6 || (FP8 == 1 && !RES) || GELU != 0);
  if constexpr (kPlanned)
    if (exact && threads <= 256)
      return launch_reg_t<T, FP8, RES, GELU, VEC, VPL, true, 256>(p, threads, s);
  return FLN_ERR_INVALID;
}

template <class T, int FP8, bool RES, int GELU, int VEC>
int launch_reg_vpl(const FwdParams& p, int vpl, bool exact, int threads, hipStream_t s) {
  constexpr int CAP = max_vpl<VEC>();
  switch (vpl) {
    case 1: return launch_reg_exact<T, FP8, RES, GELU, VEC, 1>(p, exact, threads, s);
    case 2: return launch_reg_exact<T, FP8, RES, GELU, VEC, 2>(p, exact, threads, s);
    case 4: return launch_reg_exact<T, FP8, RES, GELU, VEC, 4>(p, exact, threads, s);
    // Odd and six-vector tiles (3, 5, 6, 7 vectors per lane): exact tilings only, in blocks of at
    // most 256 threads, for the 16-bit flavours that the plan gives them.
    case 3: return launch_reg_odd<T, FP8, RES, GELU, VEC, 3>(p, exact, threads, s);
    case 5: return launch_reg_odd<T, FP8, RES, GELU, VEC, 5>(p, exact, threads, s);
    case 6: return launch_reg_odd<T, FP8, RES, GELU, VEC, 6>(p, exact, threads, s);
    case 7: return launch_reg_odd<T, FP8, RES, GELU, VEC, 7>(p, exact, threads, s);
    case 8:
      if constexpr (CAP >= 8)
        return launch_reg_exact<T, FP8, RES, GELU, VEC, 8>(p, exact, threads, s);
      return FLN_ERR_INVALID;
    case 16:
      if constexpr (CAP >= 16)
        return launch_reg_exact<T, FP8, RES, GELU, VEC, 16>(p, exact, threads, s);
      return FLN_ERR_INVALID;
    default: return FLN_ERR_INVALID;
  }
}

// Flavour dispatch: GELU only exists without residual and fp8 output.  FP8: 0 none, 1 fp8 with
// a per-row scale, 2 OCP MX fp8 (E8M0 scale per 32 elements).
template <class T, int FP8, int VEC>
int launch_reg_flavour(const FwdParams& p, int vpl, bool exact, int threads, hipStream_t s) {
  if (p.res) return launch_reg_vpl<T, FP8, true, 0, VEC>(p, vpl, exact, threads, s);
  if constexpr (FP8 == 0) {
    if (p.gelu == FLN_GELU_ERF)
      return launch_reg_vpl<T, false, false, 1, VEC>(p, vpl, exact, threads, s);
    if (p.gelu == FLN_GELU_TANH)
      return launch_reg_vpl<T, false, false, 2, VEC>(p, vpl, exact, threads, s);
  }
  return launch_reg_vpl<T, FP8, false, 0, VEC>(p, vpl, exact, threads, s);
}

template <class T, int FP8, int VEC>
int launch_lds(const FwdParams& p, hipStream_t s) {
  int64_t grid = device_cu_count();  // one block per CU: the parked row fills most of the LDS
  if (grid > p.rows) grid = p.rows;
  const dim3 g(static_cast<unsigned>(grid)), b(kFwdLdsThreads);
  if (p.res) {
    hipLaunchKernelGGL((fwd_lds_kernel<T, FP8, true, 0, VEC>), g, b, 0, s, p);
  } else if (FP8 == 0 && p.gelu == FLN_GELU_ERF) {
    hipLaunchKernelGGL((fwd_lds_kernel<T, 0, false, 1, VEC>), g, b, 0, s, p);
  } else if (FP8 == 0 && p.gelu == FLN_GELU_TANH) {
    hipLaunchKernelGGL((fwd_lds_kernel<T, 0, false, 2, VEC>), g, b, 0, s, p);
  } else {
    hipLaunchKernelGGL((fwd_lds_kernel<T, FP8, false, 0, VEC>), g, b, 0, s, p);
  }
  return static_cast<int>(hipGetLastError());
}

// LayerNorm / RMSNorm rows (and LN + GELU: tanh, or fp32) of 8193..16384 vectors (16-bit
// 65537..131072 columns, fp32 32769..65536), without residual or fp8 output: 8 vectors per
// thread parked in LDS, up to 8 in registers, so x is read from HBM once.  Against the
// streamed wide-row kernel (which reads x twice), us: bf16 512 x 131072
// LN 70.3 -> 58.5, RMSNorm 64.3 -> 55.1, 1024 x 65544 72.0 -> 60.2; fp16 512 x 131072 68.7 ->
// 59.3; fp32 512 x 65536 66.8 -> 56.1, 1024 x 32772 70.1 -> 58.8; GELU tanh bf16 512 x 131072
// 75.1 -> 67.9, fp32 1024 x 32772 71.7 -> 59.1; exact GELU fp32 512 x 65536 69.6 -> 59.9.  The
// exact GELU of 16-bit rows keeps the streamed kernel (its polynomial, VALU-bound in one block
// per CU: bf16 512 x 131072 79.0 -> 85.9 us), as do the residual and fp8 flavours (their extra
// registers spill: 17-42 VGPRs; LN -> fp8 bf16 512 x 131072 72.1 -> 75.1 us, MXFP8 58.6 ->
// 77.7 us, though 1024 x 65544 gained, 79.4 -> 72.3).
template <class T, int VEC>
int launch_lds_reg(const FwdParams& p, hipStream_t s) {
  int64_t grid = device_cu_count();
  if (grid > p.rows) grid = p.rows;
  const dim3 g(static_cast<unsigned>(grid)), b(kFwdLdsThreads);
  if (p.gelu == FLN_GELU_ERF)
    hipLaunchKernelGGL((fwd_lds_kernel<T, 0, false, 1, VEC, kFwdLdsCpt>), g, b, 0, s, p);
  else if (p.gelu == FLN_GELU_TANH)
    hipLaunchKernelGGL((fwd_lds_kernel<T, 0, false, 2, VEC, kFwdLdsCpt>), g, b, 0, s, p);
  else
    hipLaunchKernelGGL((fwd_lds_kernel<T, 0, false, 0, VEC, kFwdLdsCpt>), g, b, 0, s, p);
  return static_cast<int>(hipGetLastError());
}

// ---------------------------------------------------------------------------------------------
// Few rows past the register tiles (vector path, y overlapping no input): one block per row left
// most CUs idle (bf16 64 x 1048576: 64 blocks, 1.9 TB/s).  Each row splits into S <= 64 column
// chunks of whole steps, one 256-thread block per (row, chunk), in three launches (four with
// the fp8 row scale) and without a workspace (the forward entry points take none).  The first
// bytes of the row's own y (the "head") carry what the blocks of a row hand to each other:
//   fwd_split_stats_kernel: the chunk's (count, sum, M2 about the chunk's mean) -- RMSNorm:
//     (count, 0, sum of squares) -- as float4 s of the head; with a residual, h = x + r is
//     written as well;
//   fwd_split_max_kernel (fp8 row scale): every block merges its row's S triples (lane k loads
//     triple k, wave_allreduce sums in a fixed order: the pairwise merge of Chan, Golub and
//     LeVeque, the same bits in every block) and writes its chunk's maximum |output| as float s
//     after the triples;
//   fwd_split_out_kernel<HEAD = false>: the same statistics (and the row maximum from the
//     chunk maxima), then the outputs of its chunk, but not the head's vectors (for MX a whole
//     number of 32-element blocks);
//   fwd_split_out_kernel<HEAD = true>: one block per row: the same statistics, the head's
//     outputs, mean, rstd and the row scale.  Stream order puts it after every read of the head.
// x (h with a residual) is read twice (three times with a row scale), as in the streamed
// wide-row kernel, but by every CU; successive passes over a chunk alternate direction.
// ---------------------------------------------------------------------------------------------
constexpr int kFwdSplitThreads = 256;
constexpr int kFwdSplitU = 2;                                        // vectors per thread, step
constexpr int kFwdSplitStep = kFwdSplitThreads * kFwdSplitU;         // vectors per step
constexpr int kFwdSplitMax = kWave;                                  // chunks per row
// The head (at most 64 x 20 bytes: 320 fp8 vectors of 4 codes) lies within one step, so within
// chunk 0 and the one step of the head launch.  Steps of 512 vectors (2 per thread) rather than
// 1024 give shorter rows more chunks (bf16, us: 32 x 131072 10.84 -> 10.51, 60 x 131072 13.27 ->
// 12.91, 16 x 1048576 21.03 -> 20.32; 64 x 1048576 and LN -> fp8 unchanged).
static_assert(kFwdSplitMax * 20 / 4 <= kFwdSplitStep, "split head past one step");

// The row statistics (mean, rstd) from the S <= 64 chunk triples at the row's head.  All 64
// lanes must be active; the result is wave-uniform and identical in every block of the row.
__device__ __forceinline__ float2 split_row_stats(const float4* head, int S, int lane,
                                                  float fn, float inv_n, float eps, bool rms) {
  const float4 tr = lane < S ? head[lane] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (rms) {
    const float q = wave_allreduce<SumOp>(tr.z);
    return make_float2(0.0f, __builtin_amdgcn_rsqf(q * inv_n + eps));  // v_rsq_f32, 1 ulp
  }
  const float sum = wave_allreduce<SumOp>(tr.y);
  float mean = sum * inv_n;
  mean = fmaf(fmaf(-mean, fn, sum), inv_n, mean);
  const float d = (tr.x > 0.0f ? tr.y / tr.x : 0.0f) - mean;  // chunk mean - row mean
  const float q = wave_allreduce<SumOp>(fmaf(tr.x * d, d, tr.z));
  return make_float2(mean, __builtin_amdgcn_rsqf(q * inv_n + eps));
}

// Bytes of y per row: fp8 codes or the I/O type.
template <class T, int FP8>
__device__ __forceinline__ char* split_y_row(const FwdParams& p, int64_t row) {
  return static_cast<char*>(p.y) + row * p.cols * (FP8 ? 1 : static_cast<int64_t>(sizeof(T)));
}

// A block's share of its row: chunk s of S, vectors [v_lo, v_hi).
struct SplitChunk {
  int64_t row;
  uint32_t s, v_lo, v_hi;
};
template <bool HEAD>
__device__ __forceinline__ SplitChunk split_chunk(const FwdParams& p, uint32_t nvec,
                                                  uint32_t head_vecs) {
  SplitChunk c;
  const int S = p.splits;
  c.row = HEAD ? static_cast<int64_t>(blockIdx.x) : blockIdx.x / S;
  c.s = HEAD ? 0u : static_cast<uint32_t>(blockIdx.x - c.row * S);
  const uint32_t chunk = static_cast<uint32_t>(p.split_chunk);
  c.v_lo = HEAD ? 0u : c.s * chunk;
  c.v_hi = HEAD ? head_vecs : (c.v_lo + chunk < nvec ? c.v_lo + chunk : nvec);
  return c;
}

template <class T, int FP8, bool RES, int VEC>
__global__ __launch_bounds__(kFwdSplitThreads) void fwd_split_stats_kernel(const FwdParams p) {
  constexpr int kT = kFwdSplitThreads;
  constexpr int kW = kT / kWave;
  constexpr int U = kFwdSplitU;
  using P = Pack<T, VEC>;
  __shared__ float red[2][kW + 16];
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int64_t N = p.cols;
  const SplitChunk c = split_chunk<false>(p, static_cast<uint32_t>(N / VEC), 0u);
  const int64_t row = c.row;
  const uint32_t v_lo = c.v_lo, v_hi = c.v_hi;
  const uint32_t hi_bytes = v_hi * static_cast<uint32_t>(sizeof(P));  // nothing past the chunk
  const rsrc_t xq = make_rsrc(static_cast<const T*>(p.x) + row * N, hi_bytes);
  const rsrc_t rq = make_rsrc(RES ? static_cast<const T*>(p.res) + row * N : nullptr, hi_bytes);
  const rsrc_t hq = make_rsrc(RES && p.h ? static_cast<T*>(p.h) + row * N : nullptr, hi_bytes);
  float cnt = 0.0f, mu = 0.0f, m2 = 0.0f;  // this thread's elements: count, mean, M2
  for (uint32_t base = v_lo; base < v_hi; base += kFwdSplitStep) {
    P hv[U], rv[RES ? U : 1];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      hv[u] = buf_load<P>(xq, base + t + kT * u);
      if constexpr (RES) rv[u] = buf_load<P>(rq, base + t + kT * u);
    }
    if constexpr (RES) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          hv[u].v[e] = from_f32<T>(to_f32(hv[u].v[e]) + to_f32(rv[u].v[e]));
        buf_store<P>(hv[u], hq, base + t + kT * u);  // kept in cache for the later passes
      }
    }
    if (p.rms) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int e = 0; e < VEC; ++e) m2 = fmaf(to_f32(hv[u].v[e]), to_f32(hv[u].v[e]), m2);
      continue;
    }
    float cs = 0.0f, sm = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + t + kT * u < v_hi) {
        cs += static_cast<float>(VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) sm += to_f32(hv[u].v[e]);
      }
    }
    if (cs > 0.0f) {
      const float mg = sm / cs;
      float q = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (base + t + kT * u < v_hi) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float d = to_f32(hv[u].v[e]) - mg;
            q = fmaf(d, d, q);
          }
        }
      }
      const float nn = cnt + cs;
      const float d = mg - mu;
      const float w = cs / nn;
      mu = fmaf(d, w, mu);
      m2 += fmaf(d * d, cnt * w, q);
      cnt = nn;
    }
  }
  const float nb = static_cast<float>((v_hi - v_lo) * static_cast<uint32_t>(VEC));
  float4 out;
  if (p.rms) {
    out = make_float4(nb, 0.0f, row_allreduce<SumOp>(m2, red[0], kW, 0, wave, lane), 0.0f);
  } else {
    const float sum = row_allreduce<SumOp>(cnt * mu, red[0], kW, 0, wave, lane);
    const float dm = mu - sum / nb;
    out = make_float4(nb, sum,
                      row_allreduce<SumOp>(fmaf(cnt * dm, dm, m2), red[1], kW, 0, wave, lane),
                      0.0f);
  }
  if (t == 0) reinterpret_cast<float4*>(split_y_row<T, FP8>(p, row))[c.s] = out;
}

// The source vectors of one step (h, or x + r rounded to T, or x) and the affine outputs.
template <class T, bool RES, int VEC>
struct SplitSource {
  using P = Pack<T, VEC>;
  rsrc_t xq, rq;
  bool from_h;
  __device__ __forceinline__ SplitSource(const FwdParams& p, int64_t row, uint32_t hi_bytes) {
    const int64_t N = p.cols;
    from_h = RES && p.h != nullptr;  // h was written by the statistics pass
    xq = make_rsrc(from_h ? static_cast<const T*>(p.h) + row * N
                          : static_cast<const T*>(p.x) + row * N, hi_bytes);
    rq = make_rsrc(RES && !from_h ? static_cast<const T*>(p.res) + row * N : nullptr, hi_bytes);
  }
  template <int U, int POL>
  __device__ __forceinline__ void load(uint32_t base, int t, P (&hv)[U]) const {
    P rv[RES ? U : 1];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      hv[u] = buf_load<P, POL>(xq, base + t + kFwdSplitThreads * u);
      if constexpr (RES) {
        if (!from_h) rv[u] = buf_load<P, POL>(rq, base + t + kFwdSplitThreads * u);
      }
    }
    if constexpr (RES) {
      if (!from_h) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            hv[u].v[e] = from_f32<T>(to_f32(hv[u].v[e]) + to_f32(rv[u].v[e]));
      }
    }
  }
};

// Head vectors: the S triples (and S chunk maxima with the fp8 row scale) in units of output
// vectors (16 bytes of the I/O type, or VEC fp8 codes), for MX a whole number of 32-element
// blocks.
template <class T, int FP8, int VEC>
__host__ __device__ inline uint32_t split_head_vecs(int S) {
  const uint32_t bytes = static_cast<uint32_t>(S) * (FP8 == 1 ? 20u : 16u);
  const uint32_t vb = FP8 ? static_cast<uint32_t>(VEC) : static_cast<uint32_t>(VEC * sizeof(T));
  uint32_t v = (bytes + vb - 1) / vb;
  if (FP8 == 2) {
    constexpr uint32_t G = 32 / VEC;
    v = (v + G - 1) / G * G;
  }
  return v;
}

template <class T, bool RES, int VEC>
__global__ __launch_bounds__(kFwdSplitThreads) void fwd_split_max_kernel(const FwdParams p) {
  constexpr int kT = kFwdSplitThreads;
  constexpr int kW = kT / kWave;
  constexpr int U = kFwdSplitU;
  using P = Pack<T, VEC>;
  __shared__ float red[kW + 16];
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
  const int64_t N = p.cols;
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  const float fn = static_cast<float>(N);
  const SplitChunk c = split_chunk<false>(p, static_cast<uint32_t>(N / VEC), 0u);
  char* Y = split_y_row<T, 1>(p, c.row);
  const float2 st = split_row_stats(reinterpret_cast<const float4*>(Y), p.splits, lane, fn,
                                    1.0f / fn, p.eps, p.rms != 0);
  const float mean = st.x, rstd = st.y;
  const SplitSource<T, RES, VEC> src(p, c.row, c.v_hi * static_cast<uint32_t>(sizeof(P)));
  const rsrc_t g_rs = make_rsrc(p.gamma, row_bytes);
  const rsrc_t b_rs = make_rsrc(p.beta, row_bytes);  // absent beta reads as zeros
  const bool has_g = p.gamma != nullptr;
  float am = 0.0f;
  const uint32_t steps = (c.v_hi - c.v_lo + kFwdSplitStep - 1) / kFwdSplitStep;
  for (uint32_t k = 0; k < steps; ++k) {  // backwards: from the lines the stats pass read last
    const uint32_t base = c.v_lo + (steps - 1 - k) * kFwdSplitStep;
    P hv[U];
    src.template load<U, kDefault>(base, t, hv);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = base + t + kT * u;
      const P gv = buf_load<P>(g_rs, v);
      const P bv = buf_load<P>(b_rs, v);
      if (v < c.v_hi) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          am = fmaxf(am, fabsf(fmaf((to_f32(hv[u].v[e]) - mean) * rstd,
                                    has_g ? to_f32(gv.v[e]) : 1.0f, to_f32(bv.v[e]))));
      }
    }
  }
  am = row_allreduce<MaxOp>(am, red, kW, 0, wave, lane);
  if (t == 0) reinterpret_cast<float*>(Y + p.splits * 16)[c.s] = am;
}

template <class T, int FP8, bool RES, int GELU, int VEC, bool HEAD>
__global__ __launch_bounds__(kFwdSplitThreads) void fwd_split_out_kernel(const FwdParams p) {
  constexpr int kT = kFwdSplitThreads;
  constexpr int U = kFwdSplitU;
  using P = Pack<T, VEC>;
  static_assert(sizeof(P) == 16, "vector path only");
  static_assert(FP8 == 0 || GELU == 0, "no GELU before fp8 outputs");
  constexpr bool TAB = GELU == 1 && sizeof(T) == 2;  // as in the register kernel
  __shared__ float4 gelu_tab[TAB ? kGeluLogTabN : 1];
  if constexpr (TAB) {
    if (threadIdx.x < kGeluLogTabN)
      gelu_tab[threadIdx.x] = reinterpret_cast<const float4*>(kGeluLogTabData)[threadIdx.x];
    __syncthreads();
  }
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int64_t N = p.cols;
  const uint32_t row_bytes = static_cast<uint32_t>(N * sizeof(T));
  const float fn = static_cast<float>(N);
  const int S = p.splits;
  const uint32_t head = split_head_vecs<T, FP8, VEC>(S);
  const SplitChunk c = split_chunk<HEAD>(p, static_cast<uint32_t>(N / VEC), head);
  const uint32_t v_first = HEAD ? 0u : (c.v_lo > head ? c.v_lo : head);  // first vector written
  char* Y = split_y_row<T, FP8>(p, c.row);
  const float2 st = split_row_stats(reinterpret_cast<const float4*>(Y), S, lane, fn, 1.0f / fn,
                                    p.eps, p.rms != 0);
  const float mean = st.x, rstd = st.y;
  const float poison = FP8 != 0 ? row_poison(mean, rstd) : 0.0f;  // fp8 scales: NaN
  float am = 0.0f, inv = 0.0f;
  if constexpr (FP8 == 1) {  // the row maximum from the chunk maxima (max: any order)
    const float* cm = reinterpret_cast<const float*>(Y + S * 16);
    am = wave_allreduce<MaxOp>(lane < S ? cm[lane] : 0.0f) + poison;
    inv = am > 0.0f ? 448.0f * __builtin_amdgcn_rcpf(am) : 0.0f;  // v_rcp_f32, 1 ulp
  }
  // The head block overwrites the head (several waves' worth of fp8 vectors): every wave has
  // its statistics in registers first (the reductions above waited for the loads).
  if constexpr (HEAD) __syncthreads();
  const SplitSource<T, RES, VEC> src(p, c.row, c.v_hi * static_cast<uint32_t>(sizeof(P)));
  const rsrc_t yq = make_rsrc(Y, c.v_hi * static_cast<uint32_t>(FP8 ? VEC : sizeof(P)));
  const rsrc_t g_rs = make_rsrc(p.gamma, row_bytes);
  const rsrc_t b_rs = make_rsrc(p.beta, row_bytes);  // absent beta reads as zeros
  const bool has_g = p.gamma != nullptr;
  const uint32_t steps = (c.v_hi - c.v_lo + kFwdSplitStep - 1) / kFwdSplitStep;
  for (uint32_t k = 0; k < steps; ++k) {
    // Opposite to the pass before: backwards after the statistics, forwards after the maximum.
    const uint32_t base = c.v_lo + (FP8 == 1 ? k : steps - 1 - k) * kFwdSplitStep;
    P hv[U];
    src.template load<U, kStream>(base, t, hv);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = base + t + kT * u;
      const bool put = v >= v_first;  // past the chunk the resource drops the store
      const P gv = buf_load<P>(g_rs, v);
      const P bv = buf_load<P>(b_rs, v);
      float a[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        a[e] = fmaf((to_f32(hv[u].v[e]) - mean) * rstd, has_g ? to_f32(gv.v[e]) : 1.0f,
                    to_f32(bv.v[e]));
        if constexpr (GELU == 1) a[e] = TAB ? gelu_erf_tab(gelu_tab, a[e]) : gelu_erf(a[e]);
        if constexpr (GELU == 2) a[e] = gelu_tanh(a[e]);
      }
      if constexpr (FP8 == 0) {
        P o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o.v[e] = from_f32<T>(a[e]);
        BufIO<16, FLN_FWD_STORE_POL>::store(__builtin_bit_cast(typename BufIO<16, FLN_FWD_STORE_POL>::W, o),
                                            yq, put ? v * 16u : kOutOfRange);
      } else {
        float m = inv;
        if constexpr (FP8 == 2) {
          // OCP MX: a 32-element block is G adjacent lanes' vectors (cols % 32 == 0, every
          // chunk and the head a whole number of blocks).
          constexpr int G = 32 / VEC;
          float bm = 0.0f;
#pragma unroll
          for (int e = 0; e < VEC; ++e) bm = fmaxf(bm, fabsf(a[e]));
          const MxScale ms = mx_scale_e4m3(group_max<G>(bm), mx_poison(poison));
          m = ms.mul;  // |a * m| < 512: the saturating conversion clamps to 448
          const uint32_t nblk = static_cast<uint32_t>(N / 32);
          __builtin_amdgcn_raw_buffer_store_b8(
              static_cast<uint8_t>(ms.code), make_rsrc(p.bscale + c.row * nblk, c.v_hi / G),
              put && v % G == 0 ? v / G : kOutOfRange, 0, 0);
        }
        // Per-row scale: |a * inv| <= 448 (1 + 2^-22) < 464; the saturating form is kept.
        if constexpr (VEC == 8) {
          u32x2 w;
          w.x = fp8x4(a[0] * m, a[1] * m, a[2] * m, a[3] * m);
          w.y = fp8x4(a[4] * m, a[5] * m, a[6] * m, a[7] * m);
          BufIO<8, FLN_FWD_STORE_POL>::store(w, yq, put ? v * 8u : kOutOfRange);
        } else {
          BufIO<4, FLN_FWD_STORE_POL>::store(fp8x4(a[0] * m, a[1] * m, a[2] * m, a[3] * m), yq,
                                             put ? v * 4u : kOutOfRange);
        }
      }
    }
  }
  if constexpr (HEAD) {
    const uint32_t stat_off = t == 0 ? 0u : kOutOfRange;
    buf_store_f32(mean, make_rsrc(p.mean ? p.mean + c.row : nullptr, 4u), stat_off);
    buf_store_f32(rstd, make_rsrc(p.rstd ? p.rstd + c.row : nullptr, 4u), stat_off);
    if constexpr (FP8 == 1)
      buf_store_f32(am * (1.0f / 448.0f), make_rsrc(p.scale + c.row, 4u), stat_off);
  }
}

// Chunks per row: kFwdSplitMax, at least one step each (FLN_FWD_SPLITS forces a count).  More
// chunks measured faster at every row count that takes this path (bf16, us, 16 / 32 / 64
// chunks: 64 x 1048576 81.9 / 71.0 / 67.7; 4 x 1048576 26.4 / 17.7 / 13.3; 200 x 262144 54.0 /
// 52.1 / 51.9; residual 64 x 1048576 138.5 / 126.2 / 116.4).
template <class T, int FP8, int VEC>
int launch_split(FwdParams p, hipStream_t s) {
  const int64_t nvec = p.cols / VEC;
  const int64_t steps = (nvec + kFwdSplitStep - 1) / kFwdSplitStep;
  const int forced = tuning().fwd_splits;
  int64_t splits = forced > 0 ? forced : kFwdSplitMax;
  if (splits > kFwdSplitMax) splits = kFwdSplitMax;
  if (splits > steps) splits = steps;
  if (splits < 1) splits = 1;
  p.split_chunk = (steps + splits - 1) / splits * kFwdSplitStep;
  p.splits = static_cast<int>((nvec + p.split_chunk - 1) / p.split_chunk);
  const dim3 grid(static_cast<unsigned>(p.rows * p.splits)), rows(static_cast<unsigned>(p.rows));
  const dim3 block(kFwdSplitThreads);
  auto run = [&](auto stats, auto body, auto head) {
    hipLaunchKernelGGL(stats, grid, block, 0, s, p);
    if constexpr (FP8 == 1) {
      if (p.res)
        hipLaunchKernelGGL((fwd_split_max_kernel<T, true, VEC>), grid, block, 0, s, p);
      else
        hipLaunchKernelGGL((fwd_split_max_kernel<T, false, VEC>), grid, block, 0, s, p);
    }
    hipLaunchKernelGGL(body, grid, block, 0, s, p);
    hipLaunchKernelGGL(head, rows, block, 0, s, p);
    return static_cast<int>(hipGetLastError());
  };
  if (p.res)
    return run(fwd_split_stats_kernel<T, FP8, true, VEC>,
               fwd_split_out_kernel<T, FP8, true, 0, VEC, false>,
               fwd_split_out_kernel<T, FP8, true, 0, VEC, true>);
  if constexpr (FP8 == 0) {
    if (p.gelu == FLN_GELU_ERF)
      return run(fwd_split_stats_kernel<T, 0, false, VEC>,
                 fwd_split_out_kernel<T, 0, false, 1, VEC, false>,
                 fwd_split_out_kernel<T, 0, false, 1, VEC, true>);
    if (p.gelu == FLN_GELU_TANH)
      return run(fwd_split_stats_kernel<T, 0, false, VEC>,
                 fwd_split_out_kernel<T, 0, false, 2, VEC, false>,
                 fwd_split_out_kernel<T, 0, false, 2, VEC, true>);
  }
  return run(fwd_split_stats_kernel<T, FP8, false, VEC>,
             fwd_split_out_kernel<T, FP8, false, 0, VEC, false>,
             fwd_split_out_kernel<T, FP8, false, 0, VEC, true>);
}

// Byte ranges [a, a + na) and [b, b + nb) overlap (null pointers never do).
inline bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
  if (a == nullptr || b == nullptr) return false;
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + static_cast<uintptr_t>(nb) && y < x + static_cast<uintptr_t>(na);
}

template <class T, int FP8, int VEC>
int launch_wide(const FwdParams& p, hipStream_t s) {
  auto launch = [&](auto kernel) {
    static std::atomic<int> occupancy_cache[64];  // per instantiation, per device
    int64_t grid = resident_blocks(kernel, kFwdWideThreads, occupancy_cache);
    const int forced = tuning().fwd_grid_mult;  // FLN_FWD_GRID_MULT: blocks per CU
    if (forced > 0 && grid > forced * device_cu_count()) grid = forced * device_cu_count();
    if (grid > p.rows) grid = p.rows;
    if (grid > kMaxGrid) grid = kMaxGrid;
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kFwdWideThreads), 0, s, p);
    return static_cast<int>(hipGetLastError());
  };
  if (p.res) return launch(fwd_wide_kernel<T, FP8, true, 0, VEC>);
  if constexpr (FP8 == 0) {
    if (p.gelu == FLN_GELU_ERF) return launch(fwd_wide_kernel<T, 0, false, 1, VEC>);
    if (p.gelu == FLN_GELU_TANH) return launch(fwd_wide_kernel<T, 0, false, 2, VEC>);
  }
  return launch(fwd_wide_kernel<T, FP8, false, 0, VEC>);
}

template <class T, class A, int FP8>
int launch_loop(const FwdParams& p, hipStream_t s) {
  const int threads = p.cols >= 4096 ? 1024 : 256;
  const int64_t grid = p.rows < kMaxGrid ? p.rows : kMaxGrid;
  hipLaunchKernelGGL((fwd_loop_kernel<T, A, FP8>), dim3(grid), dim3(threads), 0, s, p);
  return static_cast<int>(hipGetLastError());
}

// Launch geometry of the register path: waves per row (wpr), vectors per lane (vpl, a power of
// two) and block size.  Rows of up to 4 waves share 256-thread blocks (256 VGPRs per lane) and
// take up to `cap` vectors per lane; wider rows run in blocks of up to 1024 threads (128 VGPRs)
// and take up to `wide_cap`, or `max_cap` (the RAW tiles) when nothing narrower fits 16 waves.
// Preference order:
//   1. the fewest waves per row (power of two) that fit the row within those caps;
//   2. if that tiling leaves masked lanes, an exact tiling with any wave count <= 16 and at least
//      2 vectors per lane (e.g. a 7168-element bf16 row is 7 waves x 64 lanes x 2 vectors), so no
//      lane does masked work.  With rows enough to fill the device, exact tilings of one vector
//      per lane over an odd wave count lose to the power-of-two tiling with masked slots (16384
//      rows, bf16, us: 2560 columns 5 x 1 35.5 against 2 x 4 32.6; 4608 9 x 1 61.9 / 4 x 4 58.8;
//      6656 13 x 1 94.4 / 4 x 4 78.2; fp32 3328 97.2 / 78.8): the extra waves only add
//      cross-wave reductions;
//   3. few rows: more waves per row (fewer vectors each), up to 4, until the grid covers the
//      device.
// Rows of 1, 2 or 4 waves share 256-thread blocks; other row groups are one block each.
struct FwdGeometry {
  int wpr, vpl, threads;
  bool exact, loop;
};

inline FwdGeometry fwd_geometry(int64_t rows, int64_t nvec, int cap, int wide_cap, int max_cap,
                                bool vec_path, int forced_wpr, int64_t cus) {
  FwdGeometry g{};
  constexpr int max_wpr = 16;
  auto per_lane = [&](int w) { return (nvec + kWave * w - 1) / (kWave * w); };
  auto cap_of = [&](int w) { return w <= 4 ? cap : wide_cap; };
  int wpr = 1;
  while (per_lane(wpr) > cap_of(wpr) && wpr < max_wpr) wpr *= 2;
  const bool widest = per_lane(wpr) > cap_of(wpr);  // very long rows: widest register tiles
  if (widest && per_lane(wpr) > max_cap) {
    g.loop = true;
    return g;
  }
  auto fits = [&](int w, int v) { return v <= (widest ? max_cap : cap_of(w)); };
  int vpl = next_pow2(static_cast<int>(per_lane(wpr)));
  bool exact = nvec == static_cast<int64_t>(vpl) * kWave * wpr;
  const int64_t target_waves = 4 * cus;
  if (vec_path && !exact) {
    const int top = widest ? max_cap : (cap > wide_cap ? cap : wide_cap);
    // One vector per lane only when rows are too few to fill the device (latency-bound calls
    // want the extra waves; C1, 32 x 768 fp32: 3 x 1 at 2.61 against 2 x 2 at 2.79 us).
    const int min_v = rows * wpr < target_waves ? 1 : 2;
    for (int v = next_pow2(top) > top ? next_pow2(top) / 2 : top; v >= min_v; v >>= 1) {
      const int64_t w = nvec / (kWave * v);
      if (nvec % (kWave * v) == 0 && w <= max_wpr && fits(static_cast<int>(w), v)) {
        wpr = static_cast<int>(w);
        vpl = v;
        exact = true;
        break;
      }
    }
  }
  // Few rows: spread each row over more waves, up to 4 (latency-bound calls, HIP graph replay,
  // us: 64 x 8192 bf16 16 x 1 4.44 against 4 x 4 3.65; 8 x 4096 bf16 8 x 1 3.36 / 4 x 2 3.10;
  // 64 x 4096 fp32 + GELU 16 x 1 4.55 / 4 x 4 3.95: wider row groups add cross-wave steps).
  constexpr int kFewRowsMaxWpr = 4;
  while (rows * wpr < target_waves && wpr * 2 <= kFewRowsMaxWpr) {
    if (exact && vpl >= 2) {
      wpr *= 2;
      vpl /= 2;
    } else if (!exact && nvec > kWave * wpr * 2) {
      wpr *= 2;
      vpl = next_pow2(static_cast<int>(per_lane(wpr)));
    } else {
      break;
    }
  }
  if (forced_wpr >= 1 && forced_wpr <= max_wpr && per_lane(forced_wpr) <= max_cap) {
    wpr = forced_wpr;
    vpl = next_pow2(static_cast<int>(per_lane(wpr)));
    exact = nvec == static_cast<int64_t>(vpl) * kWave * wpr;
  }
  g.wpr = wpr;
  g.vpl = vpl;
  g.exact = vec_path && exact;
  g.threads = (4 % wpr == 0) ? 256 : kWave * wpr;
  return g;
}

// The launch plan of a forward call: which kernel route runs and its tiling.  The dispatcher
// below and the C-ABI query fln_forward_plan (what functional.get_optimal_config reports) both
// take it from here, so there is one rule.  Inputs besides the shape: the flavour (fp8 / MX
// outputs, residual, GELU form), whether the 16-byte vector path is open (row width and pointer
// alignment), whether the split forward may write its hand-over into y (y overlaps no input and,
// for fp8 codes, is 16-byte aligned), and the CU count.
struct FwdPlan {
  int route;  // FLN_ROUTE_*
  int vec;    // elements per lane load (16 bytes on the vector path, 1 on the scalar path)
  int cap, wide_cap;
  FwdGeometry g;
};

template <class T, int FP8>
FwdPlan plan_typed(int64_t rows, int64_t N, bool has_res, int gelu, bool vec_ok, bool y_ok,
                   int64_t cus) {
  constexpr int VV = 16 / sizeof(T);  // elements per 16-byte vector
  const Tuning& tun = tuning();
  FwdPlan pl{};
  pl.vec = vec_ok ? VV : 1;
  if (tun.force_loop || sizeof(T) == 8) {
    pl.route = FLN_ROUTE_LOOP;
    pl.g.loop = true;
    pl.g.threads = N >= 4096 ? 1024 : 256;  // launch_loop's block
    return pl;
  }
  const int vec = pl.vec;
  // Elements per lane: at most 32 by default (measured best or equal on the 4096-8192-wide
  // benchmark rows); more waves per row beyond that.  The exact odd tiles chosen further down
  // take up to 7 vectors (56 16-bit elements) per lane where they fill every lane.
  const int epl = tun.fwd_epl > 0 ? tun.fwd_epl : 32;
  int cap = (epl >= vec ? epl : vec) / vec;
  const int max_cap = vec_ok ? max_vpl<VV>() : max_vpl<1>();
  if (cap > max_cap) cap = max_cap;
  // Rows of more than 4 waves: 16 elements per lane (8 on the scalar path) keep every flavour
  // within the 128 VGPRs of a 1024-thread block.
  int wide_cap = vec_ok ? 16 / VV : 8;
  if (wide_cap > cap) wide_cap = cap;
  pl.cap = cap;
  pl.wide_cap = wide_cap;
  // The 32-element RAW tiles only for 16-bit types (fp32 ones would hold 64 VGPRs of gamma /
  // beta alone and spill); wider fp32 rows go to the LDS-staged kernel.
  const int raw_cap = (vec_ok && VV < 8) ? wide_cap : max_cap;
  const int64_t nvec = N / vec;
  FwdGeometry g = fwd_geometry(rows, nvec, cap, wide_cap, raw_cap, vec_ok, tun.fwd_wpr, cus);
  // The fp8 row scale (no residual) and 16-bit LN + GELU take 4 waves per row with masked tail
  // lanes over an exact tiling of 5-7 waves when at most 1/8 of the 4-wave tile is masked (bf16,
  // 32768 x 7168 LN -> fp8: 7 waves 134.5 us at its best grid, 4 waves 129.9 us; 8192 x 7168
  // GELU tanh 57.0 -> 46.6 us, erf 57.4 -> 50.0 us, f16 32768 x 7168 tanh 197.9 -> 171.4 us; at
  // 49152 x 5120, 3/8 masked, LN -> fp8 loses: 152.2 -> 161.6 us).  Plain LayerNorm keeps the
  // exact tiling (32768 x 7168: 156.8 against 167.7 us), as do the residual and MX flavours and
  // fp32 GELU (8192 x 7168 tanh 77.2 against 83.5 us).
  if ((FP8 == 1 || (FP8 == 0 && gelu != 0 && sizeof(T) == 2)) && !has_res && vec_ok &&
      !g.loop && g.exact && g.wpr >= 5 && g.wpr <= 7 && tun.fwd_wpr <= 0) {
    const int64_t per4 = (nvec + 4 * kWave - 1) / (4 * kWave);
    const int v4 = next_pow2(static_cast<int>(per4));
    const int64_t slots = static_cast<int64_t>(v4) * 4 * kWave;
    if (v4 <= cap && (slots - nvec) * 8 <= slots) {
      g.wpr = 4;
      g.vpl = v4;
      g.exact = false;
      g.threads = 256;
    }
  }
  // 16-bit rows (every flavour but MX outputs without a residual), rows enough to fill the device:
  // an exact tiling of 3, 5, 6 or 7 vectors per lane over 1-4 waves (the fewest waves that tile
  // the row, among the shapes each flavour measured faster with) replaces a power-of-two tiling
  // that masks more than 1/16 of its slots or spreads the row over more waves.  Measured on
  // MI355X, bf16, us (waves x vectors per lane; "m": masked):
  //   LN / RMSNorm: 1536 (1x3) 69.7 -> 65.6 against 1x4m; 2560 (1x5) 62.0 -> 56.1 against 2x4m;
  //     3072 (2x3) 157.4 -> 140.0 against 3x2 (1x6: 145.4); 3584 (1x7) 169.0 -> 160.8 against
  //     2x4m; 4608 (3x3) 57.4 -> 55.0 against 4x4m; 5120 (2x5) 60.0 -> 58.5 against 5x2; 6144
  //     (4x3) 70.7 -> 69.1 against 3x4 (2x6: 71.2).  Kept: 7168 (7x2 157.3, 2x7 167.4), 10240
  //     (10x2 56.7, 4x5 58.5), 7680 (4x4m with 1/16 masked: 86.4, 3x5 85.7).
  //   LN -> fp8: 1536 (1x3) 56.8 -> 54.0; 2560 (1x5) 104.6 -> 88.8; 3072 (1x6) 126.6 -> 105.5
  //     (2x3 107.4); 3584 (1x7) 64.4 -> 58.1; 4608 (3x3) 102.5 -> 88.4; 5120 (2x5) 101.2 ->
  //     88.0; 6144 (2x6) 112.6 -> 107.4; 7168 (2x7, C5) 125.1 -> 120.2 against the masked 4-wave
  //     tiling (one 256-thread block per CU; 2 blocks 125.3, 128-thread blocks 126.5-152.5);
  //     10240 (4x5) 97.5 -> 86.9 against 10x2.  Kept: 7680 (4x4m 128.8, 3x5 139.8).
  //   LN + GELU tanh / erf: 1536 (1x3) 75.1 -> 72.7 / 84.2 -> 74.5; 2560 (1x5) 75.5 -> 57.1 /
  //     84.1 -> 60.9; 3072 (1x6) 161.9 -> 132.8 / 166.5 -> 146.3 (2x3 145.6 / 151.7); 3584 tanh
  //     (1x7) 44.0 -> 42.4 (erf 46.3 -> 54.9: kept); 4608 tanh (3x3) 74.5 -> 61.0 (the erf
  //     table needs 256 threads); 5120 (2x5) 76.4 -> 59.8 / 72.6 -> 62.7; 6144 (4x3) 74.4 ->
  //     72.5 / 101.9 -> 77.0 (2x6 75.0 / 79.2); 7168 (2x7) 85.9 -> 82.8 / 93.0 -> 89.4 against
  //     the masked 4-wave tiling.
  //   Residual + LN / residual + RMSNorm -> fp8 / -> MXFP8, 3 and 5 vectors per lane only
  //     (6 and 7 need AGPRs at one wave per SIMD: residual + RMSNorm -> fp8 at 7168 (2x7) 283.1
  //     -> 289.9, MXFP8 274.7 -> 281.5): 1536 (1x3) 143.7 -> 133.6 / 124.9 -> 116.9; 2560 (1x5)
  //     121.3 -> 115.7 / 109.2 -> 97.6 / 104.9 -> 98.5; 3072 (2x3) 140.3 -> 139.0 / 133.9 ->
  //     125.1 / 125.7 -> 118.1; 4608 (3x3) 110.1 -> 100.1 / 97.1 -> 95.4; 5120 (2x5) residual +
  //     RMSNorm -> fp8 106.9 -> 104.1 (kept: residual + LN 113.7 / 114.5, MX 94.3 / 96.7); 6144
  //     (4x3) 144.2 -> 139.0 / MX 122.8 -> 117.9 (kept: -> fp8 123.5 / 124.6).
  // MX outputs without a residual keep the power-of-two tiles.
  if (VV == 8 && vec_ok && !g.loop && (FP8 != 2 || has_res) && (gelu == 0 || FP8 == 0) &&
      tun.fwd_wpr <= 0) {
    const int64_t slots = static_cast<int64_t>(g.wpr) * kWave * g.vpl;
    const bool well_tiled = !g.exact && (slots - nvec) * 16 <= slots;
    auto shape_ok = [&](int w, int v) {
      if (has_res)
        return FP8 == 1 ? ((v == 3 && w <= 3) || (v == 5 && w <= 2))
                        : (v == 3 || (v == 5 && w == 1));
      if (gelu != 0)
        return v == 3 ? (gelu == FLN_GELU_TANH || w != 3)
             : v == 5 ? w <= 2
             : v == 6 ? w == 1
                      : (w == 2 || (w == 1 && gelu == FLN_GELU_TANH));
      if (FP8 == 1) return w <= 2 || v <= 5;
      return v == 3 || (v == 5 && w <= 3) || (v == 7 && w == 1);
    };
    int w_odd = 0, v_odd = 0;
    for (int w = 1; w <= 4 && w_odd == 0 && !well_tiled; ++w) {
      for (const int v : {3, 5, 6, 7}) {
        if (shape_ok(w, v) && nvec == static_cast<int64_t>(w) * kWave * v) {
          w_odd = w;
          v_odd = v;
          break;
        }
      }
    }
    if (w_odd > 0 && rows * w_odd >= 4 * cus) {
      g.wpr = w_odd;
      g.vpl = v_odd;
      g.exact = true;
      g.threads = (4 % w_odd == 0) ? 256 : kWave * w_odd;
    }
  }
  // fp32 tiles of 8 vectors (32 floats) per lane -- rows of 2048, 4096, 6144 or 8192 columns
  // over 1-4 waves -- with rows enough for 32 waves per CU at half the vectors: twice the waves,
  // 4 vectors per lane.  LayerNorm / RMSNorm from 64 rows per CU at 8192 columns, LN + GELU from
  // 32; residual + LayerNorm / RMSNorm up to 6144 columns and from 64 waves per CU; not the fp8
  // outputs (tied: LN -> fp8 8192 x 4096 31.2 / 30.9, 16384 x 2048 30.8 / 30.8).  us, rows x
  // columns, 8 -> 4 vectors per lane:
  //   LayerNorm: 4096 x 2048 14.06 -> 13.27, 8192 x 2048 24.48 -> 23.87, 16384 x 2048 46.15 ->
  //     44.54; 2048 x 4096 14.08 -> 13.68, 4096 x 4096 24.53 -> 24.14, 8192 x 4096 45.28 ->
  //     44.77, 16384 x 4096 89.89 -> 87.45; 2048 x 6144 19.78 -> 19.36, 4096 x 6144 36.07 ->
  //     35.63, 8192 x 6144 69.80 -> 68.79, 16384 x 6144 140.56 -> 138.10; 16384 x 8192 (8
  //     waves, a 512-thread block) 186.03 -> 179.87.  Kept: 1024 x 2048 5.13 / 5.41, 2048 x
  //     2048 7.22 / 7.76, 1024 x 4096 7.42 / 7.94, 1024 x 6144 11.57 / 11.59, 4096 x 8192
  //     45.41 / 45.72, 8192 x 8192 89.74 / 89.84.
  //   LN + GELU tanh / erf: 2048 x 4096 14.94 -> 13.78 / 14.70 / 14.77, 8192 x 4096 46.25 ->
  //     45.10 / 50.93 -> 47.13, 4096 x 2048 erf 15.99 -> 14.69, 2048 x 6144 tanh 20.01 ->
  //     19.82, 8192 x 8192 erf 98.00 -> 91.22, 16384 x 8192 tanh 186.83 -> 179.58.
  //   Residual + LayerNorm: 8192 x 4096 94.99 -> 88.68, 16384 x 2048 94.67 -> 90.28.  Kept:
  //     2048 x 4096 25.11 / 24.36 and 2048 x 6144 36.02 / 35.28 (gains below 64 waves per CU),
  //     4096 x 2048 23.75 / 24.22, 16384 x 8192 406.3 / 443.6 (8 waves).
  // The halved tiles hold 64 bytes of the row per lane, as the 16-bit 4-vector tiles do; those
  // lose when halved (bf16 65536 x 2048 86.7 -> 98.4, 32768 x 4096 87.6 -> 99.2; LN -> fp8
  // 32768 x 4096 68.3 -> 80.2).
  if (VV == 4 && vec_ok && !g.loop && FP8 == 0 && tun.fwd_wpr <= 0 && tun.fwd_epl <= 0 &&
      g.exact && g.vpl == 8 && g.wpr <= 4) {
    const int64_t halved_waves = rows * 2 * g.wpr;
    const bool take = has_res ? g.wpr <= 3 && halved_waves >= 64 * cus
                              : halved_waves >= 32 * cus &&
                                    (g.wpr <= 3 || rows >= (gelu != 0 ? 32 : 64) * cus);
    if (take) {
      g.wpr *= 2;
      g.vpl = 4;
      g.threads = (4 % g.wpr == 0) ? 256 : kWave * g.wpr;
    }
  }
  // fp32 LayerNorm / RMSNorm rows of 8192 columns with 2-8 rows per CU (the reference's
  // large-row table has 1024 x 8192): 16 waves x 2 vectors per lane in a 1024-thread block, two
  // rows of loads ahead, instead of 4 waves x 8 vectors with one.  us: 512 rows 7.54 -> 7.27,
  // 1024 rows 14.12 -> 12.31, 1536 rows 19.39 -> 18.22, 2048 rows 24.7 -> 24.1; 4096 rows
  // 45.5 / 45.6.  Other fp32 widths gained less or lost (1024 x 6144 11.57 -> 11.39, 1024 x
  // 4096 7.44 -> 8.56, 1024 x 12288 18.16 -> 19.56).
  if (VV == 4 && vec_ok && !g.loop && !has_res && gelu == 0 && FP8 == 0 && tun.fwd_wpr <= 0 &&
      nvec == 16 * kWave * 2 && rows >= 2 * cus && rows <= 8 * cus) {
    g.wpr = 16;
    g.vpl = 2;
    g.exact = true;
    g.threads = 16 * kWave;
  }
  // Rows past the register tiles: the LDS-staged kernel on the vector path (up to 8 vectors
  // per thread of a 1024-thread block; LayerNorm / RMSNorm and LN + GELU -- tanh, or erf in
  // fp32 -- with half of each row in registers up to twice that), the streamed wide-row kernel
  // otherwise (buffer resources span at most 4 GiB: rows of 2 GiB or more keep the looped
  // kernel).
  const bool lds = g.loop && vec_ok && nvec <= int64_t(kFwdLdsCpt) * kFwdLdsThreads &&
                   !tun.fwd_no_lds;
  bool lds_reg = false;
  if constexpr (FP8 == 0)
    lds_reg = g.loop && !lds && vec_ok && !has_res && (gelu != FLN_GELU_ERF || sizeof(T) == 4) &&
              nvec <= int64_t(2 * kFwdLdsCpt) * kFwdLdsThreads && !tun.fwd_no_lds;
  const bool wide = g.loop && !lds && !lds_reg && N * int64_t(sizeof(T)) < (int64_t(1) << 31) &&
                    !tun.fwd_no_wide;
  // Fewer rows than CUs (16-bit / fp32 output): each row split over several blocks, its
  // statistics handed over through the head of its own y row (so y may overlap no input).
  // Against the kernels that read x once (LDS-staged, with or without half the row in
  // registers) the split's second read pays only with very few rows (bf16, us: 32 x 131072
  // 19.5 -> 11.7, 64 x 131072 19.8 -> 16.2, 64 x 65536 11.0 against 11.6, 128 x 131072 21.6 /
  // 21.6).  Against the streamed kernel, which reads x as often, it pays until that kernel's
  // one or two rows per CU balance (200 x 262144 64.4 -> 51.9, 300 x 262144 106.0 -> 74.0,
  // 512 x 262144 131.6 -> 125.4, 1024 x 262144 271.5 / 271.3, fp32 600 x 65544 93.4 -> 83.5),
  // for fp8 outputs only below 1.5 blocks per CU (LN -> fp8 300 x 262144 118.2 -> 94.8, 512 x
  // 140000 84.2 against 94.6; MX 400 x 262144 116.7 against 119.6).  Splitting rows past a
  // quarter of the CUs on the LDS-staged routes gains nothing even where their last round runs
  // part-empty (300 x 65536 21.0 against 23.1, 1638 x 40960 68.4 / 68.4, 682 x 98304 64.7 /
  // 64.7: FLN_FWD_SPLIT_ROWS overrides the row limit).
  const int64_t max_rows = tun.fwd_split_rows > 0 ? tun.fwd_split_rows
                           : (lds || lds_reg)    ? cus / 4 - 1
                           : FP8                 ? cus * 3 / 2 - 1
                                                 : 4 * cus - 1;
  const int64_t pbytes = N * static_cast<int64_t>(sizeof(T));
  const bool split = g.loop && vec_ok && y_ok && rows <= max_rows &&
                     pbytes < (int64_t(1) << 31) && !tun.fwd_no_split;
  pl.route = split ? FLN_ROUTE_SPLIT : lds ? FLN_ROUTE_LDS : lds_reg ? FLN_ROUTE_LDS_REG
           : wide  ? FLN_ROUTE_WIDE  : g.loop ? FLN_ROUTE_LOOP : FLN_ROUTE_REGISTERS;
  if (pl.route == FLN_ROUTE_REGISTERS) {
    // The exact-GELU kernels fill their LDS table with one entry per thread: rows of three
    // waves (192 threads) take two row groups per block.
    if (gelu == FLN_GELU_ERF)
      while (g.threads < kGeluLogTabN) g.threads *= 2;
  } else {
    g.wpr = g.vpl = 0;
    g.exact = false;
    g.threads = pl.route == FLN_ROUTE_SPLIT ? 256
              : pl.route == FLN_ROUTE_LOOP  ? (N >= 4096 ? 1024 : 256)
                                            : 1024;
  }
  pl.g = g;
  return pl;
}

// The plan of a contiguous, 16-byte aligned call whose y overlaps no input (fln_forward_plan).
template <class T>
int plan_query(int64_t rows, int64_t cols, int fp8, bool res, int gelu, int64_t cus,
               fln_forward_plan_t* out) {
  constexpr int VV = 16 / sizeof(T);
  const bool vec_ok = cols % VV == 0;
  const bool y_ok = fp8 == 0 || cols % 16 == 0;
  const FwdPlan pl = fp8 == 0 ? plan_typed<T, 0>(rows, cols, res, gelu, vec_ok, y_ok, cus)
                   : fp8 == 1 ? plan_typed<T, 1>(rows, cols, res, gelu, vec_ok, y_ok, cus)
                              : plan_typed<T, 2>(rows, cols, res, gelu, vec_ok, y_ok, cus);
  out->route = pl.route;
  out->vector_elems = pl.vec;
  out->waves_per_row = pl.g.wpr;
  out->vectors_per_lane = pl.g.vpl;
  out->exact = pl.g.exact ? 1 : 0;
  out->threads = pl.g.threads;
  return FLN_OK;
}

inline const char* route_name(int route) {
  switch (route) {
    case FLN_ROUTE_REGISTERS: return "registers";
    case FLN_ROUTE_LDS: return "lds";
    case FLN_ROUTE_LDS_REG: return "lds+registers";
    case FLN_ROUTE_WIDE: return "wide";
    case FLN_ROUTE_SPLIT: return "split";
    default: return "loop";
  }
}

template <class T, int FP8>
int dispatch_typed(FwdParams p, hipStream_t s) {
  constexpr int VV = 16 / sizeof(T);  // elements per 16-byte vector
  const int64_t N = p.cols;
  bool vec_ok = (N % VV == 0) && aligned16(p.x) && aligned16(p.gamma) && aligned16(p.beta) &&
                aligned16(p.res) && aligned16(p.h);
  if (FP8)
    vec_ok = vec_ok && (reinterpret_cast<uintptr_t>(p.y) % VV == 0);
  else
    vec_ok = vec_ok && aligned16(p.y);
  // The split forward hands each row's chunk statistics over through the head of its own y row:
  // y may overlap no input, and fp8 codes need 16-byte aligned rows for the float4 triples.
  const int64_t bytes = p.rows * N * static_cast<int64_t>(sizeof(T));
  const int64_t ybytes = FP8 ? p.rows * N : bytes;
  const int64_t pbytes = N * static_cast<int64_t>(sizeof(T));
  const bool y_ok = (FP8 == 0 || (N % 16 == 0 && aligned16(p.y))) &&
                    !overlaps(p.y, ybytes, p.x, bytes) && !overlaps(p.y, ybytes, p.res, bytes) &&
                    !overlaps(p.y, ybytes, p.h, bytes) && !overlaps(p.y, ybytes, p.gamma, pbytes) &&
                    !overlaps(p.y, ybytes, p.beta, pbytes);
  const FwdPlan pl = plan_typed<T, FP8>(p.rows, N, p.res != nullptr, p.gelu, vec_ok, y_ok,
                                        device_cu_count());
  if (tuning().debug_geometry)
    fprintf(stderr, "fln forward: rows=%lld cols=%lld vec=%d cap=%d/%d -> %s wpr=%d vpl=%d "
            "exact=%d threads=%d\n", static_cast<long long>(p.rows), static_cast<long long>(N),
            pl.vec, pl.cap, pl.wide_cap, route_name(pl.route), pl.g.wpr, pl.g.vpl,
            static_cast<int>(pl.g.exact), pl.g.threads);
  switch (pl.route) {
    case FLN_ROUTE_SPLIT: return launch_split<T, FP8, VV>(p, s);
    case FLN_ROUTE_LDS: return launch_lds<T, FP8, VV>(p, s);
    case FLN_ROUTE_LDS_REG:
      if constexpr (FP8 == 0) return launch_lds_reg<T, VV>(p, s);
      return FLN_ERR_INVALID;  // not planned for fp8 outputs
    case FLN_ROUTE_WIDE:
      return vec_ok ? launch_wide<T, FP8, VV>(p, s) : launch_wide<T, FP8, 1>(p, s);
    case FLN_ROUTE_LOOP: return launch_loop<T, float, FP8>(p, s);
    default: break;
  }
  p.wpr = pl.g.wpr;
  if (vec_ok) return launch_reg_flavour<T, FP8, VV>(p, pl.g.vpl, pl.g.exact, pl.g.threads, s);
  return launch_reg_flavour<T, FP8, 1>(p, pl.g.vpl, false, pl.g.threads, s);
}

}  // namespace detail

}  // namespace fln
