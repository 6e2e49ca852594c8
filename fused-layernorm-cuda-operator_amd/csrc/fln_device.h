// fln_device.h -- device-side building blocks shared by the forward and backward kernels.
//
// Everything here is written for CDNA4 (gfx950) wave64: cross-lane sums use DPP row
// permutations inside each 16-lane row, ds_swizzle across the two rows of a 32-lane half, and
// v_readlane across the halves, so a reduction never touches LDS unless a row of the tensor is
// spread over several waves.  The reference's warp32 shuffle tree and its shared-memory block
// step (csrc/layernorm_cuda_kernel.cu:7-28) play the same role there.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fln_gelu_table.h"

namespace fln {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------------
// Element types.  __bf16 / _Float16 are clang's native storage types: widening is exact and the
// narrowing cast lowers to v_cvt_pk_bf16_f32 (round-to-nearest-even) on gfx950.
// ---------------------------------------------------------------------------------------------
template <class T> __device__ __forceinline__ float to_f32(T v) { return static_cast<float>(v); }
template <class T> __device__ __forceinline__ T from_f32(float v) { return static_cast<T>(v); }

template <class T, int N> struct alignas(sizeof(T) * N) Pack {
  T v[N];
};

// Makes a packed value opaque to the optimizer for one use site.  Applied inside a row loop to
// loop-invariant 16-bit parameter packs, it stops the compiler from hoisting their widening to
// fp32 out of the loop (which would double their VGPR footprint and cost occupancy).
template <class T, int N> __device__ __forceinline__ void keep_packed(Pack<T, N>& p) {
  if constexpr (sizeof(T) == 2 && (sizeof(Pack<T, N>) % 4) == 0) {
    constexpr int W = sizeof(Pack<T, N>) / 4;
    struct Words {
      uint32_t w[W];
    };
    Words u = __builtin_bit_cast(Words, p);
#pragma unroll
    for (int k = 0; k < W; ++k) asm volatile("" : "+v"(u.w[k]));
    p = __builtin_bit_cast(Pack<T, N>, u);
  }
}

template <class T, int N> __device__ __forceinline__ Pack<T, N> zero_pack() {
  Pack<T, N> p;
#pragma unroll
  for (int e = 0; e < N; ++e) p.v[e] = static_cast<T>(0.0f);
  return p;
}

// ---------------------------------------------------------------------------------------------
// Raw buffer access.  A buffer resource (V#) describes [base, base + nbytes); a raw buffer load
// whose byte offset falls outside returns zeros and such a store is dropped, by the hardware.
// The kernels build one resource per row (nbytes = 0 for a row past the end of the tensor), so
// tails, missing rows and absent tensors need no branches -- which keeps the compiler's wait-count
// bookkeeping exact and lets a row's prefetch stay in flight across the loop.
// Word 3 of the V# is 0x00020000 on gfx9-family targets (raw, untyped access).
// ---------------------------------------------------------------------------------------------
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr uint32_t kOutOfRange = 0x80000000u;  // an offset no resource here reaches

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                           base ? static_cast<int>(nbytes) : 0, 0x00020000);
}

// Cache policy: the last operand of the raw buffer builtins (gfx950 CPol bits: 1 = sc0,
// 2 = nt, 16 = sc1).  0 is the default policy; kStream (nt) marks data touched once, so it is
// not kept in the caches at the expense of data that is reused.
constexpr int kDefault = 0;
constexpr int kStream = 2;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int BYTES, int POL = kDefault> struct BufIO;
template <int POL> struct BufIO<16, POL> {
  using W = u32x4;
  __device__ static W load(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL);
  }
  __device__ static void store(W w, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, POL);
  }
};
template <int POL> struct BufIO<8, POL> {
  using W = u32x2;
  __device__ static W load(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POL);
  }
  __device__ static void store(W w, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b64(w, r, off, 0, POL);
  }
};
template <int POL> struct BufIO<4, POL> {
  using W = uint32_t;
  __device__ static W load(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL);
  }
  __device__ static void store(W w, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b32(w, r, off, 0, POL);
  }
};
template <int POL> struct BufIO<2, POL> {
  using W = uint16_t;
  __device__ static W load(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, POL);
  }
  __device__ static void store(W w, rsrc_t r, uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b16(w, r, off, 0, POL);
  }
};

// Load / store the v-th Pack of a resource (byte offset v * sizeof(P)).
template <class P, int POL = kDefault>
__device__ __forceinline__ P buf_load(rsrc_t r, uint32_t v) {
  using IO = BufIO<sizeof(P), POL>;
  return __builtin_bit_cast(P, IO::load(r, v * static_cast<uint32_t>(sizeof(P))));
}
template <class P, int POL = kDefault>
__device__ __forceinline__ void buf_store(const P& p, rsrc_t r, uint32_t v) {
  using IO = BufIO<sizeof(P), POL>;
  IO::store(__builtin_bit_cast(typename IO::W, p), r, v * static_cast<uint32_t>(sizeof(P)));
}
__device__ __forceinline__ void buf_store_f32(float x, rsrc_t r, uint32_t byte_off) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), r, byte_off, 0, 0);
}

// ---------------------------------------------------------------------------------------------
// Wave64 all-reduce.  After the four DPP steps every lane of a 16-lane row holds that row's
// total; ds_swizzle (xor 16) combines the two rows of each 32-lane half; two readlanes combine
// the halves into a wave-uniform value.  Every combining step adds a value to its mirror image,
// so all lanes end with the bitwise-identical result (fp add is commutative).
// All 64 lanes must be active when these are called.
// ---------------------------------------------------------------------------------------------
template <int CTRL> __device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swz_xor16(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float readlane(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

struct SumOp {
  __device__ __forceinline__ static float apply(float a, float b) { return a + b; }
};
// Maximum of non-negative floats (every maximum reduced here is of |value|): their IEEE bit
// patterns order like unsigned integers, so v_max_u32 gives the same result without the NaN
// canonicalization fmaxf costs (one extra VALU op per step); a NaN propagates, as in amax.
// Written as the umax builtin: the DPP operand then folds into one v_max_u32_dpp per step
// (the equivalent `x > y ? x : y` compiles to v_mov_dpp + v_cmp + v_cndmask and a wait state).
__device__ __forceinline__ float max_nonneg(float a, float b) {
  const uint32_t x = __builtin_bit_cast(uint32_t, a), y = __builtin_bit_cast(uint32_t, b);
  return __builtin_bit_cast(float, __builtin_elementwise_max(x, y));
}
struct MaxOp {
  __device__ __forceinline__ static float apply(float a, float b) { return max_nonneg(a, b); }
};

template <class Op> __device__ __forceinline__ float wave_allreduce(float v) {
  v = Op::apply(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]: lane ^ 1
  v = Op::apply(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]: lane ^ 2
  v = Op::apply(v, dpp<0x141>(v));  // row_half_mirror: 4-lane groups within 8
  v = Op::apply(v, dpp<0x140>(v));  // row_mirror: 8-lane groups within 16
  v = Op::apply(v, swz_xor16(v));   // 16-lane rows within 32
  return Op::apply(readlane(v, 0), readlane(v, 32));
}

// Reduce the values of lanes 0..15 (the first 16-lane row) in a fixed order with four DPP
// steps; the result is wave-uniform.
template <class Op> __device__ __forceinline__ float reduce16(float v) {
  v = Op::apply(v, dpp<0xB1>(v));
  v = Op::apply(v, dpp<0x4E>(v));
  v = Op::apply(v, dpp<0x141>(v));
  v = Op::apply(v, dpp<0x140>(v));
  return readlane(v, 0);
}

// Combine the per-wave partials slot[base .. base + n - 1] (n <= 16) of one row group: lane k
// reads partial k (one LDS read per lane, all in parallel), lanes k >= n contribute `ident`, and
// reduce16 combines them; the result is wave-uniform.  slot must be readable up to base + 15
// (callers pad it).
template <class Op>
__device__ __forceinline__ float combine_partials(const float* slot, int base, int n, int lane,
                                                  float ident) {
  const int k = lane & 15;
  float v = slot[base + k];
  v = k < n ? v : ident;
  return reduce16<Op>(v);
}

// Generic-type wave sum through ds_bpermute (used by the looped fallback kernels, which also
// handle fp64 accumulation).
template <class A> __device__ __forceinline__ A wave_sum_generic(A v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// ---------------------------------------------------------------------------------------------
// GELU.  mode 1: exact erf form (torch approximate='none'); mode 2: tanh form, the one fused by
// the reference (csrc/layernorm_cuda_kernel.cu:31-36).
//
// The tanh form is evaluated through the identity 0.5 v (1 + tanh(u)) = v sigmoid(2u) =
// v / (1 + e^(-2u)), u = sqrt(2/pi) (v + 0.044715 v^3): one hardware exp2 (v_exp_f32) and one
// hardware reciprocal (v_rcp_f32) instead of a tanh, and no cancellation for large negative v
// (the quotient stays relatively accurate where 1 + tanh(u) would cancel).  Its derivative is
//   s + 2 v s (1 - s) sqrt(2/pi) (1 + 3 * 0.044715 v^2),   s = sigmoid(2u).
// The erf form is v Phi(v) with Phi the standard normal CDF, and its derivative
//   Phi(v) + v exp(-v^2 / 2) / sqrt(2 pi);
// erfc_terms() below gives both from one hardware exp2 and one hardware reciprocal.
// ---------------------------------------------------------------------------------------------
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kGeluK0 = 0.79788456080286535588f;  // sqrt(2/pi)
constexpr float kGeluK1 = 0.044715f;

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// For the tanh form, u = sqrt(2/pi) (v + k1 v^3): e = e^(-2u) and sigmoid(2u) = 1 / (1 + e);
// 1 - sigmoid(2u) = e / (1 + e) is formed as a product, not a difference (no cancellation where
// the sigmoid approaches 1).  The exponent -2u log2(e) is v (c0 + c1 v^2) with the constants
// folded (c0 = -2 sqrt(2/pi) log2(e), c1 = c0 k1): one multiply, one FMA and one multiply.
struct GeluTanhTerms {
  float e, sg;
};
__device__ __forceinline__ GeluTanhTerms gelu_tanh_terms(float v) {
  constexpr float kC0 = -2.0f * 0.79788456080286535588f * 1.44269504088896340736f;
  constexpr float kC1 = kC0 * 0.044715f;
  const float e = exp2_fast(v * fmaf(kC1, v * v, kC0));
  return {e, __builtin_amdgcn_rcpf(1.0f + e)};  // v_rcp_f32: 1 ulp
}
__device__ __forceinline__ float gelu_tanh_sigmoid(float v) { return gelu_tanh_terms(v).sg; }

// The erf form.  With x = |v| / sqrt 2 and t = 1 / (1 + 0.35 x),
//   h = 0.5 erfc(x) = t F(t) exp(-x^2),
// where F(t) = 0.5 erfcx(x) / t (erfcx(x) = exp(x^2) erfc(x)) is smooth on t in (0, 1] and is
// replaced by a degree-7 polynomial: a relative-error least-squares fit on Chebyshev nodes, max
// relative error 8.3e-7 (fit_erfc.py beside this file derives and checks the coefficients).
// Phi(v) = h for v < 0 and 1 - h otherwise, so
//   GELU(v)  = v Phi(v) = max(v, 0) - |v| h
//   GELU'(v) = Phi(v) + v exp(-v^2 / 2) / sqrt(2 pi) = 1/2 + sign(v) (1/2 - exp(-x^2) w),
//   w = t F(t) - |v| / sqrt(2 pi)
// (for v >= 0 it is 1 - e w, for v < 0 it is e w: Phi and v phi(v) share the Gaussian factor).
// GELU is a difference only where v >= 0 and then at most v / 2 is taken off, so its lower tail
// keeps the relative accuracy of h where 0.5 v (1 + erf(v / sqrt 2)) cancels; the derivative's
// error is absolute (about one ulp of 1/2 in the tail, like that of Phi + v phi in fp32).
// Each costs one hardware exp2 (v_exp_f32), one hardware reciprocal (v_rcp_f32), seven FMAs
// for F and four (GELU) or five (derivative) more VALU operations.  Under an fp32 emulation
// over |v| <= 13: GELU within 2.4e-7 (absolute) and 6.9e-6 (relative, |GELU| > 1e-30) of the
// float64 value, the derivative within 5.6e-7.  GELU(+inf) = +inf, GELU(-inf) = 0; NaN
// propagates.
struct ErfcTerms {
  float t, e, f;  // t, exp(-v^2 / 2), F(t)
};
// F(t), Horner form.
__device__ __forceinline__ float erfc_poly(float t) {
  constexpr float kF[8] = {9.873314202e-02f, 9.872655571e-02f, 9.295467287e-02f,
                           7.733605057e-02f, 8.147227019e-02f, -7.275486365e-03f,
                           1.006051227e-01f, -4.255273566e-02f};
  float f = kF[7];
#pragma unroll
  for (int k = 6; k >= 0; --k) f = fmaf(f, t, kF[k]);
  return f;
}
__device__ __forceinline__ ErfcTerms erfc_terms(float v) {
  const float e = exp2_fast((-0.5f * kLog2e * v) * v);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.35f * 0.70710678118654752440f, fabsf(v), 1.0f));
  return {t, e, erfc_poly(t)};
}
// |a| * b with 0 * anything = 0 (v_mul_legacy_f32): |v| (t e) stays 0 at v = +-inf, where
// t e = 0.  Neither operand may be the direct result of a transcendental instruction (v_rcp,
// v_exp, ...): a VALU read of such a result needs a wait state, which the compiler does not
// insert in front of inline assembly.  Callers pass an affine output and a v_mul product.
__device__ __forceinline__ float abs_mul_zero_wins(float a, float b) {
  float r;
  asm("v_mul_legacy_f32 %0, |%1|, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float gelu_erf(float v) {
  const ErfcTerms k = erfc_terms(v);
  return fmaf(-abs_mul_zero_wins(v, k.t * k.e), k.f, fmaxf(v, 0.0f));
}
__device__ __forceinline__ float gelu_tanh(float v) { return v * gelu_tanh_sigmoid(v); }
__device__ __forceinline__ float gelu_erf_grad(float v) {
  constexpr float kInvSqrt2Pi = 0.39894228040143267794f;
  const ErfcTerms k = erfc_terms(v);
  const float w = fmaf(-kInvSqrt2Pi, fabsf(v), k.t * k.f);
  return 0.5f + __builtin_copysignf(fmaf(-k.e, w, 0.5f), v);
}
// GELU' from a table, for the backward's register kernel (where evaluating the formulas above
// is most of the per-element VALU work).  For either form, T(v) = 2 GELU'(v) - 1 is odd, smooth,
// and within 1e-7 of its limit +-1 past |v| = 6 (erf form: erf(v / sqrt 2) + v sqrt(2 / pi)
// exp(-v^2 / 2); tanh form: tanh(u) + v u'(v) sech^2(u)).  Interval k of kGeluTabData /
// kGeluTanhTabData (fln_gelu_table.h, generated by fit_erfc.py) covers |v| in [k h, (k + 1) h),
// h = 6 / 255, and holds the quadratic through T at its ends and middle, c0 + c1 f + c2 f^2 with
// f in [0, 1) the position in the interval; the last interval (|v| >= 6) is the constant 1.
// Built in float64 and rounded to fp32, the lookup is within 2.1e-7 of GELU' for both forms (the
// erf polynomial: 5.6e-7).  A lookup is one multiply-add (the caller forms u = v / h from
// gamma / h and beta / h), fract, min, convert, shift, one ds_read_b128 from the block's LDS
// copy, two FMAs and a copysign: no transcendental instruction.
constexpr float kGeluTabInvH = (kGeluTabN - 1) / kGeluTabMax;  // 42.5: u = v / h

// sign(v) T(|v|) for u = v / h: 2 GELU'(v) = 1 + the result (NaN propagates through fract; so
// does an infinite u, as with the formulas above).
__device__ __forceinline__ float gelu_grad2_sign_tab(const float4* tab, float u) {
  const float au = fabsf(u);
  const float f = __builtin_amdgcn_fractf(au);
  const uint32_t k = static_cast<uint32_t>(fminf(au, static_cast<float>(kGeluTabN - 1)));
  const float4 c = tab[k];
  return __builtin_copysignf(fmaf(fmaf(c.z, f, c.y), f, c.x), u);
}
// The exact GELU from a table, for the forward's register kernel: with x = |v|,
// GELU(v) = max(v, 0) - x Phi(-x), and L(x) = log2(Phi(-x)) is smooth, so interval k of
// kGeluLogTabData (fln_gelu_table.h, generated by fit_erfc.py) holds the quadratic through
// L - 4 at the ends and middle of x in [k / 16, (k + 1) / 16) (the last interval, x >= 255 / 16,
// is -inf: Phi(-x) is far below the fp32 range there).  With uc = min(16 x, 255) (exact: the
// interval width is a power of two), GELU = fma(-uc, 2^L, max(v, 0)).  The product keeps the
// relative accuracy of Phi(-x) in the lower tail; under an fp32 emulation over |v| <= 13.5 it is
// within 2.4e-7 (absolute) and 5.3e-6 (relative, |GELU| > 1e-30) of the float64 GELU, as the
// polynomial is.  One multiply, min, fract, convert, shift, one ds_read_b128 from the block's LDS
// copy, two FMAs, one v_exp_f32, a NaN-propagating maximum (v_maximum3_f32) and one FMA:
// 9 VALU operations and one transcendental (the polynomial: 14 and two).  NaN propagates,
// GELU(+inf) = +inf, GELU(-inf) = 0.
__device__ __forceinline__ float gelu_erf_tab(const float4* tab, float v) {
  const float uc = fminf(fabsf(v) * kGeluLogTabInvH, static_cast<float>(kGeluLogTabN - 1));
  const float f = __builtin_amdgcn_fractf(uc);
  const float4 c = tab[static_cast<uint32_t>(uc)];
  const float r = exp2_fast(fmaf(fmaf(c.z, f, c.y), f, c.x));
  return fmaf(-uc, r, __builtin_elementwise_maximum(v, 0.0f));
}

__device__ __forceinline__ float gelu_tanh_grad(float v) {
  const GeluTanhTerms t = gelu_tanh_terms(v);
  // 1 - sigmoid(2u) = e sigmoid(2u), with e kept finite: where e overflows, sigmoid(2u) = 0 and
  // the product must not become inf * 0.
  const float one_minus = fminf(t.e, 3.0e38f) * t.sg;
  // 2 v s (1 - s) sqrt(2/pi) (1 + 3 k1 v^2) + s, the constants folded into one FMA.
  constexpr float kD0 = 2.0f * kGeluK0, kD1 = 2.0f * kGeluK0 * 3.0f * kGeluK1;
  return fmaf(v * fmaf(kD1, v * v, kD0), t.sg * one_minus, t.sg);
}
__device__ __forceinline__ float gelu_grad(float v, int mode) {
  return mode == 1 ? gelu_erf_grad(v) : gelu_tanh_grad(v);
}

template <class A> __device__ __forceinline__ A apply_gelu(A v, int mode) {
  if (mode == 1) return gelu_erf(static_cast<float>(v));
  if (mode == 2) return gelu_tanh(static_cast<float>(v));
  return v;
}
__device__ __forceinline__ double apply_gelu(double v, int mode) {
  if (mode == 1) return 0.5 * v * (1.0 + erf(v * 0.70710678118654752440));
  if (mode == 2) return 0.5 * v * (1.0 + tanh(0.79788456080286535588 * (v + 0.044715 * v * v * v)));
  return v;
}

// ---------------------------------------------------------------------------------------------
// OCP fp8 e4m3fn.  v_cvt_pk_fp8_f32 (gfx950: OCP encoding, round-to-nearest-even) converts two
// fp32 values into two bytes of a dword half.  Values are clamped to +-448 first, so the
// conversion never sees an out-of-range input (saturating semantics).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float sat448(float v) {
  return __builtin_amdgcn_fmed3f(v, -448.0f, 448.0f);
}

// The first conversion writes the low 16 bits and keeps the high ones of its `old` operand,
// which the second conversion then replaces: any register serves as `old` (the first input's
// bits here, which saves the v_mov of a constant).
__device__ __forceinline__ uint32_t fp8x4(float a, float b, float c, float d) {
  const float sa = sat448(a);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(sa, sat448(b), __builtin_bit_cast(int, sa), false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(c), sat448(d), w, true);
  return static_cast<uint32_t>(w);
}
// Without the clamp, for values already known to lie within +-464 (anything in (448, 464)
// rounds to 448 under round-to-nearest-even): a row scaled by 448 / max|row| stays within
// 448 (1 + 2^-23).
__device__ __forceinline__ uint32_t fp8x4_inrange(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return static_cast<uint32_t>(w);
}
// OCP MX (Microscaling v1.0) block scale for E4M3 elements: for a block maximum m, the shared
// exponent is floor(log2 m) - 8 (8 = emax of E4M3), clamped to [-127, 127]; the E8M0 code is
// exponent + 127 (2^(code - 127)), i.e. the maximum's biased exponent field minus 8, at least
// `floor`; elements are v * 2^-exponent, saturated to +-448.  A zero (or subnormal) maximum gives
// code 0.  floor is 0, or 0xFF (E8M0's NaN) for a row whose every block is to read as NaN
// (mx_poison): the clamp the code needs anyway then yields 0xFF at no cost, and the block's codes,
// scaled by the meaningless mul that goes with it, carry no value.
struct MxScale {
  int code;     // E8M0 byte
  float mul;    // 2^-exponent (exact)
};
__device__ __forceinline__ MxScale mx_scale_e4m3(float block_max, int floor = 0) {
  const int eb = static_cast<int>((__builtin_bit_cast(uint32_t, block_max) >> 23) & 0xFF);
  const int code = eb - 8 < floor ? floor : eb - 8;  // <= 247 for finite maxima
  return {code, __builtin_bit_cast(float, (254u - static_cast<uint32_t>(code)) << 23)};
}

// fp8 outputs of a row whose statistics are not usable: a mean that is not finite, or an rstd
// outside (0, inf), which is what a NaN or an infinity in the row, an fp32 sum of squares that
// overflows, or a constant row with eps = 0 leave.  Every output of such a row is meaningless, so
// its row scale is NaN and each of its MX block scales 0xFF, and a reader sees NaN throughout.
// row_poison is +0 for a usable row and NaN otherwise (x - x is NaN exactly for x infinite or
// NaN; 0 * (1 / rstd) is NaN for rstd = 0): added to the row maximum, it leaves a usable row's
// unchanged.  mx_poison is its exponent field, 0 or 0xFF: the floor of each E8M0 block code.
// Tested on the statistics, which stay live through the epilogue anyway, rather than per element:
// the row maximum keeps its two-elements-per-instruction chain (v_max3_f32), whose maxNum
// semantics would drop a NaN.  Every lane of a wave works on one row, so the value is
// wave-uniform: read from the first lane, it lives in an SGPR and costs the epilogue no VGPR.
__device__ __forceinline__ float row_poison(float mean, float rstd) {
  const float p = ((mean - mean) + (rstd - rstd)) + 0.0f * __builtin_amdgcn_rcpf(rstd);
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, p)));
}
__device__ __forceinline__ int mx_poison(float poison) {
  return static_cast<int>((__builtin_bit_cast(uint32_t, poison) >> 23) & 0xFF);
}

// Max over aligned groups of G adjacent lanes (G = 2 ... 32) of non-negative values, result in
// every lane of the group.  All lanes of each group must be active.
template <int G> __device__ __forceinline__ float group_max(float v) {
  static_assert(G >= 2 && G <= 32 && (G & (G - 1)) == 0, "group of 2..32 lanes");
  v = max_nonneg(v, dpp<0xB1>(v));                        // lane ^ 1
  if constexpr (G >= 4) v = max_nonneg(v, dpp<0x4E>(v));   // lane ^ 2
  if constexpr (G >= 8) v = max_nonneg(v, dpp<0x141>(v));  // mirror within 8
  if constexpr (G >= 16) v = max_nonneg(v, dpp<0x140>(v)); // mirror within 16
  if constexpr (G >= 32) v = max_nonneg(v, swz_xor16(v));  // lane ^ 16
  return v;
}

__device__ __forceinline__ uint8_t fp8x1(float a) {
  const float sa = sat448(a);  // low byte: the code of a (the rest of the word is discarded)
  return static_cast<uint8_t>(
      __builtin_amdgcn_cvt_pk_fp8_f32(sa, 0.0f, __builtin_bit_cast(int, sa), false) & 0xFF);
}

}  // namespace fln
