// fln_internal.h -- parameter blocks and host helpers shared by the libfln translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>
#include <tuple>
#include <type_traits>
#include <utility>

#include "../../include/fused_layernorm.h"

namespace fln {

// Forward launch description (one struct for every forward flavour).
struct FwdParams {
  const void* x;
  const void* res;    // residual, or nullptr
  const void* gamma;  // [cols] or nullptr
  const void* beta;   // [cols] or nullptr (LayerNorm only)
  void* y;            // [rows, cols] of dtype, or fp8 bytes when out_fp8
  void* h;            // residual sum output, or nullptr
  float* mean;        // [rows] or nullptr
  float* rstd;        // [rows] or nullptr
  float* scale;       // [rows] fp8 row scales (out_fp8, per-row scaling)
  uint8_t* bscale;    // [rows, cols / 32] E8M0 block scales (out_fp8 with mx)
  int64_t rows;
  int64_t cols;
  float eps;
  int rms;   // 1: RMSNorm (no centring, no beta)
  int gelu;  // FLN_GELU_*
  int mx;    // out_fp8: 0 per-row scale, 1 OCP MX blocks of 32 with E8M0 scales
  int wpr;   // waves per row (register path)
  int splits;           // column chunks per row (few-row split forward)
  int64_t split_chunk;  // vectors per chunk (few-row split forward)
};

// Backward launch description.
struct BwdParams {
  const void* dy;
  const void* x;
  const float* mean;  // LayerNorm only
  const float* rstd;
  const void* gamma;  // or nullptr (treated as ones)
  const void* beta;   // LayerNorm + GELU only: the affine shift GELU was applied after
  const void* dres;   // gradient added into dx, or nullptr
  void* dx;           // or nullptr
  float* part_g;      // [blocks, cols] stage-1 partial of sum(dy * xhat), or nullptr
  float* part_b;      // [blocks, cols] stage-1 partial of sum(dy), or nullptr
  float* rowstat;     // [rows, stat_splits, 2] row sums of g and g xhat over each column
                      // split (two-pass path), in the workspace
  int64_t stat_chunk; // vectors per column split of the row statistics (two-pass path)
  int stat_splits;    // column splits per row of the row statistics (two-pass path)
  void* out_g;        // two-pass path with one block row: dgamma written by the column pass
  void* out_b;        // ... and dbeta (no partial rows, no column reduction)
  int out_dtype;      // their dtype
  int64_t rows;
  int64_t cols;
  int64_t rows_per_block;
  int rms;
  int gelu;  // 0, or the GELU form (1 erf, 2 tanh) applied after the LayerNorm affine step
  int wpr;   // waves per row
  int rgs;   // row groups per block
};

int element_size(int dtype);
int device_cu_count();  // CU count of the current device (256 when no device answers)
int current_device();   // current device index (0..63)

// Caches the current device and its CU count for the duration of an entry point's call, so its
// launch path queries them once (RAII; nests).
class CallDevice {
 public:
  CallDevice();
  ~CallDevice();
  CallDevice(const CallDevice&) = delete;
  CallDevice& operator=(const CallDevice&) = delete;

 private:
  int prev_dev_, prev_cus_;
};

// Launch through a function handle cached per device and instantiation (`cache`: 64 slots,
// static at the call site): hipModuleLaunchKernel skips hipLaunchKernel's lookup of the kernel
// by its host address (MI355X, empty kernel: 2.35 -> 2.18 us of host time per launch).  Falls
// back to hipLaunchKernel if no handle is available.  Arguments are converted to the kernel's
// parameter types before their addresses are taken.
template <class... P, class... A, size_t... I>
int launch_cached_impl(void (*kernel)(P...), std::atomic<void*>* cache, dim3 grid, dim3 block,
                       hipStream_t s, std::index_sequence<I...>, A&&... a) {
  std::tuple<std::remove_cv_t<std::remove_reference_t<P>>...> vals(std::forward<A>(a)...);
  const int dev = current_device();
  void* f = cache[dev].load(std::memory_order_relaxed);
  if (!f) {
    hipFunction_t h = nullptr;
    if (hipGetFuncBySymbol(&h, reinterpret_cast<const void*>(kernel)) == hipSuccess && h) {
      f = reinterpret_cast<void*>(h);
      cache[dev].store(f, std::memory_order_relaxed);
    } else {
      (void)hipGetLastError();
      hipLaunchKernelGGL(kernel, grid, block, 0, s, std::get<I>(vals)...);
      return static_cast<int>(hipGetLastError());
    }
  }
  void* params[] = {static_cast<void*>(&std::get<I>(vals))...};
  return static_cast<int>(hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(f), grid.x,
                                                grid.y, grid.z, block.x, block.y, block.z, 0, s,
                                                params, nullptr));
}

template <class... P, class... A>
int launch_cached(void (*kernel)(P...), std::atomic<void*>* cache, dim3 grid, dim3 block,
                  hipStream_t s, A&&... a) {
  static_assert(sizeof...(P) == sizeof...(A), "one argument per kernel parameter");
  return launch_cached_impl(kernel, cache, grid, block, s, std::index_sequence_for<P...>{},
                            std::forward<A>(a)...);
}
bool aligned16(const void* p);

// FLN_* tuning / debugging environment variables (0 = unset: the built-in default).
struct Tuning {
  int force_loop;      // FLN_FORCE_LOOP: forward through the looped kernel
  int fwd_epl;         // FLN_FWD_EPL: forward elements per lane for rows of up to 4 waves
  int fwd_wpr;         // FLN_FWD_WPR: forward waves per row
  int fwd_grid_mult;   // FLN_FWD_GRID_MULT: forward grid = this many blocks per CU
  int debug_geometry;  // FLN_DEBUG_GEOMETRY: one stderr line per forward launch
  int fwd_no_lds;      // FLN_FWD_NO_LDS: never the LDS-staged forward
  int fwd_no_wide;     // FLN_FWD_NO_WIDE: the looped forward instead of the streamed wide-row one
  int fwd_no_split;    // FLN_FWD_NO_SPLIT: never the few-row split forward
  int fwd_splits;      // FLN_FWD_SPLITS: column chunks per row of the split forward
  int fwd_split_rows;  // FLN_FWD_SPLIT_ROWS: split the forward of up to this many rows
  int bwd_epl;         // FLN_BWD_EPL: backward elements per lane
  int bwd_wpr;         // FLN_BWD_WPR: backward waves per row
  int bwd_threads;     // FLN_BWD_THREADS: backward block size (256, 512, 1024)
  int bwd_grid_mult;   // FLN_BWD_GRID_MULT: backward blocks per CU (1-4)
  int bwd_no_lds;      // FLN_BWD_NO_LDS: never the LDS-staged backward
  int bwd_no_two_pass; // FLN_BWD_NO_TWO_PASS: never the two-pass backward
  int bwd_stat_splits; // FLN_BWD_STAT_SPLITS: column splits per row of the two-pass statistics
  int bwd_colpass_per_cu; // FLN_BWD_COLPASS_PER_CU: column-pass blocks per CU (two-pass path)
};
const Tuning& tuning();  // read at the first call; fln_reload_tuning() reads again
void reload_tuning();

int launch_forward(const FwdParams& p, int dtype, bool out_fp8, hipStream_t s);
// have_workspace: p.part_g points at workspace_bytes of 16-byte aligned workspace; a call whose
// geometry needs more returns FLN_ERR_TOO_LARGE before anything is launched.
int launch_backward(const BwdParams& p, int dtype, void* dgamma, void* dbeta, int dparam_dtype,
                    bool have_workspace, size_t workspace_bytes, hipStream_t s);

// Stage-1 geometry of the backward (shared by workspace sizing and the launch).
struct BwdGeometry {
  bool reg_path;  // register-resident rows
  int lds_cpt;    // > 0: rows staged through LDS, this many vectors per thread (reg_path false)
  bool two_pass;  // row statistics pass + column pass (rows past the register / LDS tiles)
  int vec;        // elements per vector access
  int vpl;        // vectors per lane (power of two, <= 16)
  int wpr;        // waves per row
  int threads;    // block size
  int rgs;        // row groups per block
  int64_t blocks; // stage-1 blocks == partial rows
  int64_t rows_per_block;
};
BwdGeometry backward_geometry(int64_t rows, int64_t cols, int dtype, bool vec_ok, bool dres,
                              bool gelu, bool have_workspace);
// Partial rows the backward workspace holds (an upper bound on every path's stage-1 blocks).
int64_t workspace_partial_rows(int64_t rows);

}  // namespace fln
