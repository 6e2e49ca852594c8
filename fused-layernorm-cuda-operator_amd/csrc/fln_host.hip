// fln_host.hip -- host-only helpers of libfln: device queries, the reference's utility
// functions (csrc/layernorm_cuda.cpp:144-195) and version / error strings.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <stdlib.h>

#include <atomic>
#include <mutex>
#include <string>

#include "fln_internal.h"

namespace fln {

int element_size(int dtype) {
  switch (dtype) {
    case FLN_F32: return 4;
    case FLN_BF16: return 2;
    case FLN_F16: return 2;
    case FLN_F64: return 8;
    case FLN_F8E4M3FN: return 1;
    default: return 0;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// CU count of device `dev`, cached per device index (lock-free after the first query; two
// threads racing on the first query store the same value).
namespace {
int cus_of(int dev) {
  static std::atomic<int> cache[64];
  int cus = cache[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

// The current device while an entry point runs (CallDevice): its launch path asks for the
// device and its CU count a dozen times, and each hipGetDevice costs ~0.05 us.
thread_local int tl_call_dev = -1;
thread_local int tl_call_cus = 0;
}  // namespace

CallDevice::CallDevice() : prev_dev_(tl_call_dev), prev_cus_(tl_call_cus) {
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
    tl_call_dev = dev;
    tl_call_cus = cus_of(dev);
  }
}

CallDevice::~CallDevice() {
  tl_call_dev = prev_dev_;
  tl_call_cus = prev_cus_;
}

int current_device() {
  if (tl_call_dev >= 0) return tl_call_dev;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  return dev;
}

int device_cu_count() {
  if (tl_call_dev >= 0) return tl_call_cus;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  return cus_of(dev);
}

// Tuning and debugging knobs: getenv scans the whole environment (~0.1 us each with ~100
// variables), so the knobs are read once, at the first launch, into a snapshot that
// fln_reload_tuning() replaces.  Replaced snapshots are never freed (a concurrent launch may
// still be reading one; each is 44 bytes and only tests and tuning sweeps reload).
namespace {
int env_knob(const char* name, int dflt) {
  const char* v = getenv(name);
  return (v && *v) ? atoi(v) : dflt;
}

Tuning read_tuning() {
  Tuning t{};
  t.force_loop = env_knob("FLN_FORCE_LOOP", 0);
  t.fwd_epl = env_knob("FLN_FWD_EPL", 0);
  t.fwd_wpr = env_knob("FLN_FWD_WPR", 0);
  t.fwd_grid_mult = env_knob("FLN_FWD_GRID_MULT", 0);
  t.debug_geometry = env_knob("FLN_DEBUG_GEOMETRY", 0);
  t.fwd_no_lds = env_knob("FLN_FWD_NO_LDS", 0);
  t.fwd_no_wide = env_knob("FLN_FWD_NO_WIDE", 0);
  t.fwd_no_split = env_knob("FLN_FWD_NO_SPLIT", 0);
  t.fwd_splits = env_knob("FLN_FWD_SPLITS", 0);
  t.fwd_split_rows = env_knob("FLN_FWD_SPLIT_ROWS", 0);
  t.bwd_epl = env_knob("FLN_BWD_EPL", 0);
  t.bwd_wpr = env_knob("FLN_BWD_WPR", 0);
  t.bwd_threads = env_knob("FLN_BWD_THREADS", 0);
  t.bwd_grid_mult = env_knob("FLN_BWD_GRID_MULT", 0);
  t.bwd_no_lds = env_knob("FLN_BWD_NO_LDS", 0);
  t.bwd_no_two_pass = env_knob("FLN_BWD_NO_TWO_PASS", 0);
  t.bwd_stat_splits = env_knob("FLN_BWD_STAT_SPLITS", 0);
  t.bwd_colpass_per_cu = env_knob("FLN_BWD_COLPASS_PER_CU", 0);
  return t;
}

std::atomic<const Tuning*> g_tuning{nullptr};
std::mutex g_tuning_mu;
}  // namespace

const Tuning& tuning() {
  const Tuning* t = g_tuning.load(std::memory_order_acquire);
  if (t) return *t;
  std::lock_guard<std::mutex> lock(g_tuning_mu);
  t = g_tuning.load(std::memory_order_acquire);
  if (!t) {
    t = new Tuning(read_tuning());
    g_tuning.store(t, std::memory_order_release);
  }
  return *t;
}

void reload_tuning() {
  std::lock_guard<std::mutex> lock(g_tuning_mu);
  g_tuning.store(new Tuning(read_tuning()), std::memory_order_release);
}

}  // namespace fln

extern "C" void fln_reload_tuning(void) { fln::reload_tuning(); }

// Same estimate as the reference's get_memory_usage (csrc/layernorm_cuda.cpp:144-164):
// forward in/out + fp32 mean/rstd, backward grad_input + grad_gamma/beta, plus a per-row
// workspace term.
extern "C" int64_t fln_get_memory_usage(int batch_size, int hidden_size,
                                        int use_mixed_precision) {
  const int64_t es = use_mixed_precision ? 2 : 4;
  const int64_t b = batch_size, h = hidden_size;
  const int64_t forward_memory = 2 * b * h * es + 2 * b * static_cast<int64_t>(sizeof(float));
  const int64_t backward_memory = b * h * es + 2 * h * es;
  const int64_t workspace = b * 32 * static_cast<int64_t>(sizeof(float));
  return forward_memory + backward_memory + workspace;
}

// Hints with the reference's wording and thresholds (csrc/layernorm_cuda.cpp:167-195), except
// that the occupancy check uses this device's CU count instead of an assumed 80 SMs.
extern "C" int fln_get_performance_hints(int batch_size, int hidden_size, char* buf,
                                         size_t buflen) {
  std::string hints;
  if (hidden_size % 32 != 0)
    hints += "Warning: hidden_size is not divisible by 32, may impact performance.\n";
  if (hidden_size > 8192)
    hints += "Info: Large hidden dimension detected. Consider using mixed precision.\n";
  if (batch_size < 8) hints += "Info: Small batch size may not fully utilize GPU.\n";
  const int cus = fln::device_cu_count();
  if (batch_size < cus) hints += "Info: Not enough blocks to saturate GPU. Consider batching.\n";
  if (buf && buflen > 0) {
    const size_t n = hints.size() < buflen - 1 ? hints.size() : buflen - 1;
    memcpy(buf, hints.data(), n);
    buf[n] = '\0';
  }
  return static_cast<int>(hints.size());
}

extern "C" const char* fln_version(void) { return "1.0.0"; }

extern "C" int fln_hip_version(void) { return HIP_VERSION; }

extern "C" const char* fln_error_string(int code) {
  if (code == FLN_OK) return "success";
  if (code == FLN_ERR_INVALID) return "invalid argument (shape, dtype, pointer or workspace)";
  if (code == FLN_ERR_TOO_LARGE)
    return "problem needs more workspace than the no-allocation scratch holds (32 MiB)";
  return hipGetErrorString(static_cast<hipError_t>(code));
}
