// Error reporting for the C-ABI: every entry point returns an int status and
// leaves a human-readable message retrievable with cdssm_last_error().
#include <cstdlib>
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>

#include "common.hpp"

namespace {
thread_local char g_err[512] = "";
}

namespace cdssm_host {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* op) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", op, hipGetErrorString(e));
    return CDSSM_EHIP;
  }
  return CDSSM_OK;
}

int resident_capacity(const void* fn, int block, size_t lds) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  struct Entry {
    const void* fn;
    int dev, block;
    size_t lds;
    int capacity;
  };
  static std::mutex mu;
  static Entry cache[64];
  static int n_cache = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_cache; ++i)
    if (cache[i].fn == fn && cache[i].dev == dev && cache[i].block == block && cache[i].lds == lds)
      return cache[i].capacity;
  int max_lds = 0, n_cu = 0, per_cu = 0, capacity = 0;
  if (hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
      hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      lds <= size_t(max_lds)) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, block, lds) == hipSuccess) capacity = per_cu * n_cu;
  }
  (void)hipGetLastError();
  if (n_cache < 64) cache[n_cache++] = Entry{fn, dev, block, lds, capacity};
  return capacity;
}

int device_cus() {
  int dev = 0, n_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 0;
  }
  static std::atomic<int> cache[64];
  const int c = cache[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  cache[dev].store(n_cu, std::memory_order_relaxed);
  return n_cu;
}

namespace {
std::atomic<int> g_scan_path{kPathAuto};
}

int scan_path() { return g_scan_path.load(std::memory_order_relaxed); }
bool wide_staging() {
  static const bool on = std::getenv("CDSSM_NARROW_STAGING") == nullptr;
  return on;
}

}  // namespace cdssm_host

extern "C" int cdssm_fused_scan_fwd_set_path(int mode) {
  if (mode < cdssm_host::kPathAuto || mode > cdssm_host::kPathSweep) {
    cdssm_host::set_error("cdssm_fused_scan_fwd_set_path: mode must be 0 (auto), 1 (four launches), 2 "
                          "(one pass required) or 3 (four launches with the chunked MFMA correction), got %d",
                          mode);
    return CDSSM_EINVAL;
  }
  return cdssm_host::g_scan_path.exchange(mode);
}

extern "C" int cdssm_lookback_status(int clear, int* status) {
  if (!status) {
    cdssm_host::set_error("cdssm_lookback_status: status must not be NULL");
    return CDSSM_EINVAL;
  }
  unsigned f = 0, b = 0;
  int st = cdssm_host::fwd_lookback_status(clear != 0, &f);
  if (st) return st;
  st = cdssm_host::bwd_lookback_status(clear != 0, &b);
  if (st) return st;
  *status = int((f & cdssm::kTimeoutFwd) | (b & cdssm::kTimeoutBwd));
  return CDSSM_OK;
}

extern "C" const char* cdssm_last_error(void) { return g_err; }

extern "C" int cdssm_abi_version(void) { return 2; }
