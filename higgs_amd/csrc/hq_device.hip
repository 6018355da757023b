// hq_device.hip -- the per-device launcher state declared in hq_device.hpp
// (one definition for every per-bit-width kernel object).
#include "hq_device.hpp"

namespace hq {

namespace {

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  return dev;
}

std::atomic<int> g_cus[kMaxCachedDevices];  // zero: not yet queried

}  // namespace

int device_cu_count() {
  const int dev = current_device();
  if (dev < kMaxCachedDevices) {
    const int c = g_cus[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
    v = 256;
  if (dev < kMaxCachedDevices) g_cus[dev].store(v, std::memory_order_relaxed);
  return v;
}

hipError_t raise_lds_limit(const void* fn, int bytes, std::atomic<uint64_t>& done) {
  const int dev = current_device();
  const uint64_t bit = dev < kMaxCachedDevices ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

}  // namespace hq
