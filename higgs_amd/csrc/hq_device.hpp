// hq_device.hpp -- per-device launcher state shared by the kernel sources:
// the CU count and the one-time opt-in to more than 64 KB of dynamic LDS
// (defined once, in hq_device.hip).
//
// Both are cached per device (the HIP device current on the calling thread)
// in atomics, so first calls that race from several threads are safe: each
// may query or set the attribute itself (the calls are idempotent), and the
// caches only ever go from "unknown" to the one value the device has.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

namespace hq {

// Devices whose state is cached (higher ids are queried on every call).
constexpr int kMaxCachedDevices = 64;

// Compute units of the current device; 256 (MI355X) if the runtime cannot
// report it.
int device_cu_count();

// Raises kernel `fn`'s dynamic-LDS limit to `bytes` on the current device,
// once per device: `done` is the call site's bit set of devices already
// raised.
hipError_t raise_lds_limit(const void* fn, int bytes, std::atomic<uint64_t>& done);

}  // namespace hq
