// Error reporting, the kernel registry and device queries of the C-ABI.
#include <cstring>
#include <string>
#include <vector>

#include "mb_internal.h"

namespace mb {
namespace {

thread_local char g_last_error[1024] = "";

std::vector<KernelEntry>& registry() {
  static std::vector<KernelEntry> entries;
  return entries;
}

}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return code;
}

int hip_status(hipError_t status, const char* what) {
  if (status == hipSuccess) return MB_OK;
  return fail(MB_ERR_HIP, "%s: %s (%s)", what, hipGetErrorString(status), hipGetErrorName(status));
}

void register_kernel(const char* name, const void* func) { registry().push_back({name, func}); }

}  // namespace mb

extern "C" {

int mb_abi_version(void) { return MB_ABI_VERSION; }

const char* mb_last_error(void) { return mb::g_last_error; }

int mb_device_query(int device, mb_device_info* out) {
  if (out == nullptr) return mb::fail(MB_ERR_INVALID, "mb_device_query: out is NULL");
  int count = 0;
  if (int rc = mb::hip_status(hipGetDeviceCount(&count), "hipGetDeviceCount")) return rc;
  if (device < 0 || device >= count)
    return mb::fail(MB_ERR_INVALID, "mb_device_query: device %d outside 0..%d", device, count - 1);
  hipDeviceProp_t prop;
  if (int rc = mb::hip_status(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties")) return rc;
  std::memset(out, 0, sizeof(*out));
  std::snprintf(out->name, sizeof(out->name), "%s", prop.name);
  std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
  out->compute_units = prop.multiProcessorCount;
  out->wavefront_size = prop.warpSize;
  out->clock_khz = prop.clockRate;
  out->memory_clock_khz = prop.memoryClockRate;
  out->memory_bus_bits = prop.memoryBusWidth;
  out->l2_cache_bytes = prop.l2CacheSize;
  out->lds_bytes_per_cu = static_cast<int64_t>(prop.maxSharedMemoryPerMultiProcessor);
  int previous = 0;
  if (int rc = mb::hip_status(hipGetDevice(&previous), "hipGetDevice")) return rc;
  if (int rc = mb::hip_status(hipSetDevice(device), "hipSetDevice")) return rc;
  size_t free_bytes = 0, total_bytes = 0;
  int rc = mb::hip_status(hipMemGetInfo(&free_bytes, &total_bytes), "hipMemGetInfo");
  hipSetDevice(previous);
  if (rc) return rc;
  out->total_memory_bytes = static_cast<int64_t>(total_bytes);
  out->free_memory_bytes = static_cast<int64_t>(free_bytes);
  return MB_OK;
}

int mb_kernel_count(void) { return static_cast<int>(mb::registry().size()); }

const char* mb_kernel_name(int index) {
  auto& entries = mb::registry();
  if (index < 0 || index >= static_cast<int>(entries.size())) {
    mb::fail(MB_ERR_INVALID, "mb_kernel_name: index %d outside 0..%zu", index, entries.size());
    return nullptr;
  }
  return entries[index].name;
}

int mb_kernel_attributes_query(const char* name, mb_kernel_attributes* out) {
  if (name == nullptr || out == nullptr)
    return mb::fail(MB_ERR_INVALID, "mb_kernel_attributes_query: NULL argument");
  for (const auto& entry : mb::registry()) {
    if (std::strcmp(entry.name, name) != 0) continue;
    hipFuncAttributes attributes;
    if (int rc = mb::hip_status(hipFuncGetAttributes(&attributes, entry.func), "hipFuncGetAttributes"))
      return rc;
    out->registers_per_thread = attributes.numRegs;
    out->max_threads_per_block = attributes.maxThreadsPerBlock;
    out->lds_bytes = static_cast<int64_t>(attributes.sharedSizeBytes);
    out->scratch_bytes = static_cast<int64_t>(attributes.localSizeBytes);
    return MB_OK;
  }
  return mb::fail(MB_ERR_INVALID, "mb_kernel_attributes_query: no kernel named '%s'", name);
}

}  // extern "C"
