// Engine-clock witness: the shader clock a kernel sustains, measured on the
// device while that kernel runs.
//
// MI355X runs matrix kernels under its power limit, so the engine clock, and
// with it the achievable rate, differs from kernel to kernel and box to box.
// The witness is one wave launched on a second stream beside the measured
// kernel's launches: it reads the shader clock counter (s_memtime, one count
// per engine clock cycle) and the constant-rate real-time counter
// (s_memrealtime, hipDeviceAttributeWallClockRate) at its start, sleeps and
// polls the real-time counter until `ticks` have passed, and reads both again.
// cycles / ticks * wall clock rate is the clock of the witness's CU over that
// interval. The wave sleeps between polls, so it takes next to no issue
// slots from the measured kernel.
//
// The loop ends when the real-time interval has passed, or after `max_polls`
// polls, whichever comes first, so every launch ends.
#include "mb_internal.h"

namespace mb {
namespace {

__global__ void __launch_bounds__(64) clock_witness_kernel(uint64_t* __restrict__ out, uint64_t ticks,
                                                           uint64_t max_polls) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  uint64_t r = r0, polls = 0;
  while (r - r0 < ticks && polls < max_polls) {
    __builtin_amdgcn_s_sleep(4);
    r = __builtin_amdgcn_s_memrealtime();
    ++polls;
  }
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x < 4) {
    const uint64_t values[4] = {c1 - c0, r1 - r0, polls, r0};
    out[threadIdx.x] = values[threadIdx.x];
  }
}

MB_REGISTER_KERNEL("clock_witness", clock_witness_kernel);

int g_wall_khz = 0;

}  // namespace
}  // namespace mb

extern "C" {

int mb_clock_witness(uint64_t* out, uint64_t out_bytes, uint32_t microseconds, void* stream) {
  using namespace mb;
  if (out == nullptr || out_bytes < 4 * sizeof(uint64_t))
    return fail(MB_ERR_INVALID, "mb_clock_witness: out needs 4 uint64 entries (%llu bytes given)",
                (unsigned long long)out_bytes);
  if (!aligned(out, 8)) return fail(MB_ERR_ALIGNMENT, "mb_clock_witness: out must be 8-byte aligned");
  if (microseconds == 0 || microseconds > 10000000u)
    return fail(MB_ERR_INVALID, "mb_clock_witness: interval %u us outside 1..10000000", microseconds);
  if (int rc = mb_wall_clock_khz(&g_wall_khz)) return rc;
  const uint64_t ticks = static_cast<uint64_t>(microseconds) * static_cast<uint64_t>(g_wall_khz) / 1000u;
  // A poll sleeps 4 x 64 engine cycles, at least 0.1 us at any clock this device runs, so the real-time
  // interval ends the loop long before this bound (which would take at least 6.4 times the interval).
  const uint64_t max_polls = 64ull * microseconds + 1000u;
  clock_witness_kernel<<<dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream)>>>(out, ticks ? ticks : 1,
                                                                                   max_polls);
  return launch_status("clock_witness");
}

int mb_wall_clock_khz(int* khz) {
  using namespace mb;
  if (khz == nullptr) return fail(MB_ERR_INVALID, "mb_wall_clock_khz: NULL argument");
  int device = 0;
  if (int rc = hip_status(hipGetDevice(&device), "hipGetDevice")) return rc;
  if (int rc = hip_status(hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, device),
                          "hipDeviceGetAttribute(WallClockRate)"))
    return rc;
  if (*khz <= 0) return fail(MB_ERR_HIP, "mb_wall_clock_khz: the runtime reports a wall clock of %d kHz", *khz);
  return MB_OK;
}

}  // extern "C"
