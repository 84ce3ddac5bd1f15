// clock_probe.hip -- the benchmark's in-process clock reading (not part of
// the attention library's C ABI).
//
// One wave records s_memtime (shader-clock cycles of its CU) and
// s_memrealtime (the constant wall clock) at its start, sleeps in a loop
// until `ticks` wall-clock ticks have passed, and records both again: the
// ratio of the two deltas times the wall-clock rate is the CU's mean clock
// over that window.  bench.py launches it on a second stream just before
// the timed steps, so the window lies inside them and the reading is the
// clock the attention kernels ran at.  Sleeping, the wave takes no issue
// slots; it holds a few registers of one SIMD for the window.
#include <hip/hip_runtime.h>
#include <stdint.h>

__global__ __launch_bounds__(64) void clock_probe_kernel(uint64_t *out, int64_t ticks) {
    if (threadIdx.x != 0) return;
    const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    uint64_t r = r0;
    while ((int64_t)(r - r0) < ticks) {
        __builtin_amdgcn_s_sleep(64);
        r = __builtin_amdgcn_s_memrealtime();
    }
    const uint64_t c1 = __builtin_amdgcn_s_memtime();
    out[0] = c1 - c0;
    out[1] = r - r0;
}

extern "C" {

// Launches the probe on `stream`; out must hold two uint64 in device memory.
// 0 on success, else the hipError_t of the launch.
int fa2_clock_probe_launch(uint64_t *out, int64_t ticks, void *stream) {
    if (!out || ticks <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, out, ticks);
    return (int)hipGetLastError();
}

// Ticks per second of s_memrealtime on the current device.
int64_t fa2_clock_probe_wall_hz(void) {
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess) return 0;
    return (int64_t)khz * 1000;
}

}  // extern "C"
