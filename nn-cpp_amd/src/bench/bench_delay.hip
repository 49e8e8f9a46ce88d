// bench_delay.hip - measurement helper for bench.py (libnnh_bench.so, not part of the nnh ABI).
//
// Small ops take less device time than a Python call takes to issue them, so timing R back-to-back calls
// with events would measure the host. nnh_bench_delay() first occupies the stream with one wave that
// spins on the constant-rate wall clock for a bounded interval; the host queues the R calls meanwhile,
// and events recorded after the delay see the calls run back to back at device speed.
#include <hip/hip_runtime.h>

namespace {

__global__ void __launch_bounds__(64) delay_kernel(unsigned long long ticks) {
	const unsigned long long t0 = wall_clock64();
	while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

}  // namespace

extern "C" {

// Blocks `stream` for `microseconds` (clamped to [0, 2 s]) of device time. Returns 0 or a HIP error code.
int nnh_bench_delay(double microseconds, void* stream) {
	int dev = 0;
	hipError_t e = hipGetDevice(&dev);
	if (e != hipSuccess) return (int)e;
	int rate_khz = 0;
	e = hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev);
	if (e != hipSuccess) return (int)e;
	if (rate_khz <= 0) rate_khz = 100000;  // the documented 100 MHz constant clock
	if (!(microseconds > 0.0)) microseconds = 0.0;
	if (microseconds > 2.0e6) microseconds = 2.0e6;
	const unsigned long long ticks = (unsigned long long)(microseconds * 1e-3 * rate_khz);
	hipLaunchKernelGGL(delay_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), ticks);
	return (int)hipGetLastError();
}

}  // extern "C"
