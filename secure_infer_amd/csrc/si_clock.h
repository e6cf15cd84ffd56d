// Device side of the clock probe of a measured launch (ClockProbe in
// si_kernels.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

// A measured launch (`stamps` non-null): lane 0 of every wave writes the
// device's constant-rate clock when the wave starts (end = 0) and when it
// ends (end = 1), into its own pair of words; waves are numbered over the
// grid (x, then y) and then the workgroup's waves.
__device__ __forceinline__ void clock_stamp(uint64_t* stamps, uint32_t end)
{
    if (stamps != nullptr && (threadIdx.x & 63u) == 0u) {
        const uint64_t wave =
            (uint64_t(blockIdx.y) * gridDim.x + blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
        stamps[2 * wave + end] = wall_clock64();
    }
}

}  // namespace si
