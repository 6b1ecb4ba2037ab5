// Lowering check for the agent-scope coherent accesses of kvrt_device.h.
//
// Never linked into libkvrt.so and never launched: the build compiles this
// file to gfx950 assembly with the library's own flags and checks, kernel by
// kernel, that each helper lowers to the instruction form the single-launch
// decode merge was validated with (stores and loads carrying the device-scope
// sc1 bit, the arrival counter an L2 atomic add that returns its old value,
// no cache write-back or invalidate). A compiler that lowers them otherwise
// fails the build instead of changing the merge's memory behaviour silently.
#include "kvrt_device.h"

using namespace kvrt;

extern "C" __global__ void kvrt_probe_store_f32(float *p, float v) { store_agent(p + threadIdx.x, v); }

extern "C" __global__ void kvrt_probe_store_f32x2(float2 *p, float2 v) { store_agent(p + threadIdx.x, v); }

extern "C" __global__ void kvrt_probe_store16(uint4 *p, uint4 v) { store_agent16(p + threadIdx.x, v); }

extern "C" __global__ void kvrt_probe_load_f32(const float *p, float *o) { o[threadIdx.x] = load_agent(p + threadIdx.x); }

extern "C" __global__ void kvrt_probe_load_f32x2(const float2 *p, float2 *o) {
    o[threadIdx.x] = load_agent(p + threadIdx.x);
}

extern "C" __global__ void kvrt_probe_arrive(uint32_t *c, uint32_t *o) { o[threadIdx.x] = arrive_agent(c); }

extern "C" __global__ void kvrt_probe_clear(uint32_t *c) { clear_agent(c + threadIdx.x); }
