// f3s_device.hpp -- device-side building blocks (wave64, gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace f3s {

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Workgroup barrier that orders LDS only.  __syncthreads() also fences
// global memory, which makes every wave wait for all of its outstanding
// vector-memory loads (s_waitcnt vmcnt(0)) at each barrier; this one waits
// for LDS operations only, so loads issued ahead of time stay in flight.
// Global stores made before it are NOT visible to the other waves after it.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Inclusive scan over the 64 lanes of a wave.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v)
{
    const int lane = lane_id();
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        T o = __shfl_up(v, off, kWave);
        if (lane >= off) v += o;
    }
    return v;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Exclusive scan across a workgroup of NT threads (NT a multiple of 64);
// `total` receives the workgroup sum.  `lds` needs NT/64 elements.  Contains
// barriers: every thread of the workgroup must call it.
template <int NT, typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* lds, T& total)
{
    constexpr int NW = NT / kWave;
    const int lane = lane_id();
    const int wid = threadIdx.x / kWave;
    T inc = wave_inclusive_scan(v);
    if (lane == kWave - 1) lds[wid] = inc;
    __syncthreads();
    T base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        T s = lds[i];
        if (i < wid) base += s;
        tot += s;
    }
    __syncthreads();
    total = tot;
    return base + inc - v;
}

}  // namespace f3s
