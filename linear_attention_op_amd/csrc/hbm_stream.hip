// HBM stream probe: the measurement yardstick for the decode kernels, whose state traffic is a plain stream
// (read once, written once).  Built into its own library, libgdn_stream.so, which only the benchmark loads.
//
// stream_kernel<MODE, U, NT>: 256 threads per workgroup; a workgroup walks blocks of 256 U float4 (16 B per
// thread and access, U accesses per thread in flight) in a grid-stride loop.
//   MODE 0 read:     sum of every element (kept live by a data-dependent store)
//   MODE 1 write:    dst = constant
//   MODE 2 copy:     dst = src
//   MODE 3 in place: src = src * c           (the decode state's pattern: read once, written once in place)
// NT: non-temporal loads and stores (the cache policy the decode kernels use for their streams).
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ f32x4 ld(const f32x4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}
template <bool NT>
__device__ __forceinline__ void st(f32x4* p, f32x4 v) {
    if constexpr (NT)
        __builtin_nontemporal_store(v, p);
    else
        *p = v;
}

template <int MODE, int U, bool NT>
__global__ __launch_bounds__(256) void stream_kernel(f32x4* src, f32x4* dst, size_t n4, float c, float* sink) {
    const size_t step = (size_t)gridDim.x * 256 * U;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (size_t base = (size_t)blockIdx.x * 256 * U + threadIdx.x; base < n4; base += step) {
        f32x4 v[U];
        if constexpr (MODE != 1) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const size_t i = base + (size_t)u * 256;
                if (i < n4) v[u] = ld<NT>(src + i);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t i = base + (size_t)u * 256;
            if (i >= n4) continue;
            if constexpr (MODE == 0) acc += v[u];
            if constexpr (MODE == 1) st<NT>(dst + i, f32x4{c, c, c, c});
            if constexpr (MODE == 2) st<NT>(dst + i, v[u]);
            if constexpr (MODE == 3) st<NT>(src + i, v[u] * c);
        }
    }
    if constexpr (MODE == 0) {
        // the sum must be used; it equals the sentinel only by accident, so the store almost never happens
        if (acc[0] + acc[1] + acc[2] + acc[3] == c) sink[threadIdx.x] = acc[0];
    }
}

template <int MODE, bool NT>
hipError_t launch_u(int unroll, f32x4* src, f32x4* dst, size_t n4, float c, float* sink, int blocks,
                    hipStream_t s) {
    switch (unroll) {
        case 1: hipLaunchKernelGGL((stream_kernel<MODE, 1, NT>), dim3(blocks), dim3(256), 0, s, src, dst, n4, c, sink); break;
        case 2: hipLaunchKernelGGL((stream_kernel<MODE, 2, NT>), dim3(blocks), dim3(256), 0, s, src, dst, n4, c, sink); break;
        case 4: hipLaunchKernelGGL((stream_kernel<MODE, 4, NT>), dim3(blocks), dim3(256), 0, s, src, dst, n4, c, sink); break;
        case 8: hipLaunchKernelGGL((stream_kernel<MODE, 8, NT>), dim3(blocks), dim3(256), 0, s, src, dst, n4, c, sink); break;
        case 16: hipLaunchKernelGGL((stream_kernel<MODE, 16, NT>), dim3(blocks), dim3(256), 0, s, src, dst, n4, c, sink); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_m(int unroll, int nt, f32x4* src, f32x4* dst, size_t n4, float c, float* sink, int blocks,
                    hipStream_t s) {
    return nt ? launch_u<MODE, true>(unroll, src, dst, n4, c, sink, blocks, s)
              : launch_u<MODE, false>(unroll, src, dst, n4, c, sink, blocks, s);
}

}  // namespace

extern "C" {

// One pass of `mode` (0 read, 1 write, 2 copy, 3 in place) over `bytes` (a multiple of 16) of src / dst with
// `blocks` workgroups of 256 threads, `unroll` (1, 2, 4, 8, 16) 16-byte accesses in flight per thread,
// non-temporal accesses if nt != 0.  sink: 256 floats of device memory (read mode).  Returns 0 or a hipError_t.
int gdn_stream_run(int mode, int unroll, int nt, void* src, void* dst, size_t bytes, int blocks, float* sink,
                   void* stream) {
    if (bytes % 16 || blocks <= 0 || !src) return (int)hipErrorInvalidValue;
    if ((mode == 1 || mode == 2) && !dst) return (int)hipErrorInvalidValue;
    if (mode == 0 && !sink) return (int)hipErrorInvalidValue;
    f32x4* s4 = static_cast<f32x4*>(src);
    f32x4* d4 = static_cast<f32x4*>(dst);
    const size_t n4 = bytes / 16;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const float c = 1.0000001f;
    switch (mode) {
        case 0: return (int)launch_m<0>(unroll, nt, s4, d4, n4, c, sink, blocks, st);
        case 1: return (int)launch_m<1>(unroll, nt, s4, d4, n4, c, sink, blocks, st);
        case 2: return (int)launch_m<2>(unroll, nt, s4, d4, n4, c, sink, blocks, st);
        case 3: return (int)launch_m<3>(unroll, nt, s4, d4, n4, c, sink, blocks, st);
        default: return (int)hipErrorInvalidValue;
    }
}

}  // extern "C"
