// Measurement aid (not part of libgemma4_qmm): a read-only HBM streaming kernel, the
// practical read ceiling the decode kernels are compared with.  Built into its own
// libhbm_probe.so, loaded only by the benchmark.
//
// Access pattern: wave w of the grid reads one contiguous 8 KiB run per step (eight
// 16-byte non-temporal loads per lane, lane-contiguous within each 1 KiB), and
// neighbouring waves read neighbouring runs; the grid strides over the buffer, two
// runs per wave in flight.  Each wave folds what it read into one word and writes it
// to sink[wave] (4 bytes per wave: the only writes).
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kLoads = 8;          // 16-byte loads per lane per run
constexpr int kRun = kLoads * 1024;  // bytes per wave per step

__global__ __launch_bounds__(256) void hbm_read_kernel(const uint4* __restrict__ buf, long runs,
                                                       uint32_t* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    const long wave = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const long waves = (long)gridDim.x * (blockDim.x >> 6);
    u32x4 a[kLoads], b[kLoads];
    uint32_t acc = 0;
    auto load = [&](u32x4* dst, long r) {
        const u32x4* p = reinterpret_cast<const u32x4*>(buf) + r * (kRun / 16) + lane;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) dst[i] = __builtin_nontemporal_load(p + i * 64);
    };
    auto fold = [&](const u32x4* v) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    };
    long r = wave;
    if (r < runs) load(a, r);
    for (; r < runs; r += 2 * waves) {
        const long r2 = r + waves;
        if (r2 < runs) load(b, r2);
        fold(a);
        if (r2 >= runs) break;
        const long r3 = r2 + waves;
        if (r3 < runs) load(a, r3);
        fold(b);
    }
    if (lane == 0) sink[wave] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 8 KiB) from buf once on `stream`; sink holds one
// uint32 per wave of the grid (wgs_per_cu x CUs workgroups of 4 waves).
int hbm_read_probe(const void* buf, size_t bytes, uint32_t* sink, int workgroups, void* stream) {
    if (buf == nullptr || sink == nullptr || bytes % kRun != 0 || workgroups <= 0) return -1;
    hipLaunchKernelGGL(hbm_read_kernel, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(buf), (long)(bytes / kRun), sink);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
