// probe.hip - calibration kernels for the measurement harness (bench.py --only probes), built
// into libgsx_probe.so beside libgsx_hip.so. They are not part of the render ABI or the gsx
// plugin: they give the counters and timers a workload whose instruction count or byte count
// is known by construction, so that a kernel's VALU figures and its store rate can be read as
// fractions of what this GPU does.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kValuChains = 16;  // independent FMA chains per lane: issue, not latency, bounds

// Each lane runs `iters` steps of kValuChains independent v_fma_f32 (one VALU instruction per
// FMA, the loop's counter and branch on the scalar unit), then stores one value so nothing is
// dead. Wave-level VALU instructions issued: blocks * 4 waves * iters * kValuChains, plus a few
// dozen per wave outside the loop.
__global__ __launch_bounds__(256) void valu_fma_kernel(int iters, float scale, float* __restrict__ out) {
    float a[kValuChains];
#pragma unroll
    for (int j = 0; j < kValuChains; ++j) a[j] = (float)(threadIdx.x + j);
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int j = 0; j < kValuChains; ++j) a[j] = __builtin_fmaf(a[j], scale, 0.5f);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kValuChains; ++j) s += a[j];
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Zero `count` floats with 16-byte stores (count % 4 == 0, dst 16-byte aligned), grid-stride.
__global__ __launch_bounds__(256) void store_zero_kernel(float4* __restrict__ dst, int64_t vecs) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < vecs; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

}  // namespace

extern "C" {

// out holds blocks * 256 floats. Returns a hipError_t value (0 on success).
int gsx_probe_valu_fma(int blocks, int iters, float* out, hipStream_t stream) {
    if (blocks <= 0 || iters <= 0 || out == nullptr) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(valu_fma_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, iters, 0.999f, out);
    return (int)hipGetLastError();
}

// The VALU instructions one wave of gsx_probe_valu_fma issues inside its loop per iteration.
int gsx_probe_valu_fma_per_iter(void) { return kValuChains; }

// dst: `count` floats, count a multiple of 4, 16-byte aligned; `blocks` workgroups of 256.
int gsx_probe_store_zero(float* dst, int64_t count, int blocks, hipStream_t stream) {
    if (dst == nullptr || count < 0 || count % 4 != 0 || (reinterpret_cast<uintptr_t>(dst) & 15u) != 0 ||
        blocks <= 0) {
        return (int)hipErrorInvalidValue;
    }
    if (count == 0) return 0;
    hipLaunchKernelGGL(store_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, reinterpret_cast<float4*>(dst),
                       count / 4);
    return (int)hipGetLastError();
}

}  // extern "C"
