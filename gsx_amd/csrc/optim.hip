// optim.hip - Adam over all parameter groups of a Gaussian set in one launch.
//
// Element arithmetic is the gsx CPU backend's (gsx/src/gsx-cpu/optim.c:712-780), operation for
// operation, so results are bit-identical to it:
//   g = clamp(g, +-max_grad) when max_grad > 0
//   m = beta1 m + (1 - beta1) g ;  v = beta2 v + (1 - beta2) g g          (float32)
//   m_hat = (float)((double)m / bc1) ; v_hat = (float)((double)v / bc2)   (bias correction in f64)
//   p -= lr * wd * p (wd > 0) ;  p -= lr * (m_hat / (sqrt(v_hat) + eps))
// The CUDA backend issues one launch per group (gsx-cuda/optim.c:757-796); here a single grid
// covers every group: each workgroup looks up its group in a small prefix table of block counts.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gsx_hip.h"

namespace {

constexpr int kAdamThreads = 256;
// Each thread updates kVecs float4 of each array. Steps whose traffic (28 bytes per element:
// parameter, gradient and both moments in, parameter and moments out) exceeds the 256 MiB
// memory-side cache take two float4 per thread with non-temporal loads and stores, so that Adam's
// streams do not displace what the next step's kernels read. Measured on one MI355X, five SH0
// groups: at 3M Gaussians Adam takes 189.0 instead of 216.8 us and the config-3 training step
// runs at 874-877 instead of 823-825 it/s; at 6M 394.8 instead of 438.0 us. At 1M (392 MB) Adam
// alone is slower (63.2 vs 57.0 us, its arrays no longer cached between repeats), but in the
// training step the next preprocess gains as much (metric step 1299-1314 vs 1297-1310 it/s).
constexpr int64_t kAdamStreamBytes = 256ll << 20;
constexpr int64_t kAdamBytesPerElement = 28;

struct AdamBatch {
    gsx_hip_adam_group groups[GSX_HIP_ADAM_MAX_GROUPS];
    uint32_t block_start[GSX_HIP_ADAM_MAX_GROUPS + 1];
    int32_t group_count;
};

__device__ inline float adam_element(float p, float g, float& m, float& v, const gsx_hip_adam_group& gr) {
    if (gr.max_grad > 0.0f) {
        if (g > gr.max_grad) {
            g = gr.max_grad;
        } else if (g < -gr.max_grad) {
            g = -gr.max_grad;
        }
    }
    const float m1 = gr.beta1 * m + (1.0f - gr.beta1) * g;
    const float v1 = gr.beta2 * v + (1.0f - gr.beta2) * g * g;
    const float mh = (float)((double)m1 / gr.bias_correction1);
    const float vh = (float)((double)v1 / gr.bias_correction2);
    m = m1;
    v = v1;
    if (gr.weight_decay > 0.0f) p -= gr.learning_rate * gr.weight_decay * p;
    p -= gr.learning_rate * (mh / (sqrtf(vh) + gr.epsilon));
    return p;
}

typedef float gsx_v4f __attribute__((ext_vector_type(4)));

template <bool kStream>
__device__ inline gsx_v4f load4(const float* p) {
    if constexpr (kStream) return __builtin_nontemporal_load(reinterpret_cast<const gsx_v4f*>(p));
    else return *reinterpret_cast<const gsx_v4f*>(p);
}

template <bool kStream>
__device__ inline void store4(float* p, gsx_v4f x) {
    if constexpr (kStream) __builtin_nontemporal_store(x, reinterpret_cast<gsx_v4f*>(p));
    else *reinterpret_cast<gsx_v4f*>(p) = x;
}

template <bool kStream>
__global__ __launch_bounds__(kAdamThreads) void adam_multi_kernel(AdamBatch batch) {
    constexpr int kVecs = kStream ? 2 : 1;
    constexpr int kChunk = kAdamThreads * 4 * kVecs;
    int k = 0;
    while (k + 1 < batch.group_count && blockIdx.x >= batch.block_start[k + 1]) ++k;
    const gsx_hip_adam_group& gr = batch.groups[k];
    const int64_t first = (int64_t)(blockIdx.x - batch.block_start[k]) * kChunk;
    const int64_t n = gr.count;
    const bool aligned = ((reinterpret_cast<uintptr_t>(gr.parameter) | reinterpret_cast<uintptr_t>(gr.gradient) |
                           reinterpret_cast<uintptr_t>(gr.first_moment) |
                           reinterpret_cast<uintptr_t>(gr.second_moment)) & 15u) == 0;
    if (aligned && first + kChunk <= n) {
        // every load of the thread is issued before the first update
        gsx_v4f p[kVecs], g[kVecs], m[kVecs], v[kVecs];
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t e = first + ((int64_t)j * kAdamThreads + threadIdx.x) * 4;
            p[j] = load4<kStream>(gr.parameter + e);
            g[j] = load4<kStream>(gr.gradient + e);
            m[j] = load4<kStream>(gr.first_moment + e);
            v[j] = load4<kStream>(gr.second_moment + e);
        }
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float mc = m[j][c], vc = v[j][c];
                p[j][c] = adam_element(p[j][c], g[j][c], mc, vc, gr);
                m[j][c] = mc;
                v[j][c] = vc;
            }
            const int64_t e = first + ((int64_t)j * kAdamThreads + threadIdx.x) * 4;
            store4<kStream>(gr.parameter + e, p[j]);
            store4<kStream>(gr.first_moment + e, m[j]);
            store4<kStream>(gr.second_moment + e, v[j]);
        }
    } else {
        // a group's partial last chunk, or arrays that are not 16-byte aligned
        const int64_t end = min(n, first + kChunk);
        for (int64_t e = first + threadIdx.x; e < end; e += kAdamThreads) {
            float mc = gr.first_moment[e];
            float vc = gr.second_moment[e];
            gr.parameter[e] = adam_element(gr.parameter[e], gr.gradient[e], mc, vc, gr);
            gr.first_moment[e] = mc;
            gr.second_moment[e] = vc;
        }
    }
}

}  // namespace

extern "C" {

gsx_hip_status gsx_hip_adam_step_multi_launch(const gsx_hip_adam_group* groups, int32_t group_count,
                                              hipStream_t stream) {
    if (groups == nullptr || group_count <= 0 || group_count > GSX_HIP_ADAM_MAX_GROUPS) {
        return GSX_HIP_ERROR_INVALID_ARGUMENT;
    }
    AdamBatch batch;
    batch.group_count = group_count;
    int64_t elements = 0;
    for (int k = 0; k < group_count; ++k) {
        if (groups[k].count < 0) return GSX_HIP_ERROR_INVALID_ARGUMENT;
        elements += groups[k].count;
    }
    const bool stream_access = elements > kAdamStreamBytes / kAdamBytesPerElement;
    const int64_t chunk = (int64_t)kAdamThreads * 4 * (stream_access ? 2 : 1);
    uint64_t blocks = 0;
    for (int k = 0; k < group_count; ++k) {
        if (groups[k].count > 0 && (groups[k].parameter == nullptr || groups[k].gradient == nullptr ||
                                    groups[k].first_moment == nullptr || groups[k].second_moment == nullptr)) {
            return GSX_HIP_ERROR_INVALID_ARGUMENT;
        }
        batch.groups[k] = groups[k];
        batch.block_start[k] = (uint32_t)blocks;
        blocks += (uint64_t)((groups[k].count + chunk - 1) / chunk);
        if (blocks > 0x7fffffffu) return GSX_HIP_ERROR_OUT_OF_RANGE;
    }
    batch.block_start[group_count] = (uint32_t)blocks;
    if (blocks == 0) return GSX_HIP_SUCCESS;
    if (stream_access) {
        hipLaunchKernelGGL(adam_multi_kernel<true>, dim3((unsigned)blocks), dim3(kAdamThreads), 0, stream, batch);
    } else {
        hipLaunchKernelGGL(adam_multi_kernel<false>, dim3((unsigned)blocks), dim3(kAdamThreads), 0, stream, batch);
    }
    return (gsx_hip_status)hipGetLastError();
}

// Replace gsx_cuda_adam_step_f32_kernel_launch (gsx-cuda/internal.h:296-311): one group.
gsx_hip_status gsx_hip_adam_step_f32_kernel_launch(float* parameter, const float* gradient, float* first_moment,
                                                   float* second_moment, int64_t total_elements, float beta1,
                                                   float beta2, float learning_rate, float weight_decay,
                                                   float epsilon, float max_grad, double bias_correction1,
                                                   double bias_correction2, hipStream_t stream) {
    gsx_hip_adam_group g;
    g.parameter = parameter;
    g.gradient = gradient;
    g.first_moment = first_moment;
    g.second_moment = second_moment;
    g.count = total_elements;
    g.beta1 = beta1;
    g.beta2 = beta2;
    g.learning_rate = learning_rate;
    g.weight_decay = weight_decay;
    g.epsilon = epsilon;
    g.max_grad = max_grad;
    g.bias_correction1 = bias_correction1;
    g.bias_correction2 = bias_correction2;
    return gsx_hip_adam_step_multi_launch(&g, 1, stream);
}

}  // extern "C"
