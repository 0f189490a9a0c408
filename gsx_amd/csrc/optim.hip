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
constexpr int kAdamItems = 4;  // float4 per thread
constexpr int kAdamChunk = kAdamThreads * kAdamItems;

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

__global__ __launch_bounds__(kAdamThreads) void adam_multi_kernel(AdamBatch batch) {
    int k = 0;
    while (k + 1 < batch.group_count && blockIdx.x >= batch.block_start[k + 1]) ++k;
    const gsx_hip_adam_group& gr = batch.groups[k];
    const int64_t base = ((int64_t)(blockIdx.x - batch.block_start[k]) * kAdamChunk) + (int64_t)threadIdx.x * kAdamItems;
    const int64_t n = gr.count;
    if (base + kAdamItems <= n && ((reinterpret_cast<uintptr_t>(gr.parameter) | reinterpret_cast<uintptr_t>(gr.gradient) |
                                    reinterpret_cast<uintptr_t>(gr.first_moment) |
                                    reinterpret_cast<uintptr_t>(gr.second_moment)) & 15u) == 0) {
        float4 p = *reinterpret_cast<const float4*>(gr.parameter + base);
        const float4 g = *reinterpret_cast<const float4*>(gr.gradient + base);
        float4 m = *reinterpret_cast<const float4*>(gr.first_moment + base);
        float4 v = *reinterpret_cast<const float4*>(gr.second_moment + base);
        p.x = adam_element(p.x, g.x, m.x, v.x, gr);
        p.y = adam_element(p.y, g.y, m.y, v.y, gr);
        p.z = adam_element(p.z, g.z, m.z, v.z, gr);
        p.w = adam_element(p.w, g.w, m.w, v.w, gr);
        *reinterpret_cast<float4*>(gr.parameter + base) = p;
        *reinterpret_cast<float4*>(gr.first_moment + base) = m;
        *reinterpret_cast<float4*>(gr.second_moment + base) = v;
    } else {
        for (int i = 0; i < kAdamItems; ++i) {
            const int64_t e = base + i;
            if (e >= n) break;
            float m = gr.first_moment[e];
            float v = gr.second_moment[e];
            gr.parameter[e] = adam_element(gr.parameter[e], gr.gradient[e], m, v, gr);
            gr.first_moment[e] = m;
            gr.second_moment[e] = v;
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
    uint64_t blocks = 0;
    for (int k = 0; k < group_count; ++k) {
        if (groups[k].count < 0) return GSX_HIP_ERROR_INVALID_ARGUMENT;
        if (groups[k].count > 0 && (groups[k].parameter == nullptr || groups[k].gradient == nullptr ||
                                    groups[k].first_moment == nullptr || groups[k].second_moment == nullptr)) {
            return GSX_HIP_ERROR_INVALID_ARGUMENT;
        }
        batch.groups[k] = groups[k];
        batch.block_start[k] = (uint32_t)blocks;
        blocks += (uint64_t)((groups[k].count + kAdamChunk - 1) / kAdamChunk);
        if (blocks > 0x7fffffffu) return GSX_HIP_ERROR_OUT_OF_RANGE;
    }
    batch.block_start[group_count] = (uint32_t)blocks;
    if (blocks == 0) return GSX_HIP_SUCCESS;
    hipLaunchKernelGGL(adam_multi_kernel, dim3((unsigned)blocks), dim3(kAdamThreads), 0, stream, batch);
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
