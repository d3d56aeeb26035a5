// Routing kernel: one wavefront per token (see route_impl.hpp). Writes the
// global top-k ids and weights; the local filter (kernel.py:442-452) is
// applied by the sort, so these ids also serve the routing-parity check.
// PACKED rows hold exactly TOPK entries (the public routing entry point's
// [T, TOPK]); otherwise rows are TOPK_LD wide with padding (the workspace).
#include "route_impl.hpp"

namespace mimoe {

template <bool PACKED>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const void* __restrict__ bias, int bias_is_f32,
                                                    int T, float rsf, int* __restrict__ topk_ids,
                                                    float* __restrict__ topk_w) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    int ids[TOPK];
    float w[TOPK];
    route_token(logits + (size_t)t * EG, bias, bias_is_f32, rsf, lane, ids, w);
    if constexpr (PACKED) {
        // lane k writes entry k
        int id = ids[0];
        float wk = w[0];
#pragma unroll
        for (int k = 1; k < TOPK; ++k) {
            id = lane == k ? ids[k] : id;
            wk = lane == k ? w[k] : wk;
        }
        if (lane < TOPK) {
            topk_ids[(size_t)t * TOPK + lane] = id;
            topk_w[(size_t)t * TOPK + lane] = wk;
        }
    } else {
        if (lane == 0) store_topk_row(topk_ids + (size_t)t * TOPK_LD, topk_w + (size_t)t * TOPK_LD, ids, w);
    }
}

hipError_t launch_route(const float* logits, const void* bias, int bias_is_f32, int T, float rsf,
                        int* topk_ids, float* topk_w, hipStream_t s, bool packed) {
    if (T <= 0) return hipSuccess;
    dim3 grid((T + 3) / 4);
    if (packed)
        hipLaunchKernelGGL(route_kernel<true>, grid, dim3(256), 0, s, logits, bias, bias_is_f32, T,
                           rsf, topk_ids, topk_w);
    else
        hipLaunchKernelGGL(route_kernel<false>, grid, dim3(256), 0, s, logits, bias, bias_is_f32, T,
                           rsf, topk_ids, topk_w);
    return hipGetLastError();
}

}  // namespace mimoe
