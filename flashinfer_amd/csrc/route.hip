// Routing kernel: one wavefront per token (see route_impl.hpp). Writes the
// global top-8 ids and weights; the local filter (kernel.py:442-452) is
// applied by the sort, so these ids also serve the routing-parity check.
#include "route_impl.hpp"

namespace mimoe {

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
    if (lane == 0) {
        int4* io = reinterpret_cast<int4*>(topk_ids + (size_t)t * TOPK);
        float4* wo = reinterpret_cast<float4*>(topk_w + (size_t)t * TOPK);
        io[0] = make_int4(ids[0], ids[1], ids[2], ids[3]);
        io[1] = make_int4(ids[4], ids[5], ids[6], ids[7]);
        wo[0] = make_float4(w[0], w[1], w[2], w[3]);
        wo[1] = make_float4(w[4], w[5], w[6], w[7]);
    }
}

hipError_t launch_route(const float* logits, const void* bias, int bias_is_f32, int T, float rsf,
                        int* topk_ids, float* topk_w, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    dim3 grid((T + 3) / 4);
    hipLaunchKernelGGL(route_kernel, grid, dim3(256), 0, s, logits, bias, bias_is_f32, T, rsf,
                       topk_ids, topk_w);
    return hipGetLastError();
}

}  // namespace mimoe
