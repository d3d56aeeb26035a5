// DeepSeek no-aux routing, one wavefront per token.
//
// Follows solution/triton/kernel.py:371-457 (_route_select_local_kernel):
//   s = sigmoid(logit), sb = s + bias                        (:400-404)
//   group score = top1 + top2 of sb within each group of 32  (:406-416)
//   keep the 4 best groups                                   (:418-426)
//   pick the 8 best experts by sb inside them                (:428-438)
//   w_k = s_k * rsf / (sum_k s_k + 1e-20)                    (:440, :450)
// Ties resolve to the lowest index, like tl.argmax. The local filter
// (:442-452) is applied later by the sort kernel, so this kernel writes the
// global ids, which also serve the routing-parity check.
//
// Lane l of the wave owns experts 4l..4l+3, so one routing group is 8 lanes
// and every reduction is a short butterfly inside the wave: no LDS, no
// barriers, one 1 KB coalesced load of logits per token.
#include "common.hpp"

namespace mimoe {

__device__ __forceinline__ uint32_t ord_f32(float f) {
    // Monotone map float -> uint32 (larger float -> larger key).
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const void* __restrict__ bias, int bias_is_f32,
                                                    int T, float rsf, int* __restrict__ topk_ids,
                                                    float* __restrict__ topk_w) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;

    const float4 x = reinterpret_cast<const float4*>(logits + (size_t)t * EG)[lane];
    float b0, b1, b2, b3;
    if (bias_is_f32) {
        const float4 bb = reinterpret_cast<const float4*>(bias)[lane];
        b0 = bb.x; b1 = bb.y; b2 = bb.z; b3 = bb.w;
    } else {
        const uint2 raw = reinterpret_cast<const uint2*>(bias)[lane];
        b0 = bf2f(raw.x & 0xffffu); b1 = bf2f(raw.x >> 16);
        b2 = bf2f(raw.y & 0xffffu); b3 = bf2f(raw.y >> 16);
    }
    float s[4] = {sigmoid_f32(x.x), sigmoid_f32(x.y), sigmoid_f32(x.z), sigmoid_f32(x.w)};
    float sb[4] = {s[0] + b0, s[1] + b1, s[2] + b2, s[3] + b3};

    // Top-2 (as a multiset) of the lane's 4 values, then of the 8-lane group.
    float m1 = fmaxf(sb[0], sb[1]), m2 = fminf(sb[0], sb[1]);
#pragma unroll
    for (int j = 2; j < 4; ++j) {
        const float v = sb[j];
        if (v > m1) { m2 = m1; m1 = v; } else { m2 = fmaxf(m2, v); }
    }
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        const float o1 = __shfl_xor(m1, off);
        const float o2 = __shfl_xor(m2, off);
        const float n1 = fmaxf(m1, o1);
        const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
        m1 = n1; m2 = n2;
    }
    const float gscore = m1 + m2;

    // Rank of this lane's group among the 8 (lower index wins ties).
    const int my_g = lane >> 3;
    int rank = 0;
#pragma unroll
    for (int h = 0; h < NGROUP; ++h) {
        const float gh = __shfl(gscore, h * 8);
        rank += (gh > gscore) || (gh == gscore && h < my_g);
    }
    const bool gsel = rank < KGROUP;

    // 64-bit keys: ordered score in the high word, (255 - id) in the low word,
    // so one max picks the best score and, on ties, the lowest id.
    unsigned long long key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        key[j] = gsel ? (((unsigned long long)ord_f32(sb[j]) << 32) |
                         (unsigned long long)(uint32_t)(255 - (lane * 4 + j)))
                      : 0ull;

    int ids[TOPK];
    float ss[TOPK];
#pragma unroll
    for (int k = 0; k < TOPK; ++k) {
        unsigned long long best = key[0];
#pragma unroll
        for (int j = 1; j < 4; ++j) best = key[j] > best ? key[j] : best;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const unsigned long long o = __shfl_xor(best, off);
            best = o > best ? o : best;
        }
        const int idx = 255 - (int)(uint32_t)(best & 0xffffffffull);
        const int owner = idx >> 2;
        const int jj = idx & 3;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane == owner && j == jj) key[j] = 0ull;
        float sv = jj == 0 ? s[0] : (jj == 1 ? s[1] : (jj == 2 ? s[2] : s[3]));
        sv = __shfl(sv, owner);
        ids[k] = idx;
        ss[k] = sv;
    }
    float denom = ss[0];
#pragma unroll
    for (int k = 1; k < TOPK; ++k) denom += ss[k];
    const float inv_den = denom + 1e-20f;

    if (lane == 0) {
        int4* io = reinterpret_cast<int4*>(topk_ids + (size_t)t * TOPK);
        float4* wo = reinterpret_cast<float4*>(topk_w + (size_t)t * TOPK);
        io[0] = make_int4(ids[0], ids[1], ids[2], ids[3]);
        io[1] = make_int4(ids[4], ids[5], ids[6], ids[7]);
        wo[0] = make_float4(ss[0] * rsf / inv_den, ss[1] * rsf / inv_den, ss[2] * rsf / inv_den,
                            ss[3] * rsf / inv_den);
        wo[1] = make_float4(ss[4] * rsf / inv_den, ss[5] * rsf / inv_den, ss[6] * rsf / inv_den,
                            ss[7] * rsf / inv_den);
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
