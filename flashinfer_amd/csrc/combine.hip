// Weighted top-k combine to the bf16 output, without atomics.
//
// Replaces solution/triton/kernel.py:337-368 (_weighted_scatter_add_kernel,
// fp32 atomic_add, so its summation order varies run to run), the fp32
// zero-fill at :801, the bf16 cast at :820-823 and the empty-routing
// zero_() at :692-695. Each token gathers its <= 8 slot rows (already
// weighted by GEMM2's epilogue; bf16, or fp32 when GEMM2 wrote part_f32) in
// ascending local-expert order
// (tok_slot from the sort kernel) and sums them in fp32 in that fixed order;
// tokens with no local slot get zeros.
// Every output row is written exactly once, so results are bit-identical
// across runs.
#include "common.hpp"

namespace mimoe {

// Grid (T, H / 1024): one workgroup per token and 1024-column chunk; each
// thread owns 4 columns and issues the loads of all its <= 8 slot rows
// before summing them, so a call costs about one memory round trip. The bf16
// rows, read once, take the non-temporal hint (per call on MI355X, T=14000
// with every token on 8 experts, 1.6 GB of rows: 6,642-6,648 against
// 6,685-6,695 us on one box, 6,361-6,375 against 6,409-6,423 on another with
// non-temporal output stores as well; level at T <= 8192). The output keeps
// plain stores: the next layer reads it.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
template <bool F32>
__global__ __launch_bounds__(256) void combine_kernel(Plan p, uint16_t* __restrict__ out) {
    const int t = blockIdx.x;
    const int c = blockIdx.y * 1024 + threadIdx.x * 4;
    const int4 s0 = reinterpret_cast<const int4*>(p.tok_slot + (size_t)t * TOPK_LD)[0];
    const int4 s1 = reinterpret_cast<const int4*>(p.tok_slot + (size_t)t * TOPK_LD)[1];
    const int slot[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    float4 v[8];
#pragma unroll
    for (int j = 0; j < TOPK; ++j) {
        if constexpr (F32) {
            v[j] = slot[j] >= 0 ? *reinterpret_cast<const float4*>(p.part_f32 + (size_t)slot[j] * H + c)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
        } else {
            u32x2 u = {0u, 0u};
            if (slot[j] >= 0)
                u = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p.part + (size_t)slot[j] * H + c));
            v[j] = make_float4(bf2f(u.x & 0xffffu), bf2f(u.x >> 16), bf2f(u.y & 0xffffu),
                               bf2f(u.y >> 16));
        }
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < TOPK; ++j) {
        if (slot[j] < 0) break;
        acc.x += v[j].x;
        acc.y += v[j].y;
        acc.z += v[j].z;
        acc.w += v[j].w;
    }
    u32x2 o;
    o.x = (uint32_t)f2bf(acc.x) | ((uint32_t)f2bf(acc.y) << 16);
    o.y = (uint32_t)f2bf(acc.z) | ((uint32_t)f2bf(acc.w) << 16);
    *reinterpret_cast<u32x2*>(out + (size_t)t * H + c) = o;
}

hipError_t launch_combine(const Plan& p, uint16_t* out, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    if (p.part_f32)
        hipLaunchKernelGGL(combine_kernel<true>, dim3(p.T, H / 1024), dim3(256), 0, s, p, out);
    else
        hipLaunchKernelGGL(combine_kernel<false>, dim3(p.T, H / 1024), dim3(256), 0, s, p, out);
    return hipGetLastError();
}

}  // namespace mimoe
