// Local-expert histogram, prefix sum and stable permute in one workgroup.
//
// Replaces solution/triton/kernel.py:460-505 (_count_local_experts_kernel,
// _scatter_local_tokens_kernel), the host-synchronising scan at :572-581 and
// the tile prefix of :508-516 (+ .item() at :718, :773). Differences:
//   * the slot order inside an expert is token-ascending (deterministic);
//     the reference's atomic_add order (:503) is not;
//   * nothing returns to the host: S, the expert offsets and the per-GEMM
//     row-tile prefixes stay in the workspace for the GEMM kernels;
//   * it also writes, per token, its slots in ascending local-expert order,
//     which the combine kernel walks instead of scattering with atomics.
//
// Placement works per chunk of 1024 tokens: each wave counts its 64 tokens'
// hits per expert with one ballot per expert, the 16 wave counts are scanned
// in LDS, and a lane's slot is chunk base + wave prefix + popcount of the
// lower lanes' ballot bits.
#include "common.hpp"

namespace mimoe {

__global__ __launch_bounds__(1024) void sort_kernel(Plan p, int bm1, int bm2) {
    __shared__ int cnt[EL];
    __shared__ int base[EL];
    __shared__ int wcnt[16][EL];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int T = p.T;
    const int off = p.local_offset;

    if (tid < EL) cnt[tid] = 0;
    __syncthreads();
    for (int t = tid; t < T; t += 1024) {
        const int4 i0 = reinterpret_cast<const int4*>(p.topk_ids + (size_t)t * TOPK)[0];
        const int4 i1 = reinterpret_cast<const int4*>(p.topk_ids + (size_t)t * TOPK)[1];
        const int ids[8] = {i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w};
#pragma unroll
        for (int k = 0; k < TOPK; ++k) {
            const int l = ids[k] - off;
            if ((unsigned)l < (unsigned)EL) atomicAdd(&cnt[l], 1);
        }
    }
    __syncthreads();
    if (tid < 64) {
        // Exclusive prefix of slot counts and of row tiles, 32 lanes in parallel.
        const int c = tid < EL ? cnt[tid] : 0;
        int v0 = c, v1 = (c + bm1 - 1) / bm1, v2 = (c + bm2 - 1) / bm2;
        const int own0 = v0, own1 = v1, own2 = v2;
#pragma unroll
        for (int d = 1; d < EL; d <<= 1) {
            const int u0 = __shfl_up(v0, d), u1 = __shfl_up(v1, d), u2 = __shfl_up(v2, d);
            if (tid >= d) { v0 += u0; v1 += u1; v2 += u2; }
        }
        if (tid < EL) {
            p.meta[META_EXPERT_OFF + tid] = v0 - own0;
            p.meta[META_MTILE1 + tid] = v1 - own1;
            p.meta[META_MTILE2 + tid] = v2 - own2;
            base[tid] = v0 - own0;
            if (tid == EL - 1) {
                p.meta[META_EXPERT_OFF + EL] = v0;
                p.meta[META_MTILE1 + EL] = v1;
                p.meta[META_MTILE2 + EL] = v2;
            }
        }
    }
    __syncthreads();

    const unsigned long long lower = (1ull << lane) - 1ull;
    for (int c0 = 0; c0 < T; c0 += 1024) {
        const int t = c0 + tid;
        const bool valid = t < T;
        int lid[TOPK];
        float lw[TOPK];
        uint32_t m = 0;
        if (valid) {
            const int4 i0 = reinterpret_cast<const int4*>(p.topk_ids + (size_t)t * TOPK)[0];
            const int4 i1 = reinterpret_cast<const int4*>(p.topk_ids + (size_t)t * TOPK)[1];
            const float4 w0 = reinterpret_cast<const float4*>(p.topk_w + (size_t)t * TOPK)[0];
            const float4 w1 = reinterpret_cast<const float4*>(p.topk_w + (size_t)t * TOPK)[1];
            const int ids[8] = {i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w};
            const float ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int k = 0; k < TOPK; ++k) {
                const int l = ids[k] - off;
                const bool loc = (unsigned)l < (unsigned)EL;
                lid[k] = loc ? l : -1;
                lw[k] = ws[k];
                m |= loc ? (1u << l) : 0u;
            }
        } else {
#pragma unroll
            for (int k = 0; k < TOPK; ++k) { lid[k] = -1; lw[k] = 0.f; }
        }
#pragma unroll
        for (int e = 0; e < EL; ++e) {
            const unsigned long long bal = __ballot((m >> e) & 1u);
            if (lane == e) wcnt[wave][e] = __popcll(bal);
        }
        __syncthreads();
        if (tid < EL) {
            int run = base[tid];
            for (int w = 0; w < 16; ++w) {
                const int c = wcnt[w][tid];
                wcnt[w][tid] = run;
                run += c;
            }
            base[tid] = run;
        }
        __syncthreads();
        int j = 0;
#pragma unroll
        for (int e = 0; e < EL; ++e) {
            const bool hit = (m >> e) & 1u;
            const unsigned long long bal = __ballot(hit);
            if (hit) {
                const int pos = wcnt[wave][e] + __popcll(bal & lower);
                float w = 0.f;
#pragma unroll
                for (int k = 0; k < TOPK; ++k) w = (lid[k] == e) ? lw[k] : w;
                p.sorted_tok[pos] = t;
                p.sorted_w[pos] = w;
                p.tok_slot[(size_t)t * TOPK + j] = pos;
                ++j;
            }
        }
        if (valid)
            for (; j < TOPK; ++j) p.tok_slot[(size_t)t * TOPK + j] = -1;
        __syncthreads();
    }
}

hipError_t launch_sort(const Plan& p, int bm1, int bm2, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    hipLaunchKernelGGL(sort_kernel, dim3(1), dim3(1024), 0, s, p, bm1, bm2);
    return hipGetLastError();
}

}  // namespace mimoe
