// DeepSeek no-aux routing of one token by one wavefront (device code shared
// by the routing kernel and the fused routing + sort kernel).
//
// Follows solution/triton/kernel.py:371-457 (_route_select_local_kernel),
// whose constexpr parameters E_GLOBAL, N_GROUP, TOPK_GROUP, TOP_K
// (kernel.py:371-389) are this build's EG, NGROUP, KGROUP, TOPK:
//   s = sigmoid(logit), sb = s + bias                               (:400-404)
//   group score = top1 + top2 of sb within each group of EG/NGROUP   (:406-416)
//   keep the KGROUP best groups                                      (:418-426)
//   pick the TOPK best experts by sb inside them                     (:428-438)
//   w_k = s_k * rsf / (sum_k s_k + 1e-20)                            (:440, :450)
// Ties resolve to the lowest index, like tl.argmax.
//
// Lane l of the wave owns experts EPL*l .. EPL*l+EPL-1 (EPL = EG/64), so one
// routing group is LPG adjacent lanes. Reductions use DPP lane exchanges (a
// few cycles each) and readlane, not LDS permutes: the group top-2 is up to
// four DPP merges, and each of the TOPK top-k rounds is one 4-step DPP max,
// 4 readlanes and a ballot for the lowest index. No LDS, no barriers, one
// coalesced load of the token's logits row.
#pragma once

#include "common.hpp"

namespace mimoe {

__device__ __forceinline__ uint32_t ord_f32(float f) {
    // Monotone map float -> uint32 (larger float -> larger key).
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// DPP lane exchanges (gfx9 encodings): xor 1 / xor 2 inside a quad, mirror
// inside each 8-lane half row, mirror inside each 16-lane row.
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, dpp_u<CTRL>(__builtin_bit_cast(uint32_t, v)));
}

__device__ __forceinline__ void top2_merge(float& m1, float& m2, float o1, float o2) {
    const float n1 = fmaxf(m1, o1);
    const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
    m1 = n1;
    m2 = n2;
}

// Largest key of the wave, returned in every lane (uniform).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t k) {
    k = max(k, dpp_u<DPP_XOR1>(k));
    k = max(k, dpp_u<DPP_XOR2>(k));
    k = max(k, dpp_u<DPP_HALF_MIRROR>(k));
    k = max(k, dpp_u<DPP_MIRROR>(k));  // every lane now holds its 16-lane row's max
    const uint32_t r0 = __builtin_amdgcn_readlane(k, 0);
    const uint32_t r1 = __builtin_amdgcn_readlane(k, 16);
    const uint32_t r2 = __builtin_amdgcn_readlane(k, 32);
    const uint32_t r3 = __builtin_amdgcn_readlane(k, 48);
    return max(max(r0, r1), max(r2, r3));
}

// Routes one token's logits row ([EG] fp32). Every lane of the wave gets the
// same ids (selection order) and weights.
__device__ __forceinline__ void route_token(const float* __restrict__ logits_row,
                                            const void* __restrict__ bias, int bias_is_f32,
                                            float rsf, int lane, int ids[TOPK], float wts[TOPK]) {
    static_assert(EPL == 1 || EPL == 2 || EPL == 4, "64, 128 or 256 global experts");
    float x[EPL], bb[EPL];
    if constexpr (EPL == 4) {
        const float4 v = reinterpret_cast<const float4*>(logits_row)[lane];
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        if (bias_is_f32) {
            const float4 b = reinterpret_cast<const float4*>(bias)[lane];
            bb[0] = b.x; bb[1] = b.y; bb[2] = b.z; bb[3] = b.w;
        } else {
            const uint2 raw = reinterpret_cast<const uint2*>(bias)[lane];
            bb[0] = bf2f(raw.x & 0xffffu); bb[1] = bf2f(raw.x >> 16);
            bb[2] = bf2f(raw.y & 0xffffu); bb[3] = bf2f(raw.y >> 16);
        }
    } else if constexpr (EPL == 2) {
        const float2 v = reinterpret_cast<const float2*>(logits_row)[lane];
        x[0] = v.x; x[1] = v.y;
        if (bias_is_f32) {
            const float2 b = reinterpret_cast<const float2*>(bias)[lane];
            bb[0] = b.x; bb[1] = b.y;
        } else {
            const uint32_t raw = reinterpret_cast<const uint32_t*>(bias)[lane];
            bb[0] = bf2f(raw & 0xffffu); bb[1] = bf2f(raw >> 16);
        }
    } else {
        x[0] = logits_row[lane];
        bb[0] = bias_is_f32 ? reinterpret_cast<const float*>(bias)[lane]
                            : bf2f(reinterpret_cast<const uint16_t*>(bias)[lane]);
    }
    float s[EPL], sb[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) { s[j] = sigmoid_f32(x[j]); sb[j] = s[j] + bb[j]; }

    // Top-2 (as a multiset) of the lane's values, then of the LPG-lane group.
    float m1, m2;
    if constexpr (EPL == 1) {
        m1 = sb[0];
        m2 = -__builtin_inff();
    } else {
        m1 = fmaxf(sb[0], sb[1]);
        m2 = fminf(sb[0], sb[1]);
#pragma unroll
        for (int j = 2; j < EPL; ++j) {
            const float v = sb[j];
            if (v > m1) { m2 = m1; m1 = v; } else { m2 = fmaxf(m2, v); }
        }
    }
    top2_merge(m1, m2, dpp_f<DPP_XOR1>(m1), dpp_f<DPP_XOR1>(m2));
    if constexpr (LPG >= 4) top2_merge(m1, m2, dpp_f<DPP_XOR2>(m1), dpp_f<DPP_XOR2>(m2));
    if constexpr (LPG >= 8)
        top2_merge(m1, m2, dpp_f<DPP_HALF_MIRROR>(m1), dpp_f<DPP_HALF_MIRROR>(m2));
    if constexpr (LPG >= 16) top2_merge(m1, m2, dpp_f<DPP_MIRROR>(m1), dpp_f<DPP_MIRROR>(m2));
    const float gscore = m1 + m2;  // identical in the LPG lanes of the group

    // Rank of this lane's group among the NGROUP (lower index wins ties).
    const int my_g = lane / LPG;
    int rank = 0;
#pragma unroll
    for (int h = 0; h < NGROUP; ++h) {
        const float gh = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, gscore), h * LPG));
        rank += (gh > gscore) || (gh == gscore && h < my_g);
    }
    const bool gsel = rank < KGROUP;

    // Candidate keys: order-preserving image of s+bias; 0 = not a candidate
    // (ord_f32 maps every non-NaN float, -inf included, above 0).
    uint32_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) key[j] = gsel ? ord_f32(sb[j]) : 0u;

    float ss[TOPK];
#pragma unroll
    for (int k = 0; k < TOPK; ++k) {
        uint32_t local = key[0];
#pragma unroll
        for (int j = 1; j < EPL; ++j) local = max(local, key[j]);
        const uint32_t best = wave_max_u32(local);
        // Lowest expert index holding the best key: lowest lane, then lowest j.
        const unsigned long long holders = __ballot(local == best);
        const int owner = __builtin_ctzll(holders);
        int jj = EPL - 1;
#pragma unroll
        for (int j = EPL - 2; j >= 0; --j) jj = key[j] == best ? j : jj;
        const int j_owner = __builtin_amdgcn_readlane(jj, owner);
        float sv = s[0];
#pragma unroll
        for (int j = 1; j < EPL; ++j) sv = j_owner == j ? s[j] : sv;
        ss[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), owner));
        ids[k] = owner * EPL + j_owner;
#pragma unroll
        for (int j = 0; j < EPL; ++j) key[j] = (lane == owner && j == j_owner) ? 0u : key[j];
    }
    float denom = ss[0];
#pragma unroll
    for (int k = 1; k < TOPK; ++k) denom += ss[k];
    // w_k = s_k * rsf / (sum + 1e-20): one division per token, then products
    // (within 2 ulp of the per-weight division of kernel.py:450).
    const float scale = rsf / (denom + 1e-20f);
#pragma unroll
    for (int k = 0; k < TOPK; ++k) wts[k] = ss[k] * scale;
}

}  // namespace mimoe
