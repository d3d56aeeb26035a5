// FP8 activation quantiser: bf16 hidden states [T, 7168] -> fp8 e4m3fn
// hidden_states [T, 7168] plus fp32 hidden_states_scale [56, T], the layout
// the MoE consumes (solution/triton/kernel.py:169 reads hs_scale[kb, t]).
//
// Per token and 128-element block: amax = max |x|, s = max(amax, 1e-10) / 448,
// q = e4m3(clamp(x / s, -448, 448)) rounded to nearest even. The division is
// IEEE fp32 (HIP's default correctly rounded divide), so q is bit-identical
// to the same formula in fp32 on the CPU.
//
// One 16-lane DPP row owns one (token, block): each lane loads 8 bf16 (16
// bytes), the row max is four xor-shuffles inside the row, and each lane
// stores 8 fp8 bytes. A 256-thread workgroup covers 16 consecutive tokens and
// NB blocks per token (all loads issued before any reduction), so the 16
// scales it writes per block are one contiguous 64-byte run of
// hidden_states_scale[b, t0 .. t0+15].
//
// quant_route_kernel runs the same quantiser and the routing kernel's work
// in one launch (they share no data): grid rows 0..HB/QUANT_NB-1 quantise a
// 16-token group as above, and 4 more rows route its 16 tokens, one per wave.
#include "route_impl.hpp"

namespace mimoe {

constexpr float FP8_MAX = 448.0f;
constexpr float QUANT_EPS = 1e-10f;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

constexpr int QUANT_NB = 2;  // blocks per token per workgroup (56 / 2 = 28 in y)

// Blocks by, by + HB/QUANT_NB, ... of the workgroup's 16 tokens.
__device__ __forceinline__ void quant_group(const uint16_t* __restrict__ x, int T,
                                            uint8_t* __restrict__ q, float* __restrict__ scale,
                                            int by) {
    const int t = blockIdx.x * 16 + (threadIdx.x >> 4);  // token of this 16-lane row
    const int sub = threadIdx.x & 15;                    // 8-element slice of the block
    const bool live = t < T;                             // uniform across the row
    float v[QUANT_NB][8];
    float amax[QUANT_NB];
#pragma unroll
    for (int j = 0; j < QUANT_NB; ++j) {
        amax[j] = 0.f;
        if (live) {
            const int b = by + j * (HB / QUANT_NB);
            const uint4 w = *reinterpret_cast<const uint4*>(x + (size_t)t * H + b * BLK + sub * 8);
            v[j][0] = bf16_lo(w.x); v[j][1] = bf16_hi(w.x);
            v[j][2] = bf16_lo(w.y); v[j][3] = bf16_hi(w.y);
            v[j][4] = bf16_lo(w.z); v[j][5] = bf16_hi(w.z);
            v[j][6] = bf16_lo(w.w); v[j][7] = bf16_hi(w.w);
        }
    }
#pragma unroll
    for (int j = 0; j < QUANT_NB; ++j) {
        if (live) {
#pragma unroll
            for (int i = 0; i < 8; ++i) amax[j] = fmaxf(amax[j], fabsf(v[j][i]));
        }
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1) amax[j] = fmaxf(amax[j], __shfl_xor(amax[j], m, 16));
    }
    if (!live) return;
#pragma unroll
    for (int j = 0; j < QUANT_NB; ++j) {
        const int b = by + j * (HB / QUANT_NB);
        const float s = fmaxf(amax[j], QUANT_EPS) / FP8_MAX;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = fminf(fmaxf(v[j][i] / s, -FP8_MAX), FP8_MAX);
        uint32_t lo = 0, hi = 0;
        lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[j][0], v[j][1], lo, false);
        lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[j][2], v[j][3], lo, true);
        hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[j][4], v[j][5], hi, false);
        hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[j][6], v[j][7], hi, true);
        *reinterpret_cast<uint2*>(q + (size_t)t * H + b * BLK + sub * 8) = make_uint2(lo, hi);
        if (sub == 0) scale[(size_t)b * T + t] = s;
    }
}

__global__ __launch_bounds__(256) void quant_fp8_kernel(const uint16_t* __restrict__ x, int T,
                                                         uint8_t* __restrict__ q,
                                                         float* __restrict__ scale) {
    quant_group(x, T, q, scale, blockIdx.y);
}

__global__ __launch_bounds__(256) void quant_route_kernel(
    const uint16_t* __restrict__ x, int T, uint8_t* __restrict__ q, float* __restrict__ scale,
    const float* __restrict__ logits, const void* __restrict__ bias, int bias_is_f32, float rsf,
    int* __restrict__ topk_ids, float* __restrict__ topk_w) {
    constexpr int QROWS = HB / QUANT_NB;
    if ((int)blockIdx.y < QROWS) {
        quant_group(x, T, q, scale, blockIdx.y);
        return;
    }
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 16 + (blockIdx.y - QROWS) * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    int ids[TOPK];
    float w[TOPK];
    route_token(logits + (size_t)t * EG, bias, bias_is_f32, rsf, lane, ids, w);
    if (lane == 0) store_topk_row(topk_ids + (size_t)t * TOPK_LD, topk_w + (size_t)t * TOPK_LD, ids, w);
}

hipError_t launch_quant_fp8(const void* x, int T, uint8_t* q, float* scale, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    static_assert(HB % QUANT_NB == 0, "blocks per workgroup");
    hipLaunchKernelGGL(quant_fp8_kernel, dim3((T + 15) / 16, HB / QUANT_NB), dim3(256), 0, s,
                       (const uint16_t*)x, T, q, scale);
    return hipGetLastError();
}

hipError_t launch_quant_route(const void* x, int T, uint8_t* q, float* scale, const float* logits,
                              const void* bias, int bias_is_f32, float rsf, int* topk_ids,
                              float* topk_w, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(quant_route_kernel, dim3((T + 15) / 16, HB / QUANT_NB + 4), dim3(256), 0, s,
                       (const uint16_t*)x, T, q, scale, logits, bias, bias_is_f32, rsf, topk_ids,
                       topk_w);
    return hipGetLastError();
}

}  // namespace mimoe
