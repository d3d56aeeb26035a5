// FP8 activation quantiser: bf16 hidden states [T, 7168] -> fp8 e4m3fn
// hidden_states [T, 7168] plus fp32 hidden_states_scale [56, T], the layout
// the MoE consumes (solution/triton/kernel.py:169 reads hs_scale[kb, t]).
//
// Per token and 128-element block: amax = max |x|, s = max(amax, 1e-10) / 448,
// q = e4m3(clamp(x / s, -448, 448)) rounded to nearest even. The division is
// IEEE fp32 (HIP's default correctly rounded divide), so q is bit-identical
// to the same formula in fp32 on the CPU.
//
// One 16-lane DPP row owns one block: each lane loads 8 bf16 (16 bytes), the
// row max is four xor-shuffles inside the row, and each lane stores 8 fp8
// bytes, so a row reads 256 contiguous bytes and writes 128. A 256-thread
// workgroup covers 16 consecutive blocks of the flattened [T * 56] block list.
#include "common.hpp"

namespace mimoe {

constexpr float FP8_MAX = 448.0f;
constexpr float QUANT_EPS = 1e-10f;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__global__ __launch_bounds__(256) void quant_fp8_kernel(const uint16_t* __restrict__ x, int T,
                                                         uint8_t* __restrict__ q,
                                                         float* __restrict__ scale) {
    const int blk = blockIdx.x * 16 + (threadIdx.x >> 4);  // flattened (token, block)
    const int sub = threadIdx.x & 15;                      // 8-element slice of the block
    const bool live = blk < T * HB;                        // uniform across the 16-lane row
    float v[8];
    float amax = 0.f;
    if (live) {
        const uint4 w = *reinterpret_cast<const uint4*>(x + (size_t)blk * BLK + sub * 8);
        v[0] = bf16_lo(w.x); v[1] = bf16_hi(w.x);
        v[2] = bf16_lo(w.y); v[3] = bf16_hi(w.y);
        v[4] = bf16_lo(w.z); v[5] = bf16_hi(w.z);
        v[6] = bf16_lo(w.w); v[7] = bf16_hi(w.w);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 16));
    if (!live) return;
    const float s = fmaxf(amax, QUANT_EPS) / FP8_MAX;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = fminf(fmaxf(v[i] / s, -FP8_MAX), FP8_MAX);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[4], v[5], hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[6], v[7], hi, true);
    *reinterpret_cast<uint2*>(q + (size_t)blk * BLK + sub * 8) = make_uint2(lo, hi);
    if (sub == 0) {
        const int t = blk / HB, b = blk - t * HB;
        scale[(size_t)b * T + t] = s;
    }
}

hipError_t launch_quant_fp8(const void* x, int T, uint8_t* q, float* scale, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    const int blocks = T * HB;
    hipLaunchKernelGGL(quant_fp8_kernel, dim3((blocks + 15) / 16), dim3(256), 0, s,
                       (const uint16_t*)x, T, q, scale);
    return hipGetLastError();
}

}  // namespace mimoe
