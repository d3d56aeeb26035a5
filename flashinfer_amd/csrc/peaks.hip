// Achievable-peak probes (include/mi_peaks.h): an HBM read, an HBM copy and
// dense MFMA loops. They give the fused MoE's rates a measured ceiling beside
// the published one (8 TB/s HBM, 5.0 PFLOP/s dense fp8, 2.5 dense bf16).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mi_peaks.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int UNROLL = 8;  // independent 16-byte loads in flight per lane

// Each wave streams its own contiguous span of `per_wave` vectors (a
// multiple of 64): one load instruction covers 1 KB (8 whole 128-byte
// lines), UNROLL of them in flight. Contiguous spans per wave beat a
// grid-wide stride by ~8 %; non-temporal loads (the streaming hint, as the
// operator's weight streams use) read ~13 % faster than plain ones here.
__device__ __forceinline__ v4i ld_nt(const v4i* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void wave_span(size_t n, size_t per_wave, size_t& i, size_t& end) {
    const size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    i = wave * per_wave + (threadIdx.x & 63);
    end = wave * per_wave + per_wave;
    if (end > n) end = n;
}

__global__ __launch_bounds__(256) void read_kernel(const v4i* __restrict__ p, size_t n,
                                                   size_t per_wave, int32_t* sink) {
    size_t i, end;
    wave_span(n, per_wave, i, end);
    v4i acc = {0, 0, 0, 0};
    for (; i + (UNROLL - 1) * 64 < end; i += UNROLL * 64) {
        v4i r[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) r[u] = ld_nt(&p[i + u * 64]);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= r[u];
    }
    for (; i < end; i += 64) acc ^= ld_nt(&p[i]);
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5EED1234) sink[0] = 1;
}

__global__ __launch_bounds__(256) void copy_kernel(v4i* __restrict__ d, const v4i* __restrict__ s,
                                                   size_t n, size_t per_wave) {
    size_t i, end;
    wave_span(n, per_wave, i, end);
    for (; i + (UNROLL - 1) * 64 < end; i += UNROLL * 64) {
        v4i r[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) r[u] = ld_nt(&s[i + u * 64]);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) d[i + u * 64] = r[u];
    }
    for (; i < end; i += 64) d[i] = ld_nt(&s[i]);
}

// Vectors per wave so that workgroups x 4 waves cover n, rounded up to 64.
size_t span_per_wave(size_t n, int32_t workgroups) {
    const size_t waves = (size_t)workgroups * 4;
    const size_t per = (n + waves - 1) / waves;
    return (per + 63) / 64 * 64;
}

constexpr int CHAINS = 8;  // independent accumulators per wave

// kind 0: fp8 e4m3 operands 1.0 (0x38) x 0.5 (0x30), unit E8M0 scales;
// kind 1: bf16 operands 1.0 (0x3F80) x 0.5 (0x3F00).
template <int KIND>
__global__ __launch_bounds__(256) void mfma_kernel(int64_t iters, float* __restrict__ sink) {
    v4f c[CHAINS];
#pragma unroll
    for (int j = 0; j < CHAINS; ++j) c[j] = (v4f){0.f, 0.f, 0.f, 0.f};
    if constexpr (KIND == 0) {
        const int one = 0x38383838 + (int)(threadIdx.x >> 30);  // opaque to constant folding
        const v8i a = {one, one, one, one, one, one, one, one};
        const v8i b = {0x30303030, 0x30303030, 0x30303030, 0x30303030,
                       0x30303030, 0x30303030, 0x30303030, 0x30303030};
        for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < CHAINS; ++j)
                c[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c[j], 0, 0, 0, 127, 0,
                                                                        127);
        }
    } else {
        const int one = 0x3F803F80 + (int)(threadIdx.x >> 30);
        const v4i ai = {one, one, one, one};
        const v4i bi = {0x3F003F00, 0x3F003F00, 0x3F003F00, 0x3F003F00};
        const v8bf a = __builtin_bit_cast(v8bf, ai);
        const v8bf b = __builtin_bit_cast(v8bf, bi);
        for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int j = 0; j < CHAINS; ++j)
                c[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c[j], 0, 0, 0);
        }
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CHAINS; ++j) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    sink[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

bool bad_wg(int32_t wg) { return wg < 1 || wg > (1 << 20); }

int status(hipError_t e) { return e == hipSuccess ? 0 : 3; }

}  // namespace

extern "C" int mi_peak_read(const void* buf, size_t bytes, int32_t workgroups, int32_t* sink,
                            void* stream) {
    if (!buf || !sink || bytes == 0 || bytes % 16 || (uintptr_t)buf % 16 || bad_wg(workgroups))
        return 1;
    hipLaunchKernelGGL(read_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                       (const v4i*)buf, bytes / 16, span_per_wave(bytes / 16, workgroups), sink);
    return status(hipGetLastError());
}

extern "C" int mi_peak_copy(void* dst, const void* src, size_t bytes, int32_t workgroups,
                            void* stream) {
    if (!dst || !src || bytes == 0 || bytes % 16 || (uintptr_t)dst % 16 || (uintptr_t)src % 16 ||
        bad_wg(workgroups))
        return 1;
    hipLaunchKernelGGL(copy_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                       (v4i*)dst, (const v4i*)src, bytes / 16, span_per_wave(bytes / 16, workgroups));
    return status(hipGetLastError());
}

extern "C" int mi_peak_mfma(int32_t kind, int64_t iters, int32_t workgroups, float* sink,
                            void* stream) {
    if (!sink || iters < 1 || iters > (1LL << 30) || bad_wg(workgroups) || (kind != 0 && kind != 1))
        return 1;
    if (kind == 0)
        hipLaunchKernelGGL(mfma_kernel<0>, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                           iters, sink);
    else
        hipLaunchKernelGGL(mfma_kernel<1>, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                           iters, sink);
    return status(hipGetLastError());
}

extern "C" double mi_peak_mfma_flops(int32_t kind, int64_t iters, int32_t workgroups) {
    const double per = kind == 0 ? 2.0 * 16 * 16 * 128 : 2.0 * 16 * 16 * 32;
    return per * CHAINS * 4.0 * (double)workgroups * (double)iters;
}
