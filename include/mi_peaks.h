/*
 * mi_peaks: achievable-peak probes for MI355X (gfx950), used to put the
 * fused MoE's measured rates beside what this GPU reaches on plain kernels.
 * Not part of the operator: no counterpart in the reference, which quotes
 * rates against the published peaks only. Built as libmi_peaks.so.
 *
 * All pointers are device pointers; every call only enqueues on `stream`
 * (a hipStream_t, NULL = default stream) and returns 0, or 1 for a bad
 * argument, or 3 if the launch failed.
 */
#ifndef MI_PEAKS_H_
#define MI_PEAKS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` (a multiple of 16, buf 16-byte aligned) with 16-byte loads
 * spread over `workgroups` workgroups of 256 threads; writes one int to
 * sink[0] only if the data's xor equals a constant no test buffer holds. */
int mi_peak_read(const void* buf, size_t bytes, int32_t workgroups, int32_t* sink, void* stream);

/* Copies `bytes` (a multiple of 16, both 16-byte aligned) src -> dst. */
int mi_peak_copy(void* dst, const void* src, size_t bytes, int32_t workgroups, void* stream);

/* Dense MFMA loops: each of `workgroups` x 4 waves runs `iters` rounds of 8
 * independent 16x16 MFMAs (kind 0: v_mfma_scale_f32_16x16x128_f8f6f4 with
 * unit scales, 65536 flops each; kind 1: v_mfma_f32_16x16x32_bf16, 16384
 * flops each). sink (fp32 [workgroups * 256]) receives the sums. */
int mi_peak_mfma(int32_t kind, int64_t iters, int32_t workgroups, float* sink, void* stream);

/* Flops one mi_peak_mfma call performs. */
double mi_peak_mfma_flops(int32_t kind, int64_t iters, int32_t workgroups);

#ifdef __cplusplus
}
#endif

#endif /* MI_PEAKS_H_ */
