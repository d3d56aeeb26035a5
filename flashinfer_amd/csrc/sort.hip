// Local-expert histogram, prefix sum and stable permute.
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
// Placement works per chunk of tokens (one per thread: 1024 in the one-
// workgroup sort, SORT_CHUNK_L in the two-pass sort for larger T): each wave
// counts its 64 tokens' hits per expert with one ballot per expert, the wave
// counts are scanned in LDS, and a lane's slot is chunk base + wave prefix +
// popcount of the lower lanes' ballot bits.
//
// Entry shapes: one wave for T <= 64 (sort_small_kernel); one workgroup for
// T <= 1024 (sort_kernel); either with the routing done in place for small T
// (route_sort_kernel, one launch for the whole front end); and for large T a
// per-chunk count kernel plus a per-chunk place kernel that scans the chunk
// totals itself. At decode sizes the K-split GEMM1 kernel can take the sort's
// place instead: each of its waves finds its row tile from the top-k ids, and
// one workgroup writes these tables for GEMM2 and the combine (gemm1.hip).
#include "route_impl.hpp"
#include "sort_impl.hpp"

namespace mimoe {

constexpr int CHUNK = SORT_CHUNK;

// Per-wave hit counts of the chunk into wcnt[wave][e] (lane e writes).
__device__ __forceinline__ void wave_counts(const TokLocal& tl, int lane, int wave,
                                            int (*wcnt)[EL]) {
#pragma unroll
    for (int e = 0; e < EL; ++e) {
        const unsigned long long bal = __ballot((tl.m >> e) & 1u);
        if (lane == e) wcnt[wave][e] = __popcll(bal);
    }
}

// Places one chunk (every thread of the 1024-thread workgroup calls it).
// base[e] holds the chunk's first slot for expert e.
template <int CH>
__device__ void place_chunk(const Plan& p, int t, bool valid, const TokLocal& tl, const int* base,
                            int (*wcnt)[EL], int tid, int lane, int wave) {
    wave_counts(tl, lane, wave, wcnt);
    __syncthreads();
    if (tid < EL) {
        int run = base[tid];
        for (int w = 0; w < CH / 64; ++w) {
            const int c = wcnt[w][tid];
            wcnt[w][tid] = run;
            run += c;
        }
    }
    __syncthreads();
    place_with_prefix(p, t, valid, tl, wcnt, lane, wave);
}

// Counts, scan and placement for T <= CHUNK in one workgroup, reading each
// token's top-k once from ids_base / w_base (global or LDS): the per-wave
// ballot counts give both the expert totals and the wave prefixes.
__device__ void sort_one_workgroup(const Plan& p, const int* ids_base, const float* w_base, int bm1,
                                   int bm2, int (*wcnt)[EL]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool valid = tid < p.T;
    const TokLocal tl = load_local(ids_base, w_base, tid, valid, p.local_offset);
    wave_counts(tl, lane, wave, wcnt);
    __syncthreads();
    if (wave == 0) {
        int total = 0;
        if (lane < EL)
            for (int w = 0; w < CHUNK / 64; ++w) total += wcnt[w][lane];
        const int off = scan_counts(p, lane, total, bm1, bm2, true);
        if (lane < EL) {
            int run = off;
            for (int w = 0; w < CHUNK / 64; ++w) {
                const int c = wcnt[w][lane];
                wcnt[w][lane] = run;
                run += c;
            }
        }
    }
    __syncthreads();
    place_with_prefix(p, tid, valid, tl, wcnt, lane, wave);
}

// T <= 64: one wave (sort_one_wave: ballots and a shuffle scan, no LDS).
__global__ __launch_bounds__(64) void sort_small_kernel(Plan p, int bm1, int bm2) {
    sort_one_wave(p, p.topk_ids, p.topk_w, bm1, bm2, threadIdx.x);
}

__global__ __launch_bounds__(1024) void sort_kernel(Plan p, int bm1, int bm2) {
    __shared__ int wcnt[CHUNK / 64][EL];
    sort_one_workgroup(p, p.topk_ids, p.topk_w, bm1, bm2, wcnt);
}

// Routing + sort in one launch for small T: the 16 waves route the tokens
// round-robin (global top-k also written for parity checks), then sort from
// the LDS copy (one wave for T <= 64).
constexpr int ROUTE_SORT_MAX_T = 256;

__global__ __launch_bounds__(1024) void route_sort_kernel(Plan p, const float* __restrict__ logits,
                                                          const void* __restrict__ bias,
                                                          int bias_is_f32, int bm1, int bm2) {
    __shared__ int wcnt[CHUNK / 64][EL];
    __shared__ __attribute__((aligned(16))) int s_ids[ROUTE_SORT_MAX_T * TOPK_LD];
    __shared__ __attribute__((aligned(16))) float s_w[ROUTE_SORT_MAX_T * TOPK_LD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int t = wave; t < p.T; t += CHUNK / 64) {
        int ids[TOPK];
        float w[TOPK];
        route_token(logits + (size_t)t * EG, bias, bias_is_f32, p.rsf, lane, ids, w);
        if (lane == 0) {
            store_topk_row(p.topk_ids + (size_t)t * TOPK_LD, p.topk_w + (size_t)t * TOPK_LD, ids, w);
            store_topk_row(s_ids + t * TOPK_LD, s_w + t * TOPK_LD, ids, w);
        }
    }
    __syncthreads();
    if (p.T <= SMALL_T) {
        if (wave == 0) sort_one_wave(p, s_ids, s_w, bm1, bm2, lane);
        return;
    }
    sort_one_workgroup(p, s_ids, s_w, bm1, bm2, wcnt);
}

// Large T, pass 1: per-chunk (SORT_CHUNK_L tokens) expert totals into chunk_cnt[chunk][EL].
__global__ __launch_bounds__(SORT_CHUNK_L) void sort_count_kernel(Plan p) {
    __shared__ int wcnt[SORT_CHUNK_L / 64][EL];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t = blockIdx.x * SORT_CHUNK_L + tid;
    const bool valid = t < p.T;
    const TokLocal tl = load_local(p.topk_ids, p.topk_w, t, valid, p.local_offset);
    wave_counts(tl, lane, wave, wcnt);
    __syncthreads();
    if (tid < EL) {
        int s = 0;
        for (int w = 0; w < SORT_CHUNK_L / 64; ++w) s += wcnt[w][tid];
        p.chunk_cnt[blockIdx.x * EL + tid] = s;
    }
}

// Large T, pass 2: each chunk derives its per-expert base from the chunk
// totals (chunk 0 also writes the expert offsets and tile prefixes), then
// places its tokens.
__global__ __launch_bounds__(SORT_CHUNK_L) void sort_place_kernel(Plan p, int nchunks, int bm1, int bm2) {
    __shared__ int base[EL];
    __shared__ int s_before[EL], s_total[EL];
    __shared__ int wcnt[SORT_CHUNK_L / 64][EL];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cb = blockIdx.x;
    // The chunk's top-k rows are loaded first, so their round trip overlaps
    // the chunk totals'.
    const int t = cb * SORT_CHUNK_L + tid;
    const bool valid = t < p.T;
    const TokLocal tl = load_local(p.topk_ids, p.topk_w, t, valid, p.local_offset);
    // Chunk totals, every (chunk, expert) count loaded by its own thread (one
    // round trip, not one per chunk) and summed with LDS integer atomics
    // (exact, so the order does not matter).
    if (tid < EL) { s_before[tid] = 0; s_total[tid] = 0; }
    __syncthreads();
    for (int i = tid; i < nchunks * EL; i += SORT_CHUNK_L) {
        const int v = p.chunk_cnt[i];
        const int c = i / EL, e = i % EL;
        if (v) {
            atomicAdd(&s_total[e], v);
            if (c < cb) atomicAdd(&s_before[e], v);
        }
    }
    __syncthreads();
    if (wave == 0) {
        const int total = lane < EL ? s_total[lane] : 0;
        const int off = scan_counts(p, lane, total, bm1, bm2, cb == 0);
        if (lane < EL) base[lane] = off + s_before[lane];
    }
    __syncthreads();
    place_chunk<SORT_CHUNK_L>(p, t, valid, tl, base, wcnt, tid, lane, wave);
}

bool route_sort_supported(int T) { return T > 0 && T <= ROUTE_SORT_MAX_T; }

__global__ __launch_bounds__(256) void repack_topk_kernel(const int* __restrict__ ids,
                                                          const float* __restrict__ w, int T,
                                                          int* __restrict__ out_ids,
                                                          float* __restrict__ out_w) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= T) return;
    int iv[TOPK];
    float wv[TOPK];
#pragma unroll
    for (int k = 0; k < TOPK; ++k) {
        iv[k] = ids[(size_t)t * TOPK + k];
        wv[k] = w[(size_t)t * TOPK + k];
    }
    store_topk_row(out_ids + (size_t)t * TOPK_LD, out_w + (size_t)t * TOPK_LD, iv, wv);
}

hipError_t launch_repack_topk(const int* ids, const float* w, int T, int* out_ids, float* out_w,
                              hipStream_t s) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(repack_topk_kernel, dim3((T + 255) / 256), dim3(256), 0, s, ids, w, T,
                       out_ids, out_w);
    return hipGetLastError();
}

hipError_t launch_route_sort(const Plan& p, const float* logits, const void* bias, int bias_is_f32,
                             int bm1, int bm2, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    hipLaunchKernelGGL(route_sort_kernel, dim3(1), dim3(CHUNK), 0, s, p, logits, bias, bias_is_f32,
                       bm1, bm2);
    return hipGetLastError();
}

hipError_t launch_sort(const Plan& p, int bm1, int bm2, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    const int nchunks = sort_chunks(p.T);
    if (p.T <= SMALL_T) {
        hipLaunchKernelGGL(sort_small_kernel, dim3(1), dim3(64), 0, s, p, bm1, bm2);
        return hipGetLastError();
    }
    if (p.T <= CHUNK) {
        hipLaunchKernelGGL(sort_kernel, dim3(1), dim3(CHUNK), 0, s, p, bm1, bm2);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(sort_count_kernel, dim3(nchunks), dim3(SORT_CHUNK_L), 0, s, p);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(sort_place_kernel, dim3(nchunks), dim3(SORT_CHUNK_L), 0, s, p, nchunks, bm1,
                       bm2);
    return hipGetLastError();
}

}  // namespace mimoe
