// Grouped FP8 GEMM1 (gate | up) with the SwiGLU epilogue fused.
//
// Replaces solution/triton/kernel.py:69-186 (_persistent_gemm1_kernel), the
// input permute at :699-703 and _swiglu_kernel (:301-330):
//   G[s, n] = sum_kb sa[kb, tok(s)] * sb1[e, n/128, kb] * sum_{k in kb} A8[tok(s), k] * W1[e, n, k]
//   act[s, j] = silu(G[s, I + j]) * G[s, j]      (SiLU on the second half, :318-326)
// A rows are gathered straight from hidden_states by the slot's token (no
// permuted copy). One v_mfma_scale_f32_16x16x128_f8f6f4 covers exactly one
// 128-wide scale block, so the product of the two block scales is applied
// to each MFMA result in the fp32 accumulator (kernel.py:168-171).
//
// "Stream" variant (template <MT, D, NW, KS>): weight tiles are not reused
// across row tiles, so they go global -> VGPR with a D-deep register prefetch
// ring instead of through LDS. A workgroup is NW * KS waves; wave w owns gate
// columns j0..j0+15 and the matching up columns I+j0..I+j0+15 of column group
// w % NW for the BM = 16*MT rows of one expert's row tile, over k-blocks
// [(w / NW) * 56/KS, +56/KS): with KS > 1 the waves of a column group split K
// and add their partial sums through LDS in a fixed order, which gives few
// active experts more waves in flight.
//
// Operand layout: lane l feeds row (l % 16) of a 16x128 operand with bytes
// [32g, 32g+32) of the 128-byte k-block, g = l / 16. The weights arrive as
// whole 128-byte lines (two non-temporal loads per k-block, exchanged within
// 16-lane rows by wl_frag where they are consumed); the activation row is
// read at the same k offsets (ld_afrag).
//
// With FRONT_SORT (T <= 64, MT = 1) the kernel also stands in for the sort
// launch: each wave builds the row-tile table from the top-k ids in its
// registers (wave_table: the one-wave sort's counts and scans) and looks up
// its row tiles there, so no kernel boundary separates routing from GEMM1.
// Workgroup 0 of the (one-dimensional) grid writes the sort's tables
// (expert offsets, tile prefixes for bm1 / bm2, slot lists) for GEMM2 and
// the combine, which run after this kernel, so no GEMM workgroup waits on
// them. With FRONT_ROUTE every workgroup first
// routes all T tokens itself (its waves take them round-robin, route_token
// as in the routing kernel) into LDS, and the tables workgroup also writes
// the top-k: the call then starts with GEMM1. A front workgroup takes row
// tiles y, y + R, y + 2R, ... (R rows of workgroups): at T <= 4 the grid has
// fewer rows than the bound on row tiles, most of which are empty there,
// and every workgroup pays for the routing.
#include "route_impl.hpp"
#include "sort_impl.hpp"

#include <algorithm>

namespace mimoe {

template <int MT, int D, int NW, int KS = 1, int FRONT = FRONT_NONE, bool NT = true>
__global__ __launch_bounds__(64 * NW * KS)
__attribute__((amdgpu_waves_per_eu(FRONT != FRONT_NONE && KS == 4 ? 5 : 1)))
void gemm1_stream_kernel(Plan p, const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
                         const uint8_t* __restrict__ w1, const float* __restrict__ w1s, FrontArgs fa) {
    constexpr int KB = HB / KS;  // k-blocks per wave
    constexpr int NWAVES = NW * KS;
    static_assert(HB % KS == 0 && KB % D == 0, "k split and prefetch depth must divide the k-blocks");
    static_assert(FRONT == FRONT_NONE || MT == 1, "the in-kernel sort gives each lane the token of one row");
    constexpr int BM = 16 * MT;
    __shared__ float sa_lds[HB][BM];
    // partial sums of waves 1..KS-1 of a column group: [split-1][group][value][lane]
    __shared__ float red[KS > 1 ? KS - 1 : 1][NW][KS > 1 ? 8 * MT : 1][64];
    // top-k of every token, routed in this workgroup (FRONT_ROUTE, T <= 64)
    constexpr int RT = FRONT == FRONT_ROUTE ? SMALL_T * TOPK_LD : 4;
    __shared__ __attribute__((aligned(16))) int s_ids[RT];
    __shared__ __attribute__((aligned(16))) float s_w[RT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // The GEMM of one row tile (expert e, slots row0 .. row0 + nrows - 1, the
    // token of this lane's row i * 16 + r in tok[i]) for this workgroup's
    // weight columns. The lane index comes in as an argument: the tile loop
    // of the front kernels passes it through an empty asm statement, so the
    // compiler recomputes the lane's addresses per tile instead of holding
    // them across the loop (77 instead of 96 VGPRs and spills).
    auto tile = [&](int e, const int row0, const int nrows, const int (&tok)[MT], const int lane,
                    const int col) __attribute__((always_inline)) {
        const int r = lane & 15, g = lane >> 4;
        const int tid = wave * 64 + lane;
        const int wc = wave % NW;         // column group
        const int ks = wave / NW;         // k split: k-blocks [ks*KB, ks*KB + KB)
        const int j0 = col * (16 * NW) + wc * 16;
        // weights of expert e through a buffer resource: gate rows, then up rows I further
        e = __builtin_amdgcn_readfirstlane(e);
        const __amdgpu_buffer_rsrc_t wr = wrsrc(w1 + (size_t)e * N1 * H, (uint32_t)((size_t)N1 * H));
        const uint32_t bg_off = (uint32_t)((size_t)j0 * H + (size_t)ks * KB * BLK + wl_off(lane, H));
        const uint32_t bu_off = bg_off + (uint32_t)((size_t)I * H);
        const uint8_t* a_ptr[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) a_ptr[i] = hs + (size_t)tok[i] * H + ks * KB * BLK + g * 32;
        const float* sbg_ptr = w1s + ((size_t)e * N1B + j0 / BLK) * HB + ks * KB;
        const float* sbu_ptr = w1s + ((size_t)e * N1B + (I + j0) / BLK) * HB + ks * KB;
        const float (*sa_k)[BM] = sa_lds + ks * KB;  // this wave's k-blocks

        WRaw bg[D], bu[D];
        v8i a[D][MT];
        v4f accg[MT], accu[MT];
        const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < MT; ++i) { accg[i] = zero; accu[i] = zero; }

        // Consume ring stage d (k-block kb): two MFMAs per row sub-tile, block
        // scales applied in fp32.
        auto compute = [&](int d, int kb) __attribute__((always_inline)) {
            const float sg = sbg_ptr[kb];
            const float su = sbu_ptr[kb];
            const v8i fg = wl_frag(bg[d]);
            const v8i fu = wl_frag(bu[d]);
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const v4f pg = mfma_f8_16x16x128(a[d][i], fg, zero);
                const v4f pu = mfma_f8_16x16x128(a[d][i], fu, zero);
                const float4 sa4 = *reinterpret_cast<const float4*>(&sa_k[kb][i * 16 + g * 4]);
                accg[i][0] += pg[0] * (sa4.x * sg);
                accg[i][1] += pg[1] * (sa4.y * sg);
                accg[i][2] += pg[2] * (sa4.z * sg);
                accg[i][3] += pg[3] * (sa4.w * sg);
                accu[i][0] += pu[0] * (sa4.x * su);
                accu[i][1] += pu[1] * (sa4.y * su);
                accu[i][2] += pu[2] * (sa4.z * su);
                accu[i][3] += pu[3] * (sa4.w * su);
            }
        };
        auto load = [&](int d, int kb) __attribute__((always_inline)) {
            const int nk = kb * BLK;
            bg[d] = ld_wraw<NT>(wr, bg_off + nk, 8 * H);
            bu[d] = ld_wraw<NT>(wr, bu_off + nk, 8 * H);
#pragma unroll
            for (int i = 0; i < MT; ++i) a[d][i] = ld_afrag(a_ptr[i] + nk);
        };

        // Start streaming weights first; the activation scales of the tile go to
        // LDS while those loads are in flight.
#pragma unroll
        for (int d = 0; d < D; ++d) load(d, d);
        // (64 * NW * KS is a multiple of BM, so entry i's row m = i % BM is the
        // same for all of a thread's entries: row tid % BM = i' * 16 + r.)
        static_assert((64 * NW * KS) % BM == 0, "scale loader row");
        {
            const int tok_m = tok[(tid % BM) / 16];
            for (int i = tid; i < HB * BM; i += 64 * NW * KS) {
                const int kb = i / BM, m = i % BM;
                sa_lds[kb][m] = hs_scale[(size_t)kb * p.T + tok_m];
            }
        }
        __syncthreads();

        // Steady state: every stage is refilled right after it is consumed.
#pragma unroll 1
        for (int kb0 = 0; kb0 < KB - D; kb0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute(d, kb0 + d);
                load(d, kb0 + d + D);
            }
        }
        // Drain the last D k-blocks.
#pragma unroll
        for (int d = 0; d < D; ++d) compute(d, KB - D + d);

        // K split: the other waves of the column group hand their partial sums to
        // the first through LDS, which adds them in split order (deterministic).
        if constexpr (KS > 1) {
            if (ks > 0) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        red[ks - 1][wc][8 * i + rr][lane] = accg[i][rr];
                        red[ks - 1][wc][8 * i + 4 + rr][lane] = accu[i][rr];
                    }
            }
            __syncthreads();
            if (ks > 0) return;
#pragma unroll
            for (int k = 0; k < KS - 1; ++k)
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        accg[i][rr] += red[k][wc][8 * i + rr][lane];
                        accu[i][rr] += red[k][wc][8 * i + 4 + rr][lane];
                    }
        }

#pragma unroll
        for (int i = 0; i < MT; ++i) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int m = i * 16 + g * 4 + rr;
                if (m < nrows) {
                    const float v = silu(accu[i][rr]) * accg[i][rr];
                    store_act(p, (size_t)(row0 + m) * I + j0 + r, v);
                }
            }
        }
    };

    if constexpr (FRONT != FRONT_NONE) {
        // One-dimensional grid: workgroup 0 writes the tables (dispatched
        // first, so it runs beside the GEMM workgroups, not after them);
        // workgroup 1 + row * NCOL + col takes column block col of row tiles
        // row, row + rows, ...
        constexpr int NCOL = I / (16 * NW);
        const int rows = (gridDim.x - 1) / NCOL;
        const bool tables = blockIdx.x == 0;
        const int col = tables ? 0 : (int)(blockIdx.x - 1) % NCOL;
        const int row = tables ? 0 : (int)(blockIdx.x - 1) / NCOL;
        const int* ids_src = p.topk_ids;
        const float* w_src = p.topk_w;
        if (FRONT == FRONT_ROUTE && p.T == 1 && !tables) {
            // One token: every wave routes it itself (the same result in each,
            // so no LDS copy and no barrier), and row tile r is its r-th local
            // expert (slot r, one row), so no per-wave table either. Per call
            // with two local slots (bitwise equal): 24.4 against 25.4 us for
            // dropping the table, 23.4 against 24.3 for routing in every wave.
            int ids[TOPK];
            float w[TOPK];
            route_token(fa.logits, fa.bias, fa.bias_is_f32, p.rsf, lane, ids, w);
            emask_t m = 0;
#pragma unroll
            for (int k = 0; k < TOPK; ++k) {
                const int l = ids[k] - p.local_offset;
                m |= (unsigned)l < (unsigned)EL ? ebit(l) : (emask_t)0;
            }
            const int n = epopc(m);  // the same in every wave of the workgroup
            for (int mt = row; mt < n; mt += rows) {  // one pass: rows = TOPK at T = 1
                const int tok[MT] = {0};
                if (mt != row) __syncthreads();  // the last tile's reads of sa_lds are done
                int ln = lane;
                asm volatile("" : "+v"(ln));
                tile(nth_set_bit((unsigned long long)m, mt), mt, 1, tok, ln, col);
            }
            return;
        }
        if constexpr (FRONT == FRONT_ROUTE) {
            for (int t = wave; t < p.T; t += NWAVES) {
                int ids[TOPK];
                float w[TOPK];
                route_token(fa.logits + (size_t)t * EG, fa.bias, fa.bias_is_f32, p.rsf, lane, ids, w);
                if (lane == 0) store_topk_row(s_ids + t * TOPK_LD, s_w + t * TOPK_LD, ids, w);
            }
            __syncthreads();
            ids_src = s_ids;
            w_src = s_w;
        }
        if (tables) {
            if (wave == 0) {
                if constexpr (FRONT == FRONT_ROUTE) {
                    if (lane < p.T) {  // the global top-k, as the routing kernel writes it
                        int4* io = reinterpret_cast<int4*>(p.topk_ids + (size_t)lane * TOPK_LD);
                        float4* wo = reinterpret_cast<float4*>(p.topk_w + (size_t)lane * TOPK_LD);
                        io[0] = reinterpret_cast<const int4*>(s_ids + lane * TOPK_LD)[0];
                        io[1] = reinterpret_cast<const int4*>(s_ids + lane * TOPK_LD)[1];
                        wo[0] = reinterpret_cast<const float4*>(s_w + lane * TOPK_LD)[0];
                        wo[1] = reinterpret_cast<const float4*>(s_w + lane * TOPK_LD)[1];
                    }
                }
                sort_one_wave<1>(p, ids_src, w_src, fa.bm1, fa.bm2, lane);
            }
            return;
        }
        const WaveTable tab = wave_table(p, ids_src, lane, BM);
        const int ntiles = table_tiles(tab);
        for (int mt = row; mt < ntiles; mt += rows) {
            const WaveTile wt = table_tile(tab, lane, mt, BM);
            const int tok[MT] = {nth_set_bit(wt.hits, wt.rank0 + min(lane & 15, wt.nrows - 1))};
            if (mt != row) __syncthreads();  // the last tile's reads of sa_lds are done
            int ln = lane;
            asm volatile("" : "+v"(ln));
            tile(wt.e, wt.row0, wt.nrows, tok, ln, col);
        }
    } else {
        int e, row0, nrows;
        if (!find_tile(p.meta, META_MTILE1, blockIdx.y, BM, e, row0, nrows)) return;
        int tok[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) tok[i] = p.sorted_tok[row0 + min(i * 16 + (lane & 15), nrows - 1)];
        tile(e, row0, nrows, tok, lane, blockIdx.x);
    }
}

int gemm1_bm(int variant) {
    switch (variant) {
        case 0: return 16;
        case 1: return 32;
        case 2: return 64;
        case 3: return 256;
        case 4: return 128;
        case 18: return 256;
        case 19: return 256;
        case 11: return 32;
        case 12: return 32;
        case 15: return 64;
        default: return 16;
    }
}

// Workgroup rows of the front kernels: at T <= 4 one per possible local
// expert of a single token (a row takes tiles y, y + 8, ...), so a call
// with a few active experts runs ~8 x 128 workgroups instead of the bound on
// row tiles (up to 32 x 128), each of which would route the tokens first.
constexpr int FRONT_ROWS_SMALL_T = 4;
constexpr int FRONT_ROWS = TOPK;

template <int MT, int D, int NW, int KS = 1, int FRONT = FRONT_NONE>
static void launch_stream1(const Plan& p, const uint8_t* hs, const float* hs_scale,
                           const uint8_t* w1, const float* w1s, hipStream_t s,
                           const FrontArgs& fa = FrontArgs{}) {
    dim3 grid(I / (16 * NW), max_mtiles(p.T, 16 * MT));
    if constexpr (FRONT != FRONT_NONE) {
        // one-dimensional: the tables workgroup, then rows x column blocks
        const int rows = p.T <= FRONT_ROWS_SMALL_T ? std::min<int>(grid.y, FRONT_ROWS) : (int)grid.y;
        grid = dim3(1 + grid.x * rows, 1);
    }
    if (wt_nt(p.T, 16 * MT))
        hipLaunchKernelGGL((gemm1_stream_kernel<MT, D, NW, KS, FRONT, true>), grid, dim3(64 * NW * KS), 0,
                           s, p, hs, hs_scale, w1, w1s, fa);
    else
        hipLaunchKernelGGL((gemm1_stream_kernel<MT, D, NW, KS, FRONT, false>), grid, dim3(64 * NW * KS),
                           0, s, p, hs, hs_scale, w1, w1s, fa);
}

bool gemm1_routes_supported(int T, int variant) {
    return (variant == 16 || variant == 5) && T > 0 && T <= SMALL_T;
}

bool gemm1_sorts_supported(int T, int variant) {
    return gemm1_routes_supported(T, variant) || (variant == 15 && gemm1_wide_sorts_supported(T));
}

hipError_t launch_gemm1_front(const Plan& p, const uint8_t* hs, const float* hs_scale,
                              const uint8_t* w1, const float* w1s, int variant, int front,
                              const FrontArgs& fa, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    if (front == FRONT_ROUTE ? !gemm1_routes_supported(p.T, variant)
                             : !gemm1_sorts_supported(p.T, variant))
        return hipErrorInvalidValue;
    if (variant == 15) return launch_gemm1_wide_sorting(p, hs, hs_scale, w1, w1s, fa.bm2, s);
    if (front == FRONT_ROUTE) {
        if (variant == 5) launch_stream1<1, 4, 1, 1, FRONT_ROUTE>(p, hs, hs_scale, w1, w1s, s, fa);
        else launch_stream1<1, 2, 1, 4, FRONT_ROUTE>(p, hs, hs_scale, w1, w1s, s, fa);
    } else {
        if (variant == 5) launch_stream1<1, 4, 1, 1, FRONT_SORT>(p, hs, hs_scale, w1, w1s, s, fa);
        else launch_stream1<1, 2, 1, 4, FRONT_SORT>(p, hs, hs_scale, w1, w1s, s, fa);
    }
    return hipGetLastError();
}

hipError_t launch_gemm1(const Plan& p, const uint8_t* hs, const float* hs_scale, const uint8_t* w1,
                        const float* w1s, int variant, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    if ((variant >= 3 && variant <= 4) || variant == 18 || variant == 19)
        return launch_gemm1_tile(p, hs, hs_scale, w1, w1s, variant, s);
    if (variant == 15) return launch_gemm1_wide(p, hs, hs_scale, w1, w1s, s);
    switch (variant) {
        case 0: launch_stream1<1, 4, 4>(p, hs, hs_scale, w1, w1s, s); break;
        case 1: launch_stream1<2, 4, 4>(p, hs, hs_scale, w1, w1s, s); break;
        case 2: launch_stream1<4, 2, 4>(p, hs, hs_scale, w1, w1s, s); break;
        case 5: launch_stream1<1, 4, 1>(p, hs, hs_scale, w1, w1s, s); break;
        case 6: launch_stream1<1, 8, 1>(p, hs, hs_scale, w1, w1s, s); break;
        case 7: launch_stream1<1, 8, 4>(p, hs, hs_scale, w1, w1s, s); break;
        case 8: launch_stream1<1, 4, 2>(p, hs, hs_scale, w1, w1s, s); break;
        case 11: launch_stream1<2, 4, 1>(p, hs, hs_scale, w1, w1s, s); break;
        case 12: launch_stream1<2, 2, 1>(p, hs, hs_scale, w1, w1s, s); break;
        case 16: launch_stream1<1, 2, 1, 4>(p, hs, hs_scale, w1, w1s, s); break;
        default: launch_stream1<1, 2, 1>(p, hs, hs_scale, w1, w1s, s); break;
    }
    return hipGetLastError();
}

}  // namespace mimoe
