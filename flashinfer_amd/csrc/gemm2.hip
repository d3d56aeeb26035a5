// Grouped GEMM2 (down projection): FP8 weights, bf16 activations.
//
// Replaces solution/triton/kernel.py:193-293 (_persistent_gemm2_kernel):
//   part[s, n] = bf16(w_s * sum_kb sb2[e, n/128, kb] * sum_{k in kb} act[s, k] * W2[e, n, k])
// (w_s = the slot's routing weight, applied here instead of in the combine)
// The reference dequantises W2 to fp32 and runs an fp32 (TF32) dot
// (:272-278). Here the fp8 weights are widened to bf16 in registers, which is
// exact for e4m3, and fed with the bf16 SwiGLU output to
// v_mfma_f32_16x16x32_bf16; the 128-block weight scale multiplies each
// block's partial sum in fp32. The activation stays bf16 rather than being
// requantised to fp8, whose 3-bit mantissa would put the output outside a
// 1e-2 relative tolerance. At decode sizes (where the call is HBM-bound and
// the MFMAs idle) the activation is split into bf16 hi + lo, which is wider
// than the reference's TF32 operand, and the partial rows are fp32.
//
// Stream variant (template <MT, D, NW, NQ, MODE, KS>): NW * KS waves per
// workgroup; wave w owns NQ 16-column sub-tiles (16 * NQ output columns of
// column group w % NW, inside one 128-column scale block) for 16 * MT slots
// of one expert, over k-blocks [(w / NW) * IB/KS, +IB/KS); weights go
// global -> VGPR through a D-deep prefetch ring. With KS > 1 the waves of a
// column group split K and the first adds the others' partial sums from LDS
// in split order (deterministic): at decode sizes that puts KS times more
// waves, and loads, in flight than one wave per column group. MODE (G2_*): the weighted
// rows go to part (bf16) or part_f32, and with G2_SPLIT the activation is
// act + act_lo (two bf16 MFMAs per k step against the same bf16 weights).
//
// Operand layout: lane l (row l % 16, g = l / 16) holds bytes [32g, 32g+32)
// of the 128-wide k-block of its weight row (whole-line non-temporal loads,
// exchanged within 16-lane rows by wl_frag where they are consumed); MFMA h
// (h = 0..3) consumes bytes [8h, 8h+8) of those 32, i.e. k-block offsets
// 32g + 8h. The activation operand is loaded with the same k offsets, so A
// and B always pair the same k.
#include "common.hpp"

namespace mimoe {

struct Frag16 {
    v4i c0, c1, c2, c3;  // four 8 x bf16 operands
};

__device__ __forceinline__ Frag16 ld_act(const uint16_t* row, int kb, int g) {
    const uint16_t* p0 = row + kb * BLK + g * 32;
    Frag16 f;
    f.c0 = ld16(p0);
    f.c1 = ld16(p0 + 8);
    f.c2 = ld16(p0 + 16);
    f.c3 = ld16(p0 + 24);
    return f;
}

// One 128-deep k-block of a 16 x 16 tile: a . b (+ al . b with PREC, the
// small remainder first).
template <bool PREC>
__device__ __forceinline__ v4f mfma_block(const Frag16& a, const Frag16& al, const v8i& b) {
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    const v4i b0 = fp8x8_to_bf16x8((uint32_t)b.s0, (uint32_t)b.s1);
    const v4i b1 = fp8x8_to_bf16x8((uint32_t)b.s2, (uint32_t)b.s3);
    const v4i b2 = fp8x8_to_bf16x8((uint32_t)b.s4, (uint32_t)b.s5);
    const v4i b3 = fp8x8_to_bf16x8((uint32_t)b.s6, (uint32_t)b.s7);
    if constexpr (PREC) {  // one chain: the NQ sub-tiles of a wave give the MFMAs their overlap
        acc = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, al.c0), __builtin_bit_cast(v8bf, b0), acc);
        acc = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, al.c1), __builtin_bit_cast(v8bf, b1), acc);
        acc = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, al.c2), __builtin_bit_cast(v8bf, b2), acc);
        acc = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, al.c3), __builtin_bit_cast(v8bf, b3), acc);
    }
    acc = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a.c0), __builtin_bit_cast(v8bf, b0), acc);
    acc = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a.c1), __builtin_bit_cast(v8bf, b1), acc);
    acc = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a.c2), __builtin_bit_cast(v8bf, b2), acc);
    acc = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a.c3), __builtin_bit_cast(v8bf, b3), acc);
    return acc;
}

template <int MT, int D, int NW, int NQ, int MODE, int KS>
__global__ __launch_bounds__(64 * NW * KS) void gemm2_stream_kernel(
    Plan p, const uint8_t* __restrict__ w2, const float* __restrict__ w2s) {
    constexpr int KB = IB / KS;  // k-blocks per wave
    static_assert(BLK % (16 * NQ) == 0, "a wave's columns stay inside one scale block");
    static_assert(IB % KS == 0 && KB % D == 0, "k split and prefetch depth must divide the k-blocks");
    constexpr bool PREC = MODE == G2_SPLIT;
    constexpr int BM = 16 * MT;
    // partial sums of waves 1..KS-1 of a column group: [split-1][group][value][lane]
    __shared__ float red[KS > 1 ? KS - 1 : 1][NW][KS > 1 ? 4 * MT * NQ : 1][64];
    int e, row0, nrows;
    if (!find_tile(p.meta, META_MTILE2, blockIdx.y, BM, e, row0, nrows)) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wc = wave % NW;       // column group
    const int ks = wave / NW;       // k split
    const int kb_first = ks * KB;   // first k-block of the wave
    const int n0 = blockIdx.x * (16 * NQ * NW) + wc * (16 * NQ);
    const int nb = n0 / BLK;  // 128-column scale block of the wave's columns
    const int r = lane & 15, g = lane >> 4;

    // weights of expert e through a buffer resource
    e = __builtin_amdgcn_readfirstlane(e);
    const __amdgpu_buffer_rsrc_t wr = wrsrc(w2 + (size_t)e * H * I, (uint32_t)((size_t)H * I));
    uint32_t b_off[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) b_off[q] = (uint32_t)((size_t)(n0 + q * 16) * I + wl_off(lane, I));
    const uint16_t* a_row[MT];
    const uint16_t* al_row[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const size_t off = (size_t)(row0 + min(i * 16 + r, nrows - 1)) * I;
        a_row[i] = p.act + off;
        al_row[i] = PREC ? p.act_lo + off : nullptr;
    }
    const float* sb_ptr = w2s + ((size_t)e * HB + nb) * IB;

    v4f acc[MT][NQ];
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int q = 0; q < NQ; ++q) acc[i][q] = zero;
    float wrow[MT][4];  // routing weights of this lane's rows

    // The k loop, with the weight load policy of the tile's expert (NT: non-
    // temporal, when this is its only row tile). Against a policy per launch
    // from T: T=160 GEMM2 68.4 against 74.3 us, level at T = 1 ... 128. The
    // asm markers keep the compiler from merging the two copies' first and
    // last instructions, which kept both copies' registers live (136 -> 244
    // VGPRs for the 64-column waves; 156 with the markers).
    auto body = [&](auto nt) __attribute__((always_inline)) {
        constexpr bool NT = decltype(nt)::value;
        asm volatile("; weight load policy %0 begin" ::"n"(NT ? 1 : 0));
        WRaw b[D][NQ];
        Frag16 a[D][MT];
        Frag16 al[D][MT];  // PREC only

        auto compute = [&](int d, int kb) __attribute__((always_inline)) {
            const float sb = sb_ptr[kb_first + kb];
#pragma unroll
            for (int i = 0; i < MT; ++i) {
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const v4f pr = mfma_block<PREC>(a[d][i], al[d][i], wl_frag(b[d][q]));
                    acc[i][q][0] += pr[0] * sb;
                    acc[i][q][1] += pr[1] * sb;
                    acc[i][q][2] += pr[2] * sb;
                    acc[i][q][3] += pr[3] * sb;
                }
            }
        };
        auto load = [&](int d, int kb) __attribute__((always_inline)) {
#pragma unroll
            for (int q = 0; q < NQ; ++q) b[d][q] = ld_wraw<NT>(wr, b_off[q] + (kb_first + kb) * BLK, 8 * I);
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                a[d][i] = ld_act(a_row[i], kb_first + kb, g);
                if constexpr (PREC) al[d][i] = ld_act(al_row[i], kb_first + kb, g);
            }
        };

#pragma unroll
        for (int d = 0; d < D; ++d) load(d, d);
#pragma unroll 1
        for (int kb0 = 0; kb0 < KB - D; kb0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute(d, kb0 + d);
                load(d, kb0 + d + D);
            }
        }
        // Routing weights of this lane's rows, loaded while the last D k-blocks
        // are consumed (the asm below keeps them from being sunk into the
        // per-row stores, where each would wait on its own load).
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) wrow[i][rr] = p.sorted_w[row0 + min(i * 16 + g * 4 + rr, nrows - 1)];
#pragma unroll
        for (int d = 0; d < D; ++d) compute(d, KB - D + d);
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) asm volatile("" : "+v"(wrow[i][rr]));
        asm volatile("; weight load policy %0 end" ::"n"(NT ? 1 : 0));
    };
    const int erows = p.meta[META_EXPERT_OFF + e + 1] - p.meta[META_EXPERT_OFF + e];
    if (__builtin_amdgcn_readfirstlane(erows) <= BM) body(BoolC<true>{});
    else body(BoolC<false>{});

    // K split: the other waves of the column group hand their partial sums to
    // the first through LDS, which adds them in split order.
    if constexpr (KS > 1) {
        if (ks > 0) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int q = 0; q < NQ; ++q)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        red[ks - 1][wc][(i * NQ + q) * 4 + rr][lane] = acc[i][q][rr];
        }
        __syncthreads();
        if (ks > 0) return;
#pragma unroll
        for (int k = 0; k < KS - 1; ++k)
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int q = 0; q < NQ; ++q)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr)
                        acc[i][q][rr] += red[k][wc][(i * NQ + q) * 4 + rr][lane];
    }

    // Epilogue: weight each slot's row by its routing weight (kernel.py:364)
    // and store it (bf16, or fp32 unless G2_BF16) for the combine.
#pragma unroll
    for (int i = 0; i < MT; ++i) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int m = i * 16 + g * 4 + rr;
            if (m < nrows) {
                const float w = wrow[i][rr];
                const size_t o = (size_t)(row0 + m) * H + n0 + r;
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    if constexpr (MODE != G2_BF16) p.part_f32[o + 16 * q] = w * acc[i][q][rr];
                    else p.part[o + 16 * q] = f2bf(w * acc[i][q][rr]);
                }
            }
        }
    }
}

int gemm2_bm(int variant) {
    switch (variant) {
        case 0: return 16;
        case 1: return 32;
        case 2: return 64;
        case 3: return 128;
        case 4: return 64;
        case 18: return 128;
        case 20: return 128;
        case 21: return 128;
        case 7: return 32;
        case 12: return 32;
        case 15: return 32;
        default: return 16;
    }
}

template <int MT, int D, int NW, int NQ, int MODE, int KS>
static void launch_stream2_mode(const Plan& p, const uint8_t* w2, const float* w2s, dim3 grid,
                                dim3 block, hipStream_t s) {
    hipLaunchKernelGGL((gemm2_stream_kernel<MT, D, NW, NQ, MODE, KS>), grid, block, 0, s, p, w2, w2s);
}

template <int MT, int D, int NW, int NQ, int KS = 1>
static void launch_stream2(const Plan& p, const uint8_t* w2, const float* w2s, hipStream_t s) {
    // a ring deeper than the shape's k-blocks allow falls back to 2 deep (or 1)
    constexpr int KB = IB / KS;
    constexpr int DD = KB % D == 0 ? D : (KB % 2 == 0 ? 2 : 1);
    dim3 grid(H / (16 * NQ * NW), max_mtiles(p.T, 16 * MT));
    const dim3 block(64 * NW * KS);
    switch (gemm2_mode(p)) {
        case G2_SPLIT: launch_stream2_mode<MT, DD, NW, NQ, G2_SPLIT, KS>(p, w2, w2s, grid, block, s); break;
        case G2_F32: launch_stream2_mode<MT, DD, NW, NQ, G2_F32, KS>(p, w2, w2s, grid, block, s); break;
        default: launch_stream2_mode<MT, DD, NW, NQ, G2_BF16, KS>(p, w2, w2s, grid, block, s);
    }
}

hipError_t launch_gemm2(const Plan& p, const uint8_t* w2, const float* w2s, int variant,
                        hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    if ((variant >= 3 && variant <= 4) || variant == 18 || variant == 20 || variant == 21)
        return launch_gemm2_tile(p, w2, w2s, variant, s);
    if (variant == 15) return launch_gemm2_wide(p, w2, w2s, s);
    switch (variant) {
        case 0: launch_stream2<1, 4, 4, 2>(p, w2, w2s, s); break;
        case 1: launch_stream2<2, 4, 4, 2>(p, w2, w2s, s); break;
        case 2: launch_stream2<4, 2, 4, 2>(p, w2, w2s, s); break;
        case 5: launch_stream2<1, 4, 1, 2>(p, w2, w2s, s); break;
        case 6: launch_stream2<1, 4, 1, 1>(p, w2, w2s, s); break;
        case 7: launch_stream2<2, 4, 1, 2>(p, w2, w2s, s); break;
        case 8: launch_stream2<1, 8, 4, 2>(p, w2, w2s, s); break;
        case 9: launch_stream2<1, 2, 1, 4, 4>(p, w2, w2s, s); break;
        case 11: launch_stream2<1, 8, 1, 1>(p, w2, w2s, s); break;
        case 12: launch_stream2<2, 4, 1, 1>(p, w2, w2s, s); break;
        case 13: launch_stream2<1, 4, 1, 4>(p, w2, w2s, s); break;
        case 14: launch_stream2<1, 2, 1, 4>(p, w2, w2s, s); break;
        case 16: launch_stream2<1, 4, 1, 2, 4>(p, w2, w2s, s); break;
        default: launch_stream2<1, 2, 1, 2>(p, w2, w2s, s); break;
    }
    return hipGetLastError();
}

}  // namespace mimoe
