// GEMM2 (down projection) fused with the weighted top-k combine, for small T.
//
// Computes output[t, n] = bf16( sum over the token's local slots s of
//   w_s * sum_kb sb2[e_s, n/128, kb] * (act[s, kb-block] . W2[e_s, n, kb-block]) )
// i.e. solution/triton/kernel.py:193-293 (GEMM2), :337-368 (weighted
// scatter-add), :801 (zero init) and :820-823 (bf16 cast) in one kernel, with
// no fp32 partial rows in HBM and no atomics.
//
// A workgroup owns 16 output columns for every local expert: its 4 waves take
// the 16-slot row tiles round-robin (tile u goes to wave u % 4) and stream the
// matching 16 x I fp8 weight rows through a D-deep register ring that runs
// across tile boundaries. At the end of a tile each lane adds w_s * result
// into a per-wave fp32 accumulator [T][16] in LDS (a tile never holds the
// same token twice, and one wave handles its tiles in order, so the
// read-modify-write is race-free). After a barrier the 4 per-wave
// accumulators are summed in wave order and written as bf16; tokens with no
// local slot get zeros. Every summation order is fixed, so results are
// bit-identical across runs. PREC: the activation is act + act_lo, each k
// step runs the MFMAs of both bf16 halves against the same weights.
#include "common.hpp"

namespace mimoe {

struct UnitInfo {
    int e, row0, nrows;
};

// Row tile u (16 slots) -> expert, first slot, rows (prefix table in meta).
__device__ __forceinline__ UnitInfo unit_info(const int* meta, int u) {
    int ee = 0;
#pragma unroll
    for (int k = 0; k < EL; ++k) ee += (meta[META_MTILE2 + k + 1] <= u) ? 1 : 0;
    UnitInfo r;
    r.e = ee;
    r.row0 = meta[META_EXPERT_OFF + ee] + (u - meta[META_MTILE2 + ee]) * 16;
    r.nrows = min(16, meta[META_EXPERT_OFF + ee + 1] - r.row0);
    return r;
}

template <int D, int KS, bool PREC, bool NT>
__global__ __launch_bounds__(256) void gemm2_combine_kernel(Plan p, const uint8_t* __restrict__ w2,
                                                            const float* __restrict__ w2s,
                                                            uint16_t* __restrict__ out) {
    // KS == 1: tile u goes to wave u % 4, which runs all IB k-blocks of it.
    // KS == 4: every wave runs every tile, over k-blocks [wave*KBW, +KBW).
    static_assert(KS == 1 || KS == 4, "k split over the 4 waves or none");
    constexpr int KBW = IB / KS;  // k-blocks of a tile per wave
    static_assert(IB % KS == 0 && KBW % D == 0, "ring depth must divide a wave's k-blocks of a tile");
    static_assert(D <= KBW && IB <= 64, "the load side stays in the tile; one lane per k-block scale");
    extern __shared__ float acc_lds[];  // [4 waves][T][16]
    const int T = p.T;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * 16;
    const int nb = n0 / BLK;
    const int r = lane & 15, g = lane >> 4;

    const int total = p.meta[META_MTILE2 + EL];
    const int nunits = KS > 1 ? total : (wave < total ? (total - wave + 3) / 4 : 0);
    const int nsteps = nunits * KBW;
    const int ustep = KS > 1 ? 1 : 4;           // tile index step between a wave's tiles
    const int u0 = KS > 1 ? 0 : wave;           // a wave's first tile
    const int kb0 = KS > 1 ? wave * KBW : 0;    // a wave's first k-block of each tile
    float* my_acc = acc_lds + wave * T * 16;
    // Each wave zeroes its own accumulator (no other wave reads it before the
    // barrier at the end), after its first loads are issued.
    auto zero_acc = [&]() __attribute__((always_inline)) {
        for (int i = lane; i < T * 16; i += 64) my_acc[i] = 0.f;
    };

    if (nsteps <= 0) zero_acc();
    if (nsteps > 0) {
        WRaw b[D];
        v4i a[D][4];
        v4i al[D][4];  // PREC only
        // Per-tile data, fetched when the load side enters a tile (D steps
        // before the compute side needs it): block scales of the 16 k-blocks,
        // and the token and routing weight of the lane's 4 output rows.
        // Lane q < IB holds the scale of k-block q; readlane picks it.
        UnitInfo lu = unit_info(p.meta, u0);
        float lu_sb = 0.f;
        int lu_tok[4];
        float lu_w[4];
        UnitInfo cu = lu;
        float cu_sb = 0.f;
        int cu_tok[4];
        float cu_w[4];
        v4f acc = {0.f, 0.f, 0.f, 0.f};

        auto fetch_unit = [&](int u) __attribute__((always_inline)) {
            lu = unit_info(p.meta, u);
            lu_sb = w2s[((size_t)lu.e * HB + nb) * IB + lane % IB];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = g * 4 + i;
                const int slot = lu.row0 + min(row, lu.nrows - 1);
                lu_tok[i] = p.sorted_tok[slot];
                lu_w[i] = row < lu.nrows ? p.sorted_w[slot] : 0.f;
            }
        };
        auto load = [&](int d, int s) __attribute__((always_inline)) {
            // step s: k-block kb of the wave's (s / KBW)-th tile
            const int kb = kb0 + s % KBW;
            if (s % KBW == 0 && s > 0) fetch_unit(u0 + ustep * (s / KBW));
            // whole-line weight loads (wl_frag), activation at the same k offsets
            const __amdgpu_buffer_rsrc_t wr = wrsrc(w2 + (size_t)lu.e * H * I, (uint32_t)((size_t)H * I));
            b[d] = ld_wraw<NT>(wr, (uint32_t)((size_t)n0 * I + wl_off(lane, I) + kb * BLK), 8 * I);
            const size_t ao = (size_t)(lu.row0 + min(r, lu.nrows - 1)) * I + kb * BLK + g * 32;
            const uint16_t* ap = p.act + ao;
            a[d][0] = ld16(ap);
            a[d][1] = ld16(ap + 8);
            a[d][2] = ld16(ap + 16);
            a[d][3] = ld16(ap + 24);
            if constexpr (PREC) {
                const uint16_t* lp = p.act_lo + ao;
                al[d][0] = ld16(lp);
                al[d][1] = ld16(lp + 8);
                al[d][2] = ld16(lp + 16);
                al[d][3] = ld16(lp + 24);
            }
        };
        auto compute = [&](int d, int s) __attribute__((always_inline)) {
            const int kb = kb0 + s % KBW;
            if (s % KBW == 0) {
                // The load side is D <= KBW steps ahead: its last load is of this
                // tile, and it enters the next tile right after this step.
                cu = lu;
                cu_sb = lu_sb;
#pragma unroll
                for (int i = 0; i < 4; ++i) { cu_tok[i] = lu_tok[i]; cu_w[i] = lu_w[i]; }
            }
            const float sb = __builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cu_sb), kb));
            v4f pr = {0.f, 0.f, 0.f, 0.f};
            const v8i bf = wl_frag(b[d]);
            const v4i b0 = fp8x8_to_bf16x8((uint32_t)bf.s0, (uint32_t)bf.s1);
            const v4i b1 = fp8x8_to_bf16x8((uint32_t)bf.s2, (uint32_t)bf.s3);
            const v4i b2 = fp8x8_to_bf16x8((uint32_t)bf.s4, (uint32_t)bf.s5);
            const v4i b3 = fp8x8_to_bf16x8((uint32_t)bf.s6, (uint32_t)bf.s7);
            v4f pl = pr;  // PREC: the act_lo products, a chain of their own
            if constexpr (PREC) {
                pl = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, al[d][0]), __builtin_bit_cast(v8bf, b0), pl);
                pl = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, al[d][1]), __builtin_bit_cast(v8bf, b1), pl);
                pl = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, al[d][2]), __builtin_bit_cast(v8bf, b2), pl);
                pl = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, al[d][3]), __builtin_bit_cast(v8bf, b3), pl);
            }
            pr = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a[d][0]), __builtin_bit_cast(v8bf, b0), pr);
            pr = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a[d][1]), __builtin_bit_cast(v8bf, b1), pr);
            pr = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a[d][2]), __builtin_bit_cast(v8bf, b2), pr);
            pr = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a[d][3]), __builtin_bit_cast(v8bf, b3), pr);
            if constexpr (PREC) pr += pl;
            acc[0] += pr[0] * sb;
            acc[1] += pr[1] * sb;
            acc[2] += pr[2] * sb;
            acc[3] += pr[3] * sb;
            if (s % KBW == KBW - 1) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (g * 4 + i < cu.nrows) my_acc[cu_tok[i] * 16 + r] += cu_w[i] * acc[i];
                }
                acc = (v4f){0.f, 0.f, 0.f, 0.f};
            }
        };

        fetch_unit(u0);
#pragma unroll
        for (int d = 0; d < D; ++d) load(d, d);
        zero_acc();
#pragma unroll 1
        for (int s0 = 0; s0 < nsteps - D; s0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute(d, s0 + d);
                load(d, s0 + d + D);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) compute(d, nsteps - D + d);
    }
    __syncthreads();

    for (int i = tid; i < T * 16; i += 256) {
        const float v = ((acc_lds[i] + acc_lds[T * 16 + i]) + acc_lds[2 * T * 16 + i]) +
                        acc_lds[3 * T * 16 + i];
        out[(size_t)(i >> 4) * H + n0 + (i & 15)] = f2bf(v);
    }
}

// Largest T the fused kernel takes (its LDS accumulators are 256*T bytes).
constexpr int FUSED_MAX_T = 256;

bool gemm2_combine_supported(int T) { return T > 0 && T <= FUSED_MAX_T; }

// One launch of the kernel for the call's activation form and weight load
// policy (non-temporal while no expert can hold a second 16-row tile).
template <int D, int KS>
static void launch_combine(const Plan& p, const uint8_t* w2, const float* w2s, uint16_t* out,
                           hipStream_t s) {
    const size_t lds = (size_t)4 * p.T * 16 * sizeof(float);
    const bool nt = p.T <= 16;
    if (p.act_lo && nt)
        hipLaunchKernelGGL((gemm2_combine_kernel<D, KS, true, true>), dim3(H / 16), dim3(256), lds, s, p,
                           w2, w2s, out);
    else if (p.act_lo)
        hipLaunchKernelGGL((gemm2_combine_kernel<D, KS, true, false>), dim3(H / 16), dim3(256), lds, s, p,
                           w2, w2s, out);
    else if (nt)
        hipLaunchKernelGGL((gemm2_combine_kernel<D, KS, false, true>), dim3(H / 16), dim3(256), lds, s, p,
                           w2, w2s, out);
    else
        hipLaunchKernelGGL((gemm2_combine_kernel<D, KS, false, false>), dim3(H / 16), dim3(256), lds, s,
                           p, w2, w2s, out);
}

hipError_t launch_gemm2_combine(const Plan& p, const uint8_t* w2, const float* w2s, uint16_t* out,
                                hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    constexpr int D = IB % 4 == 0 ? 4 : 2;  // ring depth must divide the shape's k-blocks
    launch_combine<D, 1>(p, w2, w2s, out, s);
    return hipGetLastError();
}

hipError_t launch_gemm2_combine_ks(const Plan& p, const uint8_t* w2, const float* w2s,
                                   uint16_t* out, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    // A wave's whole k-range of a tile in flight (measured on MI355X at T = 1
    // and 4 with 2 and 3 local slots: 0.4 and 1.1 us per call ahead of two
    // k-blocks)
    constexpr int KBW = IB / 4;
    constexpr int D = KBW <= 4 ? KBW : (KBW % 2 == 0 ? 2 : 1);
    launch_combine<D, 4>(p, w2, w2s, out, s);
    return hipGetLastError();
}

}  // namespace mimoe
