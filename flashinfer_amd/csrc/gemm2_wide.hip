// Grouped GEMM2 (down projection) for medium row counts per expert ("wide"
// tiles).
//
// Same contract as gemm2_stream_kernel (solution/triton/kernel.py:193-293):
//   part[s, n] = bf16(w_s * sum_kb sb2[e, n/128, kb] * (act[s, kb-block] . W2[e, n, kb-block]))
// with bf16 activations and fp8 weights widened to bf16 (exact).
//
// Shape (template <MTW, D, DA, MODE>): a workgroup of 8 waves owns BM = 16*MTW
// slots of one expert and 128 output columns; wave w owns columns n0..n0+15
// for all BM rows, so its 16 weight rows go global -> VGPR through a D-deep
// register ring (no two waves share them). The BM activation rows of a
// k-block (contiguous slots, 256 bytes each) are loaded once per workgroup
// into a DA-deep register staging ring and written to an LDS double buffer
// one k-block ahead of their use: one barrier per k-block. The 128 columns are
// one 128-column scale block, so sb2 is one uniform value per k-block. Every
// column group re-reads the tile's activation rows from L2 (as many bytes as
// the weights at T=256 with 64-column groups); 128 columns halve that: 72.7
// against 77.0 us at T=256, 136.5 against 154.9 with every token on the same
// 8 experts.
// MODE (G2_*): rows go to part (bf16) or part_f32; with G2_SPLIT the act_lo
// rows ride along as rows BM..2BM-1 of the LDS buffers and each k step runs
// the MFMAs of both halves against the same bf16 weights.
//
// Operand k order (identical for A and B, so the pairing is exact): lane
// (r = l%16, g = l/16) holds k-block offsets 32g+[0,32) (whole-line weight
// loads, wl_frag); MFMA h uses offsets 32g+8h. LDS activation rows are 256
// bytes (16 chunks of 8 bf16) with chunk c at position c ^ (row & 15); a
// lane reads chunks 4g..4g+3.
#include "tile_common.hpp"

namespace mimoe {

namespace {
constexpr int gcd2(int a, int b) { return b == 0 ? a : gcd2(b, a % b); }
constexpr int lcm2(int a, int b) { return a / gcd2(a, b) * b; }
constexpr int W2_NW = 8;           // waves per workgroup
constexpr int W2_N = 16 * W2_NW;   // output columns per workgroup
constexpr int W2_BM = 32;          // rows per workgroup (see the launcher)
}  // namespace

template <int MTW, int D, int DA, int MODE>
__global__ __launch_bounds__(64 * W2_NW) void gemm2_wide_kernel(Plan p, const uint8_t* __restrict__ w2,
                                                                const float* __restrict__ w2s) {
    constexpr bool PREC = MODE == G2_SPLIT;
    constexpr int BM = 16 * MTW;
    constexpr int AROWS = PREC ? 2 * BM : BM;         // LDS rows: act (and act_lo)
    constexpr int THREADS = 64 * W2_NW;
    constexpr int ROW_BYTES = BLK * 2;                // one k-block of a bf16 row
    constexpr int ROWS_PER_PASS = THREADS / 16;       // 16 threads x 16 B cover one row
    constexpr int A_LD = AROWS / ROWS_PER_PASS;       // 16-byte loads per thread per k-block
    static_assert(BM % ROWS_PER_PASS == 0 && BM <= THREADS, "activation loader");
    static_assert(IB % D == 0 && IB % DA == 0 && D > DA, "ring depths");
    __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][AROWS * ROW_BYTES];
    __shared__ float w_lds[THREADS];  // routing weights of the tile's slots (first BM used)

    int e, row0, nrows;
    if (!find_tile(p.meta, META_MTILE2, blockIdx.y, BM, e, row0, nrows)) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb0 = blockIdx.x * W2_N;   // first output column of the workgroup
    const int n0 = nb0 + wave * 16;      // first output column of this wave
    const int r = lane & 15, g = lane >> 4;

    // weights of expert e through a buffer resource, plain loads: the 32-row
    // tiles run at 177 <= T <= 256, where the non-temporal hint gained nothing
    // with random routing (76.8 against 76.9 us at T=256) and cost 20 % with
    // every token on the same 8 experts (8 row tiles each)
    e = __builtin_amdgcn_readfirstlane(e);
    const __amdgpu_buffer_rsrc_t wr = wrsrc(w2 + (size_t)e * H * I, (uint32_t)((size_t)H * I));
    const uint32_t b_off = (uint32_t)((size_t)n0 * I + wl_off(lane, I));
    const float* sb_ptr = w2s + ((size_t)e * HB + nb0 / BLK) * IB;

    // activation loader: thread t copies chunk t%16 of rows t/16 + 16i
    const int ac = tid & 15;
    const uint8_t* a_src[A_LD];
    uint32_t a_dst[A_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        const int row = (tid >> 4) + ROWS_PER_PASS * i;  // LDS row: act rows, then act_lo rows
        const int lo = row >= BM;
        const uint8_t* act = reinterpret_cast<const uint8_t*>(lo ? p.act_lo : p.act);
        a_src[i] = act + (size_t)(row0 + min(row - lo * BM, nrows - 1)) * (I * 2) + ac * 16;
        a_dst[i] = row * ROW_BYTES + ((ac ^ swz16(row)) << 4);
    }
    // Routing weights of the tile: loaded first, stored to LDS after the
    // prologue (every thread stores, so the load is not sunk into a branch).
    const float w_row = p.sorted_w[row0 + min(tid, nrows - 1)];

    WRaw b[D];
    v4i ast[DA][A_LD];
    v4f acc[MTW];
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < MTW; ++m) acc[m] = zero;

    auto load_w = [&](int d, int kb) __attribute__((always_inline)) {
        b[d] = ld_wraw<false>(wr, b_off + kb * BLK, 8 * I);
    };
    auto load_a = [&](int s, int kb) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) ast[s][i] = ld16(a_src[i] + kb * ROW_BYTES);
    };
    auto store_a = [&](int s, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < A_LD; ++i) *reinterpret_cast<v4i*>(&a_lds[buf][a_dst[i]]) = ast[s][i];
    };
    auto compute = [&](int d, int buf, float sb) __attribute__((always_inline)) {
        const v8i w = wl_frag(b[d]);
        const v4i b0 = fp8x8_to_bf16x8((uint32_t)w.s0, (uint32_t)w.s1);
        const v4i b1 = fp8x8_to_bf16x8((uint32_t)w.s2, (uint32_t)w.s3);
        const v4i b2 = fp8x8_to_bf16x8((uint32_t)w.s4, (uint32_t)w.s5);
        const v4i b3 = fp8x8_to_bf16x8((uint32_t)w.s6, (uint32_t)w.s7);
        const uint8_t* sA = a_lds[buf];
#pragma unroll
        for (int m = 0; m < MTW; ++m) {
            const int row = m * 16 + r;
            const uint8_t* base = sA + row * ROW_BYTES;
            const int sw = swz16(row);
            const v4i a0 = lds16(base + (((4 * g) ^ sw) << 4));
            const v4i a1 = lds16(base + (((4 * g + 1) ^ sw) << 4));
            const v4i a2 = lds16(base + (((4 * g + 2) ^ sw) << 4));
            const v4i a3 = lds16(base + (((4 * g + 3) ^ sw) << 4));
            v4f pl = zero;  // act_lo products: a chain of their own
            if constexpr (PREC) {
                // act_lo row m*16+r sits BM rows further (same swizzle: BM % 16 == 0)
                const uint8_t* lbase = base + BM * ROW_BYTES;
                const v4i l0 = lds16(lbase + (((4 * g) ^ sw) << 4));
                const v4i l1 = lds16(lbase + (((4 * g + 1) ^ sw) << 4));
                const v4i l2 = lds16(lbase + (((4 * g + 2) ^ sw) << 4));
                const v4i l3 = lds16(lbase + (((4 * g + 3) ^ sw) << 4));
                pl = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, l0), __builtin_bit_cast(v8bf, b0), pl);
                pl = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, l1), __builtin_bit_cast(v8bf, b1), pl);
                pl = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, l2), __builtin_bit_cast(v8bf, b2), pl);
                pl = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, l3), __builtin_bit_cast(v8bf, b3), pl);
            }
            v4f pr = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a0), __builtin_bit_cast(v8bf, b0), zero);
            pr = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a1), __builtin_bit_cast(v8bf, b1), pr);
            pr = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a2), __builtin_bit_cast(v8bf, b2), pr);
            pr = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a3), __builtin_bit_cast(v8bf, b3), pr);
            if constexpr (PREC) pr += pl;
            acc[m][0] += pr[0] * sb; acc[m][1] += pr[1] * sb;
            acc[m][2] += pr[2] * sb; acc[m][3] += pr[3] * sb;
        }
        // Pure arithmetic would otherwise be sunk below the following
        // barriers (as in gemm1_wide.hip); naming the accumulators pins it.
#pragma unroll
        for (int m = 0; m < MTW; ++m) asm volatile("" : "+v"(acc[m]));
    };

    // Prologue: the loads iterations -D..-1 would have issued, in their order
    // (iteration j loads A(j+1+DA), then W(j+D)); the store of A(0) belongs to
    // iteration -1. sched_barrier keeps the groups in this order.
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const int a = d - (D - DA - 1);
        if (a >= 0) {
            if (a == DA) store_a(0, 0);
            load_a(a % DA, a);
            __builtin_amdgcn_sched_barrier(0);
        }
        load_w(d, d);
        __builtin_amdgcn_sched_barrier(0);
    }
    w_lds[tid] = w_row;
    __syncthreads();

    constexpr int U = lcm2(lcm2(D, DA), 2);
    static_assert(IB % U == 0, "unroll");
#pragma unroll 1
    for (int kb0 = 0; kb0 < IB; kb0 += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kb = kb0 + u;
            const int buf = u & 1;
            const int s = (u + 1) % DA;  // staging slot holding k-block kb+1
            if (kb + 1 < IB) {
                store_a(s, buf ^ 1);
                load_a(s, min(kb + 1 + DA, IB - 1));
            }
            compute(u % D, buf, sb_ptr[kb]);
            load_w(u % D, min(kb + D, IB - 1));
            __syncthreads();
        }
    }

    // Epilogue: routing weight (kernel.py:364) and the store for the combine
    // (bf16, or fp32 unless G2_BF16).
#pragma unroll
    for (int m = 0; m < MTW; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = m * 16 + g * 4 + i;
            if (row < nrows) {
                const float w = w_lds[row];
                const size_t o = (size_t)(row0 + row) * H + n0 + r;
                if constexpr (MODE != G2_BF16) p.part_f32[o] = w * acc[m][i];
                else p.part[o] = f2bf(w * acc[m][i]);
            }
        }
    }
}

hipError_t launch_gemm2_wide(const Plan& p, const uint8_t* w2, const float* w2s, hipStream_t s) {
    // 32 rows x 128 columns, weights 2 k-blocks ahead, activations 1 ahead:
    // 74 VGPRs and 18 KB of LDS, so three 8-wave workgroups per CU. Measured
    // against 64- and 128-row tiles, 64-column workgroups and 4- and 8-deep
    // rings.
    dim3 grid(H / W2_N, max_mtiles(p.T, W2_BM));
    constexpr int MTW = W2_BM / 16;
    switch (gemm2_mode(p)) {
        case G2_SPLIT:
            hipLaunchKernelGGL((gemm2_wide_kernel<MTW, 2, 1, G2_SPLIT>), grid, dim3(64 * W2_NW), 0, s, p,
                               w2, w2s);
            break;
        case G2_F32:
            hipLaunchKernelGGL((gemm2_wide_kernel<MTW, 2, 1, G2_F32>), grid, dim3(64 * W2_NW), 0, s, p,
                               w2, w2s);
            break;
        default:
            hipLaunchKernelGGL((gemm2_wide_kernel<MTW, 2, 1, G2_BF16>), grid, dim3(64 * W2_NW), 0, s, p,
                               w2, w2s);
    }
    return hipGetLastError();
}

}  // namespace mimoe
