// Grouped FP8 GEMM1 + SwiGLU for medium row counts per expert ("wide" tiles).
//
// Same contract as gemm1_stream_kernel (solution/triton/kernel.py:69-186 and
// :301-330): act[s, j] = silu(G[s, I+j]) * G[s, j] with
//   G[s, n] = sum_kb sa[kb, tok(s)] * sb1[e, n/128, kb] * (A8[tok(s), kb-block] . W1[e, n, kb-block]).
//
// Shape (template <MTW, D, DA>): a workgroup of 4 waves owns BM = 16*MTW rows
// of one expert and 64 gate columns plus the 64 matching up columns; wave w
// owns gate columns j0..j0+15 (and up I+j0..) for all BM rows, so no two
// waves need the same weight bytes. Weights therefore go global -> VGPR
// through a D-deep register ring per wave (as in the stream kernel), while
// the BM gathered activation rows of a k-block, which every wave needs, are
// loaded once per workgroup into a DA-deep register staging ring and written
// to an LDS double buffer one k-block ahead of their use, together with the
// combined scales sa*sb (one product per row and half, computed once per
// workgroup from the tile's activation scales, which sit in LDS for the
// whole kernel): one barrier per k-block.
//
// All loads are ordinary compiler-visible loads, so the compiler's memory
// counters stay exact and a load waits only for its own data.
//
// With CH > 0 (T <= 64 * CH, CH = 4 up to T = 256, 8 up to 512) the kernel
// also stands in for the sort launch: its 4 waves ballot the 64-token chunks
// of the top-k ids (wave w takes chunks w, w + 4, ...) per local expert into LDS, every wave derives the expert
// counts, the bit-plane prefixes and the workgroup's row tile from those
// ballots, and a row's token is the n-th set bit of its expert's ballot in
// the right chunk. Workgroup (0, 0) writes the sort's tables for GEMM2 and
// the combine.
//
// Operand layout as in the stream kernel: lane l feeds row (l % 16) of a
// 16x128 operand with bytes [32g, 32g+32) of the k-block, g = l / 16 (whole-
// line weight loads, wl_frag). LDS rows are 128 bytes with chunk c of row r
// at position c ^ swz8(r); a lane reads chunks 2g and 2g + 1.
#include "sort_impl.hpp"
#include "tile_common.hpp"

namespace mimoe {

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }
constexpr int lcm_c(int a, int b) { return a / gcd_c(a, b) * b; }

constexpr int WIDE_NW = 4;                  // waves per workgroup
constexpr int WIDE_G = 16 * WIDE_NW;        // gate columns per workgroup
constexpr int WIDE_BM = 64;                 // rows per workgroup (see the launcher)

template <int MTW, int D, int DA, int CH>
__global__ __launch_bounds__(64 * WIDE_NW) void gemm1_wide_kernel(Plan p, const uint8_t* __restrict__ hs,
                                                                  const float* __restrict__ hs_scale,
                                                                  const uint8_t* __restrict__ w1,
                                                                  const float* __restrict__ w1s,
                                                                  int bm2) {
    constexpr int BM = 16 * MTW;
    constexpr int THREADS = 64 * WIDE_NW;
    constexpr int ROWS_PER_PASS = THREADS / 8;  // 8 threads x 16 B cover one 128-byte row
    constexpr int A_LD = BM / ROWS_PER_PASS;    // 16-byte loads per thread per k-block
    static_assert(BM % ROWS_PER_PASS == 0 && BM <= THREADS, "activation loader");
    static_assert(HB % D == 0 && HB % DA == 0, "ring depths must divide the k-block count");
    __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][BM * BLK];
    __shared__ float sa_lds[HB][BM];  // activation scales of the tile's rows, all k-blocks
    __shared__ __attribute__((aligned(16))) float cs_lds[2][2][BM];  // [buffer][gate, up][row]
    // CH > 0: token ballots per (64-token chunk, local expert), and the first
    // slot of each (chunk, expert) for the table writes
    constexpr bool SORT = CH > 0;
    constexpr int CPW = (CH + WIDE_NW - 1) / WIDE_NW;  // chunks per wave
    __shared__ unsigned long long s_bal[SORT ? CH : 1][EL];
    __shared__ int s_base[SORT ? CH : 1][EL];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    static_assert(THREADS % BM == 0, "scale loader row");

    // Row tile, and the tokens of this thread's loader rows and scale row.
    int e, row0, nrows, erows;  // erows: the expert's rows over all its row tiles
    int tok_a[A_LD], tok_s;
    if constexpr (SORT) {
        static_assert(BM == 64, "64-row tiles");
        const int nch = (p.T + 63) >> 6;  // 64-token chunks (T <= 64 * CH)
        // wave w ballots chunks w, w + WIDE_NW, ...
        // (with one chunk per wave every wave ballots, tokens past T as zeros)
#pragma unroll
        for (int j = 0; j < CPW; ++j) {
            const int c = wave + WIDE_NW * j;
            if (CPW > 1 && c >= nch) break;
            const int t = c * 64 + lane;
            emask_t m = 0;
            if (t < p.T) {
                int ids[TOPK];
                load_topk_ids(p.topk_ids + (size_t)t * TOPK_LD, ids);
#pragma unroll
                for (int k = 0; k < TOPK; ++k) {
                    const int l = ids[k] - p.local_offset;
                    m |= (unsigned)l < (unsigned)EL ? ebit(l) : (emask_t)0;
                }
            }
#pragma unroll
            for (int x = 0; x < EL; ++x) {
                const unsigned long long bal = __ballot((m >> x) & 1);
                if (lane == x) s_bal[c][x] = bal;
            }
        }
        __syncthreads();
        // lane x < EL: expert x's count over the chunks; prefixes as in wave_table
        int cnt = 0;
#pragma unroll
        for (int c = 0; c < CH; ++c)
            cnt += (CPW == 1 || c < nch) ? __popcll(s_bal[c][lane & (EL - 1)]) : 0;
        if (lane >= EL) cnt = 0;
        const int tiles = (cnt + BM - 1) / BM;
        const int v0 = excl_prefix_small<10>(cnt) + cnt;  // cnt <= T <= 512
        const int v1 = excl_prefix_small(tiles) + tiles;
        if (blockIdx.x == 0 && blockIdx.y == 0) {
            // the sort's tables: expert offsets, both tile prefixes, slots
            const int t2 = (cnt + bm2 - 1) / bm2;
            const int o2 = excl_prefix_small(t2);
            if (lane < EL && wave == 0) {
                p.meta[META_EXPERT_OFF + lane] = v0 - cnt;
                p.meta[META_MTILE1 + lane] = v1 - tiles;
                p.meta[META_MTILE2 + lane] = o2;
                if (lane == EL - 1) {
                    p.meta[META_EXPERT_OFF + EL] = v0;
                    p.meta[META_MTILE1 + EL] = v1;
                    p.meta[META_MTILE2 + EL] = o2 + t2;
                }
            }
#pragma unroll
            for (int j = 0; j < CPW; ++j) {
                const int c = wave + WIDE_NW * j;
                if (c >= nch) break;
                if (lane < EL) {  // chunk c's first slot of expert `lane`
                    int base = v0 - cnt;
                    for (int c2 = 0; c2 < c; ++c2) base += __popcll(s_bal[c2][lane]);
                    s_base[c][lane] = base;
                }
                const int t = c * 64 + lane;
                const TokLocal tl = load_local(p.topk_ids, p.topk_w, t, t < p.T, p.local_offset);
                place_with_prefix(p, t, t < p.T, tl, s_base, lane, c);
            }
        }
        const int mt = blockIdx.y;
        if (mt >= __builtin_amdgcn_readlane(v1, EL - 1)) return;  // the same for every wave
        const int ee = __popcll(__ballot(lane < EL && v1 <= mt));
        const int tfirst = __builtin_amdgcn_readlane(v1 - tiles, ee);
        const int sfirst = __builtin_amdgcn_readlane(v0 - cnt, ee);
        const int ce = __builtin_amdgcn_readlane(cnt, ee);
        e = ee;
        erows = ce;
        const int rank0 = (mt - tfirst) * BM;
        row0 = sfirst + rank0;
        nrows = min(BM, ce - rank0);
        // token of tile row `row`: the (rank0 + row)-th token of expert ee,
        // found by walking the chunks' ballots of ee (k < ce, so the walk ends
        // inside the last chunk at the latest)
        // (one chunk per wave: the CH ballots held in registers; more: read
        // from LDS as the walk goes, which keeps scalar registers from spilling)
        unsigned long long eb[CPW == 1 ? CH : 1];
#pragma unroll
        for (int c = 0; c < (CPW == 1 ? CH : 1); ++c) eb[c] = s_bal[c][ee];
        auto row_token = [&](int row) __attribute__((always_inline)) {
            int k = rank0 + min(row, nrows - 1);
            int chunk = 0;
            unsigned long long bc = eb[0];
            if constexpr (CPW == 1) {
#pragma unroll
                for (int c = 0; c < CH - 1; ++c) {
                    const int cc = __popcll(eb[c]);
                    if (chunk == c && k >= cc) {
                        k -= cc;
                        chunk = c + 1;
                        bc = eb[c + 1];
                    }
                }
            } else {
                for (int c = 0; c + 1 < nch; ++c) {
                    const int cc = __popcll(bc);
                    if (k < cc) break;
                    k -= cc;
                    chunk = c + 1;
                    bc = s_bal[c + 1][ee];
                }
            }
            return chunk * 64 + nth_set_bit(bc, k);
        };
#pragma unroll
        for (int i = 0; i < A_LD; ++i) tok_a[i] = row_token((tid >> 3) + ROWS_PER_PASS * i);
        tok_s = row_token(tid % BM);
    } else {
        if (!find_tile(p.meta, META_MTILE1, blockIdx.y, BM, e, row0, nrows)) return;
        erows = p.meta[META_EXPERT_OFF + e + 1] - p.meta[META_EXPERT_OFF + e];
#pragma unroll
        for (int i = 0; i < A_LD; ++i)
            tok_a[i] = p.sorted_tok[row0 + min((tid >> 3) + ROWS_PER_PASS * i, nrows - 1)];
        tok_s = p.sorted_tok[row0 + min(tid % BM, nrows - 1)];
    }
    const int jb = blockIdx.x * WIDE_G;  // first gate column of the workgroup
    const int j0 = jb + wave * 16;       // first gate column of this wave
    const int r = lane & 15, g = lane >> 4;

    // weight fragments of this wave (gate and up rows of W1[e])
    // weights of expert e through a buffer resource: gate rows, then up rows I further
    e = __builtin_amdgcn_readfirstlane(e);
    const __amdgpu_buffer_rsrc_t wr = wrsrc(w1 + (size_t)e * N1 * H, (uint32_t)((size_t)N1 * H));
    const uint32_t bg_off = (uint32_t)((size_t)j0 * H + wl_off(lane, H));
    const uint32_t bu_off = bg_off + (uint32_t)((size_t)I * H);
    // 64 gate columns lie inside one 128-column scale block, as do the up ones
    const float* sbg_ptr = w1s + ((size_t)e * N1B + jb / BLK) * HB;
    const float* sbu_ptr = w1s + ((size_t)e * N1B + (I + jb) / BLK) * HB;

    // activation loader: thread t copies chunk t%8 of rows t/8 + 32i
    const int ac = tid & 7;
    const uint8_t* a_src[A_LD];
    uint32_t a_dst[A_LD];
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
        const int row = (tid >> 3) + ROWS_PER_PASS * i;
        a_src[i] = hs + (size_t)tok_a[i] * H + ac * 16;
        a_dst[i] = row * BLK + ((ac ^ swz8(row)) << 4);
    }

    v4f accg[MTW], accu[MTW];
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < MTW; ++m) { accg[m] = zero; accu[m] = zero; }

    // The k loop, with the weight load policy of the tile's expert (NT: non-
    // temporal, when this is its only row tile). Measured against a policy
    // per launch from T: level at T = 100 / 256 / 512 with random routing,
    // 13 % faster at T=1024 offset 64 (399 slots, one tile per expert), 5 %
    // with every token on the same 8 experts at T=256; the two copies of the
    // loop leave the kernel at 136 VGPRs, no spills.
    auto body = [&](auto nt) __attribute__((always_inline)) {
        constexpr bool NT = decltype(nt)::value;
        WRaw bg[D], bu[D];
        v4i ast[DA][A_LD];
        float sgs[DA], sus[DA];  // weight scales of the staged k-blocks (uniform)

        auto load_w = [&](int d, int kb) __attribute__((always_inline)) {
            bg[d] = ld_wraw<NT>(wr, bg_off + kb * BLK, 8 * H);
            bu[d] = ld_wraw<NT>(wr, bu_off + kb * BLK, 8 * H);
        };
        auto load_a = [&](int s, int kb) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < A_LD; ++i) ast[s][i] = ld16(a_src[i] + kb * BLK);
            sgs[s] = sbg_ptr[kb];
            sus[s] = sbu_ptr[kb];
        };
        auto store_a = [&](int s, int buf, int kb) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < A_LD; ++i)
                *reinterpret_cast<v4i*>(&a_lds[buf][a_dst[i]]) = ast[s][i];
            if (tid < BM) {
                const float sa = sa_lds[kb][tid];
                cs_lds[buf][0][tid] = sa * sgs[s];
                cs_lds[buf][1][tid] = sa * sus[s];
            }
        };
        auto compute = [&](int d, int buf) __attribute__((always_inline)) {
            const uint8_t* sA = a_lds[buf];
            const v8i fg = wl_frag(bg[d]);
            const v8i fu = wl_frag(bu[d]);
#pragma unroll
            for (int m = 0; m < MTW; ++m) {
                const int row = m * 16 + r;
                const uint8_t* base = sA + row * BLK;
                const int sw = swz8(row);
                const v4i lo = lds16(base + (((2 * g) ^ sw) << 4));
                const v4i hi = lds16(base + (((2 * g + 1) ^ sw) << 4));
                const v8i a = (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                const v4f pg = mfma_f8_16x16x128(a, fg, zero);
                const v4f pu = mfma_f8_16x16x128(a, fu, zero);
                const float4 sg = *reinterpret_cast<const float4*>(&cs_lds[buf][0][m * 16 + g * 4]);
                const float4 su = *reinterpret_cast<const float4*>(&cs_lds[buf][1][m * 16 + g * 4]);
                accg[m][0] += pg[0] * sg.x; accg[m][1] += pg[1] * sg.y;
                accg[m][2] += pg[2] * sg.z; accg[m][3] += pg[3] * sg.w;
                accu[m][0] += pu[0] * su.x; accu[m][1] += pu[1] * su.y;
                accu[m][2] += pu[2] * su.z; accu[m][3] += pu[3] * su.w;
            }
            // The products are pure arithmetic, which the compiler would
            // otherwise sink below the following barriers into the last unrolled
            // k-block, keeping every LDS fragment of the unrolled body live.
            // Naming the accumulators here pins each k-block's work before its
            // barrier.
#pragma unroll
            for (int m = 0; m < MTW; ++m) asm volatile("" : "+v"(accg[m]), "+v"(accu[m]));
        };

        // Activation scales of every k-block into LDS once: in the loop they come
        // from LDS, so no vector load there waits on anything but its own data.
        for (int i = tid; i < HB * BM; i += THREADS) {
            const int kb = i / BM, m = i % BM;  // m == tid % BM: the row of tok_s
            sa_lds[kb][m] = hs_scale[(size_t)kb * p.T + tok_s];
        }
        __syncthreads();

        // Prologue: the loads that iterations -D..-1 of the loop would have
        // issued, in their order (iteration j loads A(j+1+DA), then W(j+D); the
        // store of A(0) to LDS buffer 0 belongs to iteration -1), so every wait in
        // the loop sees as many younger loads on the first trip as on later ones.
        static_assert(D > DA, "prologue order");
        // (sched_barrier keeps the scheduler from reordering the groups.)
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int a = d - (D - DA - 1);
            if (a >= 0) {
                if (a == DA) store_a(0, 0, 0);  // frees staging slot 0 for A(DA)
                load_a(a % DA, a);
                __builtin_amdgcn_sched_barrier(0);
            }
            load_w(d, d);
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();

        // k-block kb: stage kb+1 into the other LDS buffer (its staging slot is
        // refilled with kb+1+DA), consume kb, refill the weight ring with kb+D.
        // Loads past the last k-block re-read the last one; their values are
        // never consumed.
        constexpr int U = lcm_c(lcm_c(D, DA), 2);  // ring slots and LDS buffer repeat every U
        static_assert(HB % U == 0, "unroll");
#pragma unroll 1
        for (int kb0 = 0; kb0 < HB; kb0 += U) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int kb = kb0 + u;
                const int buf = u & 1;
                const int s = (u + 1) % DA;  // staging slot holding k-block kb+1
                if (kb + 1 < HB) {
                    store_a(s, buf ^ 1, kb + 1);
                    load_a(s, min(kb + 1 + DA, HB - 1));
                }
                compute(u % D, buf);
                load_w(u % D, min(kb + D, HB - 1));
                __syncthreads();
            }
        }
    };
    if (__builtin_amdgcn_readfirstlane(erows) <= BM) body(BoolC<true>{});
    else body(BoolC<false>{});

#pragma unroll
    for (int m = 0; m < MTW; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = m * 16 + g * 4 + i;
            if (row < nrows) {
                const float v = silu(accu[m][i]) * accg[m][i];
                store_act(p, (size_t)(row0 + row) * I + j0 + r, v);
            }
        }
    }
}

hipError_t launch_gemm1_wide(const Plan& p, const uint8_t* hs, const float* hs_scale,
                             const uint8_t* w1, const float* w1s, hipStream_t s) {
    // 64 rows, weights 2 k-blocks ahead, activations 1 ahead: 130 VGPRs, so
    // three waves per SIMD. Measured against 32-, 96- and 128-row tiles and
    // 4- to 8-deep rings, more resident waves beat deeper rings here.
    dim3 grid(I / WIDE_G, max_mtiles(p.T, WIDE_BM));
    hipLaunchKernelGGL((gemm1_wide_kernel<WIDE_BM / 16, 2, 1, 0>), grid, dim3(64 * WIDE_NW), 0, s,
                       p, hs, hs_scale, w1, w1s, 0);
    return hipGetLastError();
}

// Largest T the sorting wide kernel takes: 4 chunks of 64 tokens (one per
// wave) to T = 256, 8 (two per wave) to T = 512. Per call against the
// separate sort launch: T=256 220.5 -> 215.9 us, T=200 208.0 -> 202.5, T=160
// 205.1 -> 199.2 (GEMM1 +1 us, the ~7 us sort launch gone); T=320 176.7 ->
// 173.7, T=448 260.4 -> 258.2, T=512 182.7 -> 180.4 (four passes, one
// process per build); at T=576 the separate sort was 2 us faster.
constexpr int WIDE_SORT_CH_SMALL = 4, WIDE_SORT_CH = 8;
constexpr int WIDE_SORT_MAX_T = 64 * WIDE_SORT_CH;

bool gemm1_wide_sorts_supported(int T) { return T > 0 && T <= WIDE_SORT_MAX_T; }

hipError_t launch_gemm1_wide_sorting(const Plan& p, const uint8_t* hs, const float* hs_scale,
                                     const uint8_t* w1, const float* w1s, int bm2, hipStream_t s) {
    if (p.T <= 0) return hipSuccess;
    if (p.T > WIDE_SORT_MAX_T) return hipErrorInvalidValue;
    dim3 grid(I / WIDE_G, max_mtiles(p.T, WIDE_BM));
    if (p.T <= 64 * WIDE_SORT_CH_SMALL)
        hipLaunchKernelGGL((gemm1_wide_kernel<WIDE_BM / 16, 2, 1, WIDE_SORT_CH_SMALL>), grid,
                           dim3(64 * WIDE_NW), 0, s, p, hs, hs_scale, w1, w1s, bm2);
    else
        hipLaunchKernelGGL((gemm1_wide_kernel<WIDE_BM / 16, 2, 1, WIDE_SORT_CH>), grid,
                           dim3(64 * WIDE_NW), 0, s, p, hs, hs_scale, w1, w1s, bm2);
    return hipGetLastError();
}

}  // namespace mimoe
