// Grouped FP8 GEMM1 + SwiGLU, LDS-tiled variant for many rows per expert.
//
// Same contract as gemm1_stream_kernel (solution/triton/kernel.py:69-186 and
// :301-330): act[s, j] = silu(G[s, I+j]) * G[s, j] with
//   G[s, n] = sum_kb sa[kb, tok(s)] * sb1[e, n/128, kb] * (A8[tok(s), kb-block] . W1[e, n, kb-block]).
//
// A workgroup of WM x WN waves computes a tile of BM = 64*WM rows (slots of
// one expert) by BG = 64*WN gate columns plus the BG matching up columns.
// Per 128-wide k-block (one scale block) the A rows (gathered by token), the
// 2*BG weight rows and the BM activation scales are copied global -> LDS
// with global_load_lds_dwordx4 into one of two stages, so the copy of
// k-block kb+1 overlaps the MFMAs on kb; one barrier per k-block.
// Each wave owns 64 rows x (64 gate + 64 up) columns: 4 x 8 MFMA tiles of
// v_mfma_scale_f32_16x16x128_f8f6f4, each scaled by sa*sb in fp32 as it is
// accumulated. The SwiGLU epilogue pairs gate and up columns in registers.
//
// LDS rows are 128 bytes; 16-byte chunk c of row r sits at position
// c ^ swz8(r), so the 16 rows read by lanes 0..15 hit distinct banks.
#include "tile_common.hpp"

namespace mimoe {

template <int WM, int WN>
struct G1Tile {
    static constexpr int NW = WM * WN;
    static constexpr int THREADS = 64 * NW;
    static constexpr int BM = 64 * WM;
    static constexpr int BG = 64 * WN;
    static constexpr int NT = I / BG;
    static constexpr int A_BYTES = BM * BLK;
    static constexpr int B_BYTES = 2 * BG * BLK;
    static constexpr int SA_BYTES = BM * 4;
    static constexpr int STAGE = A_BYTES + B_BYTES + SA_BYTES;
    static constexpr int A_LD = A_BYTES / 1024 / NW;  // 1 KB copies per wave per stage
    static constexpr int B_LD = B_BYTES / 1024 / NW;
    static constexpr int SA_WAVES = BM / 64;          // waves copying one scale each per lane
    static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "loader split");
    static_assert(SA_WAVES <= NW, "scale loader");
    static_assert(2 * STAGE <= 160 * 1024, "LDS budget");
};

template <int WM, int WN, int GM>
__global__ __launch_bounds__(64 * WM * WN) void gemm1_tile_kernel(
    Plan p, const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w1, const float* __restrict__ w1s) {
    using C = G1Tile<WM, WN>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE];

    int e, row0, nrows, nt;
    if (!tile_coords<C::NT, GM>(p.meta, META_MTILE1, C::BM, e, row0, nrows, nt)) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int jb = nt * C::BG;

    // Loader: in its i-th copy, wave w fills LDS rows 8*(w*LD + i) .. +7;
    // lane l takes row +l/8, chunk position l%8.
    uint32_t a_off[C::A_LD], b_off[C::B_LD];
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
        const int row = 8 * (wave * C::A_LD + i) + (lane >> 3);
        const int c = (lane & 7) ^ swz8(row);
        const int tok = p.sorted_tok[row0 + min(row, nrows - 1)];
        a_off[i] = (uint32_t)tok * H + c * 16;
    }
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) {
        const int row = 8 * (wave * C::B_LD + i) + (lane >> 3);
        const int c = (lane & 7) ^ swz8(row);
        const int wrow = row < C::BG ? jb + row : I + jb + (row - C::BG);
        b_off[i] = (uint32_t)((e * N1 + wrow) * H + c * 16);
    }
    uint32_t sa_off = 0;
    if (wave < C::SA_WAVES) {
        const int row = 64 * wave + lane;
        sa_off = (uint32_t)p.sorted_tok[row0 + min(row, nrows - 1)];
    }

    // Copies whose 8 rows all lie past the expert's last row are skipped
    // (wave-uniform): those LDS rows only feed MFMA rows that are never
    // stored, and at medium T most of a 256-row tile is such rows.
    auto issue = [&](int stage, int kb) __attribute__((always_inline)) {
        uint8_t* s = smem + stage * C::STAGE;
#pragma unroll
        for (int i = 0; i < C::A_LD; ++i)
            if (8 * (wave * C::A_LD + i) < nrows)
                g2l16(hs + a_off[i] + kb * BLK, s + (wave * C::A_LD + i) * 1024);
#pragma unroll
        for (int i = 0; i < C::B_LD; ++i)
            g2l16(w1 + b_off[i] + kb * BLK, s + C::A_BYTES + (wave * C::B_LD + i) * 1024);
        if (wave < C::SA_WAVES)
            g2l4(hs_scale + (size_t)kb * p.T + sa_off, s + C::A_BYTES + C::B_BYTES + wave * 256);
    };

    const int wm = wave % WM, wn = wave / WM;
    const int r = lane & 15, g = lane >> 4;
    const float* sbg_p = w1s + ((size_t)e * N1B + jb / BLK) * HB;
    const float* sbu_p = w1s + ((size_t)e * N1B + (I + jb) / BLK) * HB;

    v4f acc[4][8];
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < 8; ++n) acc[m][n] = zero;

    issue(0, 0);
    wait_vmem();
    __syncthreads();

#pragma unroll 1
    for (int kb = 0; kb < HB; ++kb) {
        const int cur = kb & 1;
        const uint8_t* sA = smem + cur * C::STAGE;
        const uint8_t* sB = sA + C::A_BYTES;
        const float* sSA = reinterpret_cast<const float*>(sB + C::B_BYTES);

        // Waves whose 64 rows lie past the expert's last row (partial row
        // tiles) only copy; the branch is wave-uniform.
        const bool active = wm * 64 < nrows;
        v8i a[4];
        if (active) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int row = wm * 64 + m * 16 + r;
                const uint8_t* base = sA + row * BLK;
                const int sw = swz8(row);
                const v4i lo = lds16(base + ((g ^ sw) << 4));
                const v4i hi = lds16(base + (((g + 4) ^ sw) << 4));
                a[m] = (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            }
        }
        // The copy of k-block kb+1 goes out after this wave's A reads, so its
        // LDS writes do not compete with them.
        if (kb + 1 < HB) issue(cur ^ 1, kb + 1);
        if (!active) {
            wait_vmem();
            __syncthreads();
            continue;
        }
        // Per-row scale products sa*sb for the gate half, then (re-read from
        // LDS) for the up half: one set of 16 registers instead of two.
        float cs[4][4];
        auto set_scales = [&](float sb) __attribute__((always_inline)) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float4 s4 = *reinterpret_cast<const float4*>(sSA + wm * 64 + m * 16 + g * 4);
                cs[m][0] = s4.x * sb; cs[m][1] = s4.y * sb; cs[m][2] = s4.z * sb; cs[m][3] = s4.w * sb;
            }
        };
        // B fragments are read one column tile ahead so the LDS latency of
        // tile n+1 overlaps the MFMAs of tile n.
        auto read_b = [&](int n) __attribute__((always_inline)) {
            const int brow = (n < 4) ? (wn * 64 + n * 16 + r) : (C::BG + wn * 64 + (n - 4) * 16 + r);
            const uint8_t* base = sB + brow * BLK;
            const int sw = swz8(brow);
            const v4i lo = lds16(base + ((g ^ sw) << 4));
            const v4i hi = lds16(base + (((g + 4) ^ sw) << 4));
            return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        };
        set_scales(sbg_p[kb]);
        v8i bnext = read_b(0);
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            if (n == 4) set_scales(sbu_p[kb]);
            const v8i b = bnext;
            if (n < 7) bnext = read_b(n + 1);
            // four independent MFMAs, then their scale-and-accumulate
            v4f pr[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) pr[m] = mfma_f8_16x16x128(a[m], b, zero);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                acc[m][n][0] += pr[m][0] * cs[m][0];
                acc[m][n][1] += pr[m][1] * cs[m][1];
                acc[m][n][2] += pr[m][2] * cs[m][2];
                acc[m][n][3] += pr[m][3] * cs[m][3];
            }
        }
        wait_vmem();
        __syncthreads();
    }

#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int n = 0; n < 4; ++n) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = wm * 64 + m * 16 + g * 4 + i;
                if (row < nrows) {
                    const float v = silu(acc[m][n + 4][i]) * acc[m][n][i];
                    store_act(p, (size_t)(row0 + row) * I + jb + wn * 64 + n * 16 + r, v);
                }
            }
        }
    }
}

// The same tile with the MFMA operands swapped and the MFMAs software-
// pipelined against their scale FMAs (variant 18).
//
// Weight rows are the MFMA's A operand and gathered activation rows its B
// operand, so lane l receives D[4g+v][l%16]: four output columns 4g..4g+3 of
// one row (r = l%16) of a 16x16 tile. The per-(row, k-block) activation
// scale and the per-(128 columns, k-block) weight scale then combine into a
// single factor u per lane and tile: 8 products per k-block per lane instead
// of 32, and the SwiGLU epilogue stores 4 adjacent bf16 (8 bytes) per lane.
// The activation scales sit in LDS as [row group][r][m], so one 16-byte read
// gives a lane the scales of its rows m*16 + r (m = 0..3).
//
// Inside a k-block the 32 MFMAs of a wave (8 column tiles x 4 row tiles) run
// as one sequence; the four scale-and-accumulate FMAs of MFMA t issue after
// MFMA t+2, so they execute while the matrix core works on later tiles
// rather than waiting on the result just issued. The last two MFMAs' FMAs
// carry into the next k-block. Weight fragments are read from LDS one column
// tile ahead.
template <int WM, int WN, int GM>
__global__ __launch_bounds__(64 * WM * WN) void gemm1_tile_t_kernel(
    Plan p, const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w1, const float* __restrict__ w1s) {
    using C = G1Tile<WM, WN>;
    static_assert(WN * 64 * 2 == 2 * C::BG && C::BG == 64 * WN, "column tiling");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE];

    int e, row0, nrows, nt;
    if (!tile_coords<C::NT, GM>(p.meta, META_MTILE1, C::BM, e, row0, nrows, nt)) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int jb = nt * C::BG;

    uint32_t a_off[C::A_LD], b_off[C::B_LD];
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
        const int row = 8 * (wave * C::A_LD + i) + (lane >> 3);
        const int c = (lane & 7) ^ swzq(row);
        const int tok = p.sorted_tok[row0 + min(row, nrows - 1)];
        a_off[i] = (uint32_t)tok * H + c * 16;
    }
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) {
        const int row = 8 * (wave * C::B_LD + i) + (lane >> 3);
        const int c = (lane & 7) ^ swzq(row);
        const int wrow = row < C::BG ? jb + row : I + jb + (row - C::BG);
        b_off[i] = (uint32_t)((e * N1 + wrow) * H + c * 16);
    }
    // scale loader: wave w < WM copies the 64 scales of rows 64w.., lane l
    // to LDS position 64w + l, which holds row 64w + (l % 4) * 16 + l / 4
    uint32_t sa_off = 0;
    if (wave < C::SA_WAVES) {
        const int row = 64 * wave + (lane & 3) * 16 + (lane >> 2);
        sa_off = (uint32_t)p.sorted_tok[row0 + min(row, nrows - 1)];
    }

    auto issue = [&](int stage, int kb) __attribute__((always_inline)) {
        uint8_t* s = smem + stage * C::STAGE;
#pragma unroll
        for (int i = 0; i < C::A_LD; ++i)
            if (8 * (wave * C::A_LD + i) < nrows)
                g2l16(hs + a_off[i] + kb * BLK, s + (wave * C::A_LD + i) * 1024);
#pragma unroll
        for (int i = 0; i < C::B_LD; ++i)
            g2l16(w1 + b_off[i] + kb * BLK, s + C::A_BYTES + (wave * C::B_LD + i) * 1024);
        if (wave < C::SA_WAVES)
            g2l4(hs_scale + (size_t)kb * p.T + sa_off, s + C::A_BYTES + C::B_BYTES + wave * 256);
    };

    const int wm = wave % WM, wn = wave / WM;
    const int r = lane & 15, g = lane >> 4;
    const float* sbg_p = w1s + ((size_t)e * N1B + jb / BLK) * HB;
    const float* sbu_p = w1s + ((size_t)e * N1B + (I + jb) / BLK) * HB;

    // acc[n][m]: column tile n (0..3 gate, 4..7 up) x row tile m
    v4f acc[8][4];
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[n][m] = zero;

    issue(0, 0);
    wait_vmem();
    __syncthreads();

    const bool active = wm * 64 < nrows;  // wave-uniform: rows past the expert only copy
    // MFMA results of the last two tiles of the previous k-block and their
    // scale factors, applied early in the next one
    v4f carry0 = zero, carry1 = zero;
    float cu0 = 0.f, cu1 = 0.f;

#pragma unroll 1
    for (int kb = 0; kb < HB; ++kb) {
        const int cur = kb & 1;
        const uint8_t* sA = smem + cur * C::STAGE;
        const uint8_t* sB = sA + C::A_BYTES;
        const float* sSA = reinterpret_cast<const float*>(sB + C::B_BYTES);

        v8i a[4];
        float4 s4 = {0.f, 0.f, 0.f, 0.f};
        auto read_b = [&](int n) __attribute__((always_inline)) {
            const int brow = (n < 4) ? (wn * 64 + n * 16 + r) : (C::BG + wn * 64 + (n - 4) * 16 + r);
            const uint8_t* base = sB + brow * BLK;
            const int sw = swzq(brow);
            const v4i lo = lds16(base + ((g ^ sw) << 4));
            const v4i hi = lds16(base + (((g + 4) ^ sw) << 4));
            return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        };
        v8i bcur = {0, 0, 0, 0, 0, 0, 0, 0};
        if (active) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int row = wm * 64 + m * 16 + r;
                const uint8_t* base = sA + row * BLK;
                const int sw = swzq(row);
                const v4i lo = lds16(base + ((g ^ sw) << 4));
                const v4i hi = lds16(base + (((g + 4) ^ sw) << 4));
                a[m] = (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            }
            s4 = *reinterpret_cast<const float4*>(sSA + wm * 64 + r * 4);
            bcur = read_b(0);
        }
        // The copy of k-block kb+1 goes out after this wave's fragment reads.
        if (kb + 1 < HB) issue(cur ^ 1, kb + 1);
        if (!active) {
            wait_vmem();
            __syncthreads();
            continue;
        }
        const float sbg = sbg_p[kb], sbu = sbu_p[kb];
        const float sam[4] = {s4.x, s4.y, s4.z, s4.w};
        float ug[4], uu[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) { ug[m] = sam[m] * sbg; uu[m] = sam[m] * sbu; }

        v4f pr[32];
        v8i bnext = bcur;
#pragma unroll
        for (int t = 0; t < 32; ++t) {
            const int n = t >> 2, m = t & 3;
            if (m == 0 && n + 1 < 8) bnext = read_b(n + 1);
            pr[t] = mfma_f8_16x16x128(bcur, a[m], zero);
            if (m == 3) bcur = bnext;
            if (t >= 2) {
                const int tn = (t - 2) >> 2, tm = (t - 2) & 3;
                const float u = tn < 4 ? ug[tm] : uu[tm];
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[tn][tm][v] += pr[t - 2][v] * u;
            } else if (t == 0) {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[7][2][v] += carry0[v] * cu0;
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[7][3][v] += carry1[v] * cu1;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        carry0 = pr[30];
        carry1 = pr[31];
        cu0 = uu[2];
        cu1 = uu[3];
        wait_vmem();
        __syncthreads();
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        acc[7][2][v] += carry0[v] * cu0;
        acc[7][3][v] += carry1[v] * cu1;
    }

    if (!active) return;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int row = wm * 64 + m * 16 + r;
        if (row < nrows) {
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                uint32_t w[2], wl[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float v0 = silu(acc[n + 4][m][2 * h]) * acc[n][m][2 * h];
                    const float v1 = silu(acc[n + 4][m][2 * h + 1]) * acc[n][m][2 * h + 1];
                    const uint16_t h0 = f2bf(v0), h1 = f2bf(v1);
                    w[h] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                    wl[h] = (uint32_t)f2bf(v0 - bf2f(h0)) | ((uint32_t)f2bf(v1 - bf2f(h1)) << 16);
                }
                const size_t idx = (size_t)(row0 + row) * I + jb + wn * 64 + n * 16 + 4 * g;
                *reinterpret_cast<uint2*>(p.act + idx) = make_uint2(w[0], w[1]);
                if (p.act_lo) *reinterpret_cast<uint2*>(p.act_lo + idx) = make_uint2(wl[0], wl[1]);
            }
        }
    }
}

// The same 256 x (128 + 128) tile as one software pipeline (variant 19).
//
// The 8 waves form 2 row groups x 4 column groups: wave (wm, wn) owns rows
// 128wm .. 128wm+127 (8 row tiles of 16) and gate columns 32wn .. 32wn+31
// (2 column tiles) plus the matching up columns, 32 MFMAs per k-block as in
// variants 3 and 18. A wave keeps its four weight fragments of a k-block in
// registers (32 VGPRs) and streams the 8 activation fragments from LDS. The
// two barriers of a k-block sit inside the MFMA stream, so no wave waits on
// LDS or on a barrier with an empty matrix core queue:
//   * barrier X, after row tile 0: every wave has its weight fragments of
//     k-block kb in registers (read during k-block kb-1), so that stage's
//     weight region is free and the copy of the weights of k-block kb+2 goes
//     there: a weight copy has ~1.75 k-blocks to arrive;
//   * barrier Y, before row tile 7: the copies of k-block kb+1 have landed
//     (vmcnt leaves only the weights of kb+2 outstanding), and every wave has
//     read its last activation fragment of kb, so the activation rows of
//     k-block kb+2 are copied into this stage's activation region (one
//     k-block to arrive). During row tile 7 each wave reads the next
//     k-block's weight fragments into the same registers right after their
//     last MFMA, its first activation fragment and its row scales.
// Weights are the operand that comes from HBM (an expert's column tile is
// read by its few row tiles, an activation row tile by all 16 column tiles).
// MFMA operands are swapped as in variant 18 (weights are the A operand, so
// a lane holds four output columns of one row and one scale factor per
// tile), and each MFMA's four scale FMAs issue after the MFMA four later
// (the next row tile's, same column tile); the last row tile's carry into
// the next k-block.
struct G1W {
    static constexpr int NW = 8;
    static constexpr int THREADS = 64 * NW;
    static constexpr int BM = 256;
    static constexpr int BG = 128;
    static constexpr int NT = I / BG;
    static constexpr int A_BYTES = BM * BLK;
    static constexpr int B_BYTES = 2 * BG * BLK;
    static constexpr int SA_BYTES = BM * 4;
    static constexpr int STAGE = A_BYTES + B_BYTES + SA_BYTES;
    static constexpr int A_LD = A_BYTES / 1024 / NW;
    static constexpr int B_LD = B_BYTES / 1024 / NW;
    static_assert(A_LD == 4 && B_LD == 4, "loader split: vmcnt(4) leaves one k-block of weight copies");
    static_assert(2 * STAGE + 2 * 64 * 4 <= 160 * 1024, "LDS budget");
    static_assert(HB <= 64 && HB >= 2, "weight scales: one lane per k-block");
};

template <int GM>
__global__ __launch_bounds__(512) void gemm1_tile_w_kernel(
    Plan p, const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w1, const float* __restrict__ w1s) {
    using C = G1W;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE];
    __shared__ __attribute__((aligned(16))) float s_sb[2 * 64];  // [gate | up][kb] weight scales

    int e, row0, nrows, nt;
    if (!tile_coords<C::NT, GM>(p.meta, p.g1_mtile, C::BM, e, row0, nrows, nt)) return;
    // wave-uniform by construction; kept in SGPRs for the copies' scalar bases
    e = __builtin_amdgcn_readfirstlane(e);
    nt = __builtin_amdgcn_readfirstlane(nt);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int jb = nt * C::BG;

    uint32_t a_off[C::A_LD], b_off[C::B_LD];
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
        const int row = 8 * (wave * C::A_LD + i) + (lane >> 3);
        const int c = (lane & 7) ^ swzq(row);
        const int tok = p.sorted_tok[row0 + min(row, nrows - 1)];
        a_off[i] = (uint32_t)tok * H + c * 16;
    }
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) {
        const int row = 8 * (wave * C::B_LD + i) + (lane >> 3);
        const int c = (lane & 7) ^ swzq(row);
        const int wrow = row < C::BG ? jb + row : I + jb + (row - C::BG);
        b_off[i] = (uint32_t)((e * N1 + wrow) * H + c * 16);
    }
    // Activation scales sit in LDS as [row group wm][r][m] (row 128wm + 16m
    // + r), so a lane reads the scales of its 8 rows as two 16-byte vectors.
    // Waves 0..3 copy 64 of them each; lane l of wave w takes index 64w + l.
    uint32_t sa_off = 0;
    if (wave < 4) {
        const int idx = 64 * wave + lane;
        const int row = 128 * (idx >> 7) + 16 * (idx & 7) + ((idx & 127) >> 3);
        sa_off = (uint32_t)p.sorted_tok[row0 + min(row, nrows - 1)];
    }

    // copies address their rows as a k-block base (SGPRs) + a 32-bit offset
    auto issue_a = [&](int stage, int kb) __attribute__((always_inline)) {
        uint8_t* s = smem + stage * C::STAGE;
        const uint8_t* base = hs + kb * BLK;
#pragma unroll
        for (int i = 0; i < C::A_LD; ++i) g2l16s(base, a_off[i], s + (wave * C::A_LD + i) * 1024);
        if (wave < 4) g2l4s(hs_scale + (size_t)kb * p.T, sa_off * 4, s + C::A_BYTES + C::B_BYTES + wave * 256);
    };
    auto issue_b = [&](int stage, int kb) __attribute__((always_inline)) {
        uint8_t* s = smem + stage * C::STAGE + C::A_BYTES;
        const uint8_t* base = w1 + kb * BLK;
#pragma unroll
        for (int i = 0; i < C::B_LD; ++i) g2l16s(base, b_off[i], s + (wave * C::B_LD + i) * 1024);
    };

    // The tile's weight scales (one 128-column block of gate, one of up, for
    // every k-block) are copied once by waves 4 and 5.
    if (wave == 4 || wave == 5) {
        const int nb = wave == 4 ? jb / BLK : (I + jb) / BLK;
        if (lane < HB) g2l4s(w1s + ((size_t)e * N1B + nb) * HB, lane * 4, s_sb + (wave - 4) * 64);
    }
    // Prologue, in the order of the steady state: weights and activations of
    // k-block 0, weights of 1; then (after the barrier that plays barrier Y
    // of k-block -1) activations of 1.
    issue_b(0, 0);
    issue_a(0, 0);
    issue_b(1, 1);
    asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
    issue_a(1, 1);

    const int wn = wave & 3, wm = wave >> 2;
    const int r = lane & 15, g = lane >> 4;
    const bool active = wm * 128 < nrows;  // wave-uniform: rows past the expert only copy

    auto frag = [&](const uint8_t* s, int row) __attribute__((always_inline)) {
        const uint8_t* base = s + row * BLK;
        const int sw = swzq(row);
        const v4i lo = lds16(base + ((g ^ sw) << 4));
        const v4i hi = lds16(base + (((g + 4) ^ sw) << 4));
        return (v8i){lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    };
    auto brow = [&](int n) __attribute__((always_inline)) {
        return n < 2 ? 32 * wn + 16 * n + r : C::BG + 32 * wn + 16 * (n - 2) + r;
    };

    if (!active) {
        // Rows past the expert: copies and barriers only, in step with the
        // other waves (two barriers per k-block).
#pragma unroll 1
        for (int kb = 0; kb < HB; ++kb) {
            const int kb2 = min(kb + 2, HB - 1);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            issue_b(kb & 1, kb2);
            asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            issue_a(kb & 1, kb2);
        }
        wait_vmem();  // no copy into LDS may be pending when the workgroup ends
        return;
    }

    // The arithmetic of one wave with MT row tiles (8, or 4 when the wave's
    // rows past 64 lie beyond the expert: partial row tiles at the end of an
    // expert then cost half the MFMAs). Both forms run the same copies and
    // barriers.
    auto compute = [&](auto mt_c) __attribute__((always_inline)) {
        constexpr int MT = decltype(mt_c)::value;
        static_assert(MT >= 3 && MT <= 8, "barrier X after row tile 0, Y before the last");
        constexpr int NTT = 4 * MT;        // MFMAs per k-block
        constexpr int TY = 4 * (MT - 1);   // barrier Y before the last row tile
        // scale factors sa * sb of this lane's rows (128wm + 16m + r) for the
        // gate and up column blocks of k-block kb (stage s)
        float ug[MT], uu[MT];
        auto scales = [&](const uint8_t* s, int kb) __attribute__((always_inline)) {
            const float* sSA = reinterpret_cast<const float*>(s + C::A_BYTES + C::B_BYTES);
            const float4 s0 = *reinterpret_cast<const float4*>(sSA + wm * 128 + r * 8);
            const float4 s1 = *reinterpret_cast<const float4*>(sSA + wm * 128 + r * 8 + 4);
            const float sa[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
            const float sbg = s_sb[kb], sbu = s_sb[64 + kb];
#pragma unroll
            for (int m = 0; m < MT; ++m) { ug[m] = sa[m] * sbg; uu[m] = sa[m] * sbu; }
        };

        v4f acc[MT][4];  // [row tile m][column tile n: 0, 1 gate; 2, 3 up]
        const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < 4; ++n) acc[m][n] = zero;
        // weight fragments of the k-block; activation fragments of the current
        // row tile and the next two (each read two row tiles ahead of its
        // MFMAs: one row tile of MFMAs is shorter than an LDS read under load)
        v8i bfr[4], acur, anx1, anx2;
#pragma unroll
        for (int n = 0; n < 4; ++n) bfr[n] = frag(smem + C::A_BYTES, brow(n));
        acur = frag(smem, wm * 128 + r);
        anx1 = frag(smem, wm * 128 + 16 + r);
        scales(smem, 0);

        // The k-loop is straight-line code: the copies of the last two
        // k-blocks repeat k-block HB-1 into regions no wave reads again, and
        // the fragments and scales read for "k-block HB" are never used.
#pragma unroll 1
        for (int kb = 0; kb < HB; ++kb) {
            const int cur = kb & 1;
            uint8_t* const sc = smem + cur * C::STAGE;        // this k-block's stage
            uint8_t* const sn = smem + (cur ^ 1) * C::STAGE;  // the next one's
            const int kb1 = min(kb + 1, HB - 1), kb2 = min(kb + 2, HB - 1);
            // scale-and-accumulate of MFMA result x (row tile tm, column tile tn)
            auto fma4 = [&](const v4f& x, int tm, int tn) __attribute__((always_inline)) {
                const float u = tn < 2 ? ug[tm] : uu[tm];
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[tm][tn][v] += x[v] * u;
            };
            // The compiler would sink the MFMAs and FMAs below the barriers
            // (they touch no memory) and hoist all fragment reads to the top,
            // keeping every fragment live at once: empty asm statements naming
            // the accumulators pin the arithmetic before each barrier, and a
            // compiler-only memory fence per row tile keeps each activation
            // fragment read in its row tile.
            auto pin_rows = [&](int m0, int m1) __attribute__((always_inline)) {
#pragma unroll
                for (int m = m0; m < m1; ++m)
                    asm volatile("" : "+v"(acc[m][0]), "+v"(acc[m][1]), "+v"(acc[m][2]), "+v"(acc[m][3]));
            };
            v4f pr[NTT];
#pragma unroll
            for (int t = 0; t < NTT; ++t) {
                const int m = t >> 2, n = t & 3;
                if (n == 0) asm volatile("" ::: "memory");
                if (t == 4) {  // barrier X: weight fragments of kb are in registers everywhere
                    pin_rows(MT - 2, MT);
                    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    issue_b(cur, kb2);
                }
                if (t == TY) {  // barrier Y: k-block kb+1 has landed; activations of kb all read
                    pin_rows(0, MT - 2);
                    asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    issue_a(cur, kb2);
                }
                // activation fragments two row tiles ahead: rows of kb while
                // m < MT - 2; the first two row tiles of kb+1 once it has landed
                if (n == 0 && m < MT - 2) anx2 = frag(sc, wm * 128 + 16 * (m + 2) + r);
                if (t == TY) anx1 = frag(sn, wm * 128 + r);
                if (t == TY + 1) anx2 = frag(sn, wm * 128 + 16 + r);
                pr[t] = mfma_f8_16x16x128(bfr[n], acur, zero);
                if (m == MT - 1) bfr[n] = frag(sn + C::A_BYTES, brow(n));
                if (n == 3) {  // the next row tile's fragment becomes current
                    acur = anx1;
                    anx1 = anx2;
                }
                if (t >= 4) fma4(pr[t - 4], (t - 4) >> 2, (t - 4) & 3);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int n = 0; n < 4; ++n) fma4(pr[NTT - 4 + n], MT - 1, n);
            scales(sn, kb1);
        }
        wait_vmem();  // no copy into LDS may be pending when the workgroup ends

#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int row = wm * 128 + m * 16 + r;
            if (row < nrows) {
#pragma unroll
                for (int n = 0; n < 2; ++n) {
                    uint32_t w[2], wl[2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float v0 = silu(acc[m][n + 2][2 * h]) * acc[m][n][2 * h];
                        const float v1 = silu(acc[m][n + 2][2 * h + 1]) * acc[m][n][2 * h + 1];
                        const uint16_t h0 = f2bf(v0), h1 = f2bf(v1);
                        w[h] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                        wl[h] = (uint32_t)f2bf(v0 - bf2f(h0)) | ((uint32_t)f2bf(v1 - bf2f(h1)) << 16);
                    }
                    const size_t idx = (size_t)(row0 + row) * I + jb + wn * 32 + n * 16 + 4 * g;
                    *reinterpret_cast<uint2*>(p.act + idx) = make_uint2(w[0], w[1]);
                    if (p.act_lo) *reinterpret_cast<uint2*>(p.act_lo + idx) = make_uint2(wl[0], wl[1]);
                }
            }
        }
    };
    if (nrows - wm * 128 > 64)
        compute(IntC<8>{});
    else
        compute(IntC<4>{});
}

hipError_t launch_gemm1_tile(const Plan& p, const uint8_t* hs, const float* hs_scale,
                             const uint8_t* w1, const float* w1s, int variant, hipStream_t s) {
    if (variant == 19) {
        const int tiles = max_mtiles(p.T, G1W::BM) * G1W::NT;
        hipLaunchKernelGGL((gemm1_tile_w_kernel<16>), dim3((tiles + 7) / 8 * 8), dim3(G1W::THREADS), 0,
                           s, p, hs, hs_scale, w1, w1s);
    } else if (variant == 18) {
        using C = G1Tile<4, 2>;
        const int tiles = max_mtiles(p.T, C::BM) * C::NT;
        hipLaunchKernelGGL((gemm1_tile_t_kernel<4, 2, 16>), dim3((tiles + 7) / 8 * 8),
                           dim3(C::THREADS), 0, s, p, hs, hs_scale, w1, w1s);
    } else if (variant == 3) {
        using C = G1Tile<4, 2>;
        const int tiles = max_mtiles(p.T, C::BM) * C::NT;
        dim3 grid((tiles + 7) / 8 * 8);
        hipLaunchKernelGGL((gemm1_tile_kernel<4, 2, 16>), grid, dim3(C::THREADS), 0, s, p, hs,
                           hs_scale, w1, w1s);
    } else {
        using C = G1Tile<2, 2>;
        const int tiles = max_mtiles(p.T, C::BM) * C::NT;
        dim3 grid((tiles + 7) / 8 * 8);
        hipLaunchKernelGGL((gemm1_tile_kernel<2, 2, 4>), grid, dim3(C::THREADS), 0, s, p, hs,
                           hs_scale, w1, w1s);
    }
    return hipGetLastError();
}

}  // namespace mimoe
