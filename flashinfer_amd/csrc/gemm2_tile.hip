// Grouped GEMM2 (down projection), LDS-tiled variant for many rows per expert.
//
// Same contract as gemm2_stream_kernel (solution/triton/kernel.py:193-293):
//   part[s, n] = bf16(w_s * sum_kb sb2[e, n/128, kb] * (act[s, kb-block] . W2[e, n, kb-block]))
// with bf16 activations and fp8 weights widened to bf16 (exact).
//
// A workgroup of WM x WN waves computes BM = 64*WM rows x BN = 64*WN output
// columns. Per 128-wide k-block the BM activation rows (256 B each, bf16) and
// the BN fp8 weight rows (128 B each) are copied global -> LDS with
// global_load_lds_dwordx4 into one of two stages (copy of kb+1 overlaps the
// MFMAs on kb). Each wave owns 64 x 64 outputs: for each 16-column weight
// fragment it converts 32 fp8 -> bf16 once and feeds four 16-row fragments,
// four v_mfma_f32_16x16x32_bf16 per 128-k block, then scales the block's
// partial sum by sb2 in fp32.
//
// Operand k order (identical for A and B, so the pairing is exact): lane
// (r = l%16, g = l/16) holds k-block offsets 16g+[0,16) and 64+16g+[0,16);
// MFMA h uses offsets 16g+8h (h<2) and 64+16g+8(h-2) (h>=2).
// LDS: weight rows are 128 B with swz8; activation rows are 256 B (16
// chunks) with chunk c at position c ^ (row & 15).
#include <algorithm>
#include <atomic>

#include "tile_common.hpp"

namespace mimoe {

template <int WM, int WN>
struct G2Tile {
    static constexpr int NW = WM * WN;
    static constexpr int THREADS = 64 * NW;
    static constexpr int BM = 64 * WM;
    static constexpr int BN = 64 * WN;
    static constexpr int NT = H / BN;
    static constexpr int A_BYTES = BM * BLK * 2;
    static constexpr int B_BYTES = BN * BLK;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int A_LD = A_BYTES / 1024 / NW;
    static constexpr int B_LD = B_BYTES / 1024 / NW;
    static_assert(H % BN == 0, "n tiles");
    static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "loader split");
    static_assert(2 * STAGE <= 160 * 1024, "LDS budget");
};

template <int WM, int WN, int GM, int MODE>
__global__ __launch_bounds__(64 * WM * WN) void gemm2_tile_kernel(Plan p,
                                                                  const uint8_t* __restrict__ w2,
                                                                  const float* __restrict__ w2s) {
    using C = G2Tile<WM, WN>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE];
    __shared__ float w_lds[C::THREADS];  // routing weights of the tile's rows (first BM used)

    int e, row0, nrows, nt;
    if (!tile_coords<C::NT, GM>(p.meta, META_MTILE2, C::BM, e, row0, nrows, nt)) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = nt * C::BN;

    // Activation loader: a 1 KB copy covers 4 rows of 256 B; lane l takes
    // row +l/16, chunk position l%16.
    const uint8_t* act = reinterpret_cast<const uint8_t*>(p.act);
    uint32_t a_off[C::A_LD], b_off[C::B_LD];
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) {
        const int row = 4 * (wave * C::A_LD + i) + (lane >> 4);
        const int c = (lane & 15) ^ swz16(row);
        a_off[i] = (uint32_t)(row0 + min(row, nrows - 1)) * (I * 2) + c * 16;
    }
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) {
        const int row = 8 * (wave * C::B_LD + i) + (lane >> 3);
        const int c = (lane & 7) ^ swz8(row);
        b_off[i] = (uint32_t)((e * H + n0 + row) * I + c * 16);
    }

    // Copies whose 4 rows all lie past the expert's last row are skipped
    // (wave-uniform): those LDS rows only feed output rows that are never
    // stored.
    auto issue = [&](int stage, int kb) __attribute__((always_inline)) {
        uint8_t* s = smem + stage * C::STAGE;
#pragma unroll
        for (int i = 0; i < C::A_LD; ++i)
            if (4 * (wave * C::A_LD + i) < nrows)
                g2l16(act + (size_t)a_off[i] + kb * (BLK * 2), s + (wave * C::A_LD + i) * 1024);
#pragma unroll
        for (int i = 0; i < C::B_LD; ++i)
            g2l16(w2 + b_off[i] + kb * BLK, s + C::A_BYTES + (wave * C::B_LD + i) * 1024);
    };

    const int wm = wave % WM, wn = wave / WM;
    const int r = lane & 15, g = lane >> 4;
    const float* sb_p = w2s + ((size_t)e * HB + (n0 + wn * 64) / BLK) * IB;

    v4f acc[4][4];
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[m][n] = zero;

    // Routing weights go to LDS with the first stage (one wait for both), so
    // the epilogue does not wait on a load per row.
    const float w_row = p.sorted_w[row0 + min(tid, nrows - 1)];
    issue(0, 0);
    wait_vmem();
    w_lds[tid] = w_row;
    __syncthreads();

#pragma unroll 1
    for (int kb = 0; kb < IB; ++kb) {
        const int cur = kb & 1;
        if (kb + 1 < IB) issue(cur ^ 1, kb + 1);
        // Waves whose 64 rows lie past the expert's last row only copy
        // (wave-uniform branch).
        if (wm * 64 >= nrows) {
            wait_vmem();
            __syncthreads();
            continue;
        }
        const uint8_t* sA = smem + cur * C::STAGE;
        const uint8_t* sB = sA + C::A_BYTES;
        const float sb = sb_p[kb];

        v4i a[4][4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int row = wm * 64 + m * 16 + r;
            const uint8_t* base = sA + row * (BLK * 2);
            const int sw = swz16(row);
            a[m][0] = lds16(base + (((2 * g) ^ sw) << 4));
            a[m][1] = lds16(base + (((2 * g + 1) ^ sw) << 4));
            a[m][2] = lds16(base + (((8 + 2 * g) ^ sw) << 4));
            a[m][3] = lds16(base + (((9 + 2 * g) ^ sw) << 4));
        }
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const int brow = wn * 64 + n * 16 + r;
            const uint8_t* base = sB + brow * BLK;
            const int sw = swz8(brow);
            const v4i lo = lds16(base + ((g ^ sw) << 4));
            const v4i hi = lds16(base + (((g + 4) ^ sw) << 4));
            const v4i b0 = fp8x8_to_bf16x8((uint32_t)lo.x, (uint32_t)lo.y);
            const v4i b1 = fp8x8_to_bf16x8((uint32_t)lo.z, (uint32_t)lo.w);
            const v4i b2 = fp8x8_to_bf16x8((uint32_t)hi.x, (uint32_t)hi.y);
            const v4i b3 = fp8x8_to_bf16x8((uint32_t)hi.z, (uint32_t)hi.w);
            // the four row tiles' k-chains interleaved: consecutive MFMAs are
            // independent, then one scale-and-accumulate per row tile
            v4f pr[4] = {zero, zero, zero, zero};
#pragma unroll
            for (int m = 0; m < 4; ++m)
                pr[m] = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a[m][0]), __builtin_bit_cast(v8bf, b0), pr[m]);
#pragma unroll
            for (int m = 0; m < 4; ++m)
                pr[m] = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a[m][1]), __builtin_bit_cast(v8bf, b1), pr[m]);
#pragma unroll
            for (int m = 0; m < 4; ++m)
                pr[m] = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a[m][2]), __builtin_bit_cast(v8bf, b2), pr[m]);
#pragma unroll
            for (int m = 0; m < 4; ++m)
                pr[m] = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, a[m][3]), __builtin_bit_cast(v8bf, b3), pr[m]);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                acc[m][n][0] += pr[m][0] * sb;
                acc[m][n][1] += pr[m][1] * sb;
                acc[m][n][2] += pr[m][2] * sb;
                acc[m][n][3] += pr[m][3] * sb;
            }
        }
        wait_vmem();
        __syncthreads();
    }

    // Epilogue: routing weight (kernel.py:364) and a bf16 (MODE G2_BF16) or
    // fp32 (G2_F32) row for the combine.
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = wm * 64 + m * 16 + g * 4 + i;
            if (row < nrows) {
                const float w = w_lds[row];
                const size_t o = (size_t)(row0 + row) * H + n0 + wn * 64 + r;
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    if constexpr (MODE == G2_F32)
                        p.part_f32[o + n * 16] = w * acc[m][n][i];
                    else
                        p.part[o + n * 16] = f2bf(w * acc[m][n][i]);
                }
            }
        }
    }
}


// The 128 x 256 tile of variant 3 as one software pipeline (variant 20), in
// the manner of GEMM1's variant 19. Wave (wm, wn) owns rows 64wm .. 64wm+63
// (4 row tiles of 16) and columns 64wn .. 64wn+63 (4 column tiles). It keeps
// the k-block's weight fragments, widened to bf16, in registers (64 VGPRs)
// and streams its activation fragments from LDS one row tile ahead. The two
// barriers of a k-block sit inside the MFMA stream:
//   * barrier X after row tile 0: every wave holds its weight fragments of
//     k-block kb, so that stage's weight region takes the copy of k-block
//     kb+2 (~1.75 k-blocks to land);
//   * barrier Y before row tile 3: the copies of kb+1 have landed (vmcnt
//     leaves only kb+2's weight copies outstanding) and the activation rows of
//     kb are all read, so the activation region takes kb+2's rows. During row
//     tile 3 each wave reads kb+1's raw weight fragments and first
//     activation fragment; the weights are widened at their first use.
// Per unit (row tile m, column tile n) the four MFMAs of the 128-k block
// chain from zero and the block scale is applied in fp32 one unit later, the
// arithmetic of variant 3 (bitwise equal). The routing weights and the
// tile's weight scales go to LDS by DMA, so no load of the compiler's own is
// pending inside the loop.
//
// PERSIST (variant 21): one workgroup per CU walks the tiles slot, slot +
// CPX, ... of its XCD's eighth of the tile order (CPX = workgroups per XCD),
// and the copy pipeline runs on across tiles: k-steps IB-2 and IB-1 copy the
// next tile's k-blocks 0 and 1 (and its routing weights and scales, into the
// other half of two LDS buffers), so the next tile's first copies are in
// flight during this tile's last MFMAs and its epilogue, instead of starting
// after a new workgroup is placed and has found its tile.
template <int GM, int MODE, bool PERSIST>
__global__ __launch_bounds__(512) void gemm2_tile_w_kernel(Plan p, const uint8_t* __restrict__ w2,
                                                           const float* __restrict__ w2s) {
    using C = G2Tile<2, 4>;
    static_assert(C::A_LD == 4 && C::B_LD == 4, "vmcnt(4) leaves one k-block of weight copies");
    static_assert(IB <= 32, "scales: one lane per k-block and 128-column block");
    static_assert(IB % 2 == 0, "every tile starts on stage 0");
    constexpr int NBUF = PERSIST ? 2 : 1;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE];
    __shared__ __attribute__((aligned(16))) float w_lds[NBUF][C::BM];  // routing weights of the rows
    __shared__ __attribute__((aligned(16))) float s_sb[NBUF][2][32];   // [128-column block][kb] weight scales

    int e, row0, nrows, nt;
    int t = 0, t_end = 0, t_step = 0;
    if constexpr (PERSIST) {
        const int total = p.meta[META_MTILE2 + EL] * C::NT;
        const int per_xcd = (total + 7) >> 3;
        const int t0 = (blockIdx.x & 7) * per_xcd;
        t_step = gridDim.x >> 3;
        t = t0 + (blockIdx.x >> 3);
        t_end = min(total, t0 + per_xcd);
        if (t >= t_end) return;
        tile_at<C::NT, GM>(p.meta, META_MTILE2, C::BM, t, e, row0, nrows, nt);
    } else {
        if (!tile_coords<C::NT, GM>(p.meta, META_MTILE2, C::BM, e, row0, nrows, nt)) return;
    }
    e = __builtin_amdgcn_readfirstlane(e);
    nt = __builtin_amdgcn_readfirstlane(nt);
    row0 = __builtin_amdgcn_readfirstlane(row0);
    nrows = __builtin_amdgcn_readfirstlane(nrows);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // per-lane copy offsets of a tile (activation rows of its slots, weight
    // rows of its expert and 256 columns)
    auto a_offset = [&](int i, int row0_, int nrows_) __attribute__((always_inline)) {
        const int row = 4 * (wave * C::A_LD + i) + (lane >> 4);
        const int c = (lane & 15) ^ swz16(row);
        return (uint32_t)(row0_ + min(row, nrows_ - 1)) * (I * 2) + c * 16;
    };
    auto b_offset = [&](int i, int e_, int nt_) __attribute__((always_inline)) {
        const int row = 8 * (wave * C::B_LD + i) + (lane >> 3);
        const int c = (lane & 7) ^ swz8(row);
        return (uint32_t)((e_ * H + nt_ * C::BN + row) * I + c * 16);
    };
    uint32_t a_off[C::A_LD], b_off[C::B_LD];
#pragma unroll
    for (int i = 0; i < C::A_LD; ++i) a_off[i] = a_offset(i, row0, nrows);
#pragma unroll
    for (int i = 0; i < C::B_LD; ++i) b_off[i] = b_offset(i, e, nt);
    const uint8_t* act = reinterpret_cast<const uint8_t*>(p.act);
    auto issue_a = [&](int stage, int kb, const uint32_t* off) __attribute__((always_inline)) {
        uint8_t* s = smem + stage * C::STAGE;
        const uint8_t* base = act + (size_t)kb * (BLK * 2);
#pragma unroll
        for (int i = 0; i < C::A_LD; ++i) g2l16s(base, off[i], s + (wave * C::A_LD + i) * 1024);
    };
    auto issue_b = [&](int stage, int kb, const uint32_t* off) __attribute__((always_inline)) {
        uint8_t* s = smem + stage * C::STAGE + C::A_BYTES;
        const uint8_t* base = w2 + kb * BLK;
#pragma unroll
        for (int i = 0; i < C::B_LD; ++i) g2l16s(base, off[i], s + (wave * C::B_LD + i) * 1024);
    };
    // DMA of a tile's constants: the routing weights of its rows (waves 0,
    // 1) and the weight scales of its two 128-column blocks (wave 2).
    auto consts = [&](int buf, int e_, int row0_, int nrows_, int nt_) __attribute__((always_inline)) {
        buf = __builtin_amdgcn_readfirstlane(buf);  // the LDS base goes to M0
        if (wave < 2) {
            const int row = wave * 64 + lane;
            g2l4s(p.sorted_w, (uint32_t)(row0_ + min(row, nrows_ - 1)) * 4, &w_lds[buf][wave * 64]);
        } else if (wave == 2) {
            // lane l -> s_sb[l / 32][l % 32] (k-blocks past IB repeat the last)
            const int half = lane >> 5, kb = lane & 31;
            const uint32_t off =
                (uint32_t)((((size_t)e_ * HB + nt_ * C::BN / BLK + half) * IB + min(kb, IB - 1)) * 4);
            g2l4s(w2s, off, &s_sb[buf][0][0]);
        }
    };

    // Prologue copies in the order of the steady state: the tile's
    // constants, weights and activations of k-block 0, weights of 1; then
    // (after the barrier that plays barrier Y of k-block -1) activations of 1.
    consts(0, e, row0, nrows, nt);
    issue_b(0, 0, b_off);
    issue_a(0, 0, a_off);
    issue_b(1, 1, b_off);
    asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
    issue_a(1, 1, a_off);

    const int wm = wave & 1, wn = wave >> 1;
    const int r = lane & 15, g = lane >> 4;
    const int sbcol = (wn * 64) / BLK;  // this wave's 128-column block of the tile

    // activation fragment of row tile m (4 x 16 B: k offsets 16g+[0,16) and
    // 64+16g+[0,16) in bf16 pairs, as variant 3 reads them)
    auto afrag = [&](const uint8_t* s, int m, v4i (&a)[4]) __attribute__((always_inline)) {
        const int row = wm * 64 + m * 16 + r;
        const uint8_t* base = s + row * (BLK * 2);
        const int sw = swz16(row);
        a[0] = lds16(base + (((2 * g) ^ sw) << 4));
        a[1] = lds16(base + (((2 * g + 1) ^ sw) << 4));
        a[2] = lds16(base + (((8 + 2 * g) ^ sw) << 4));
        a[3] = lds16(base + (((9 + 2 * g) ^ sw) << 4));
    };
    // raw weight fragment of column tile n (16 B at chunk g and at g + 4)
    auto braw = [&](const uint8_t* s, int n, v4i& lo, v4i& hi) __attribute__((always_inline)) {
        const int brow = wn * 64 + n * 16 + r;
        const uint8_t* base = s + C::A_BYTES + brow * BLK;
        const int sw = swz8(brow);
        lo = lds16(base + ((g ^ sw) << 4));
        hi = lds16(base + (((g + 4) ^ sw) << 4));
    };
    auto widen = [&](const v4i& lo, const v4i& hi, v4i (&b)[4]) __attribute__((always_inline)) {
        b[0] = fp8x8_to_bf16x8((uint32_t)lo.x, (uint32_t)lo.y);
        b[1] = fp8x8_to_bf16x8((uint32_t)lo.z, (uint32_t)lo.w);
        b[2] = fp8x8_to_bf16x8((uint32_t)hi.x, (uint32_t)hi.y);
        b[3] = fp8x8_to_bf16x8((uint32_t)hi.z, (uint32_t)hi.w);
    };
    const v4f zero = {0.f, 0.f, 0.f, 0.f};

    int buf = 0;
    for (;;) {
        // the next tile of this workgroup, if any
        bool has_next = false;
        int en = 0, row0n = 0, nrowsn = 1, ntn = 0;
        if constexpr (PERSIST) {
            has_next = t + t_step < t_end;
            if (has_next) {
                tile_at<C::NT, GM>(p.meta, META_MTILE2, C::BM, t + t_step, en, row0n, nrowsn, ntn);
                en = __builtin_amdgcn_readfirstlane(en);
                row0n = __builtin_amdgcn_readfirstlane(row0n);
                nrowsn = __builtin_amdgcn_readfirstlane(nrowsn);
                ntn = __builtin_amdgcn_readfirstlane(ntn);
            }
        }
        // The copies of k-step kb: at barrier X the weights of step kb + 2,
        // at barrier Y its activations. Step kb + 2 is k-block kb + 2 of this
        // tile, k-block kb + 2 - IB of the next one, or (no next tile) a
        // repeat of the last k-block into a stage that is not read again.
        // The copy offsets switch to the next tile at step IB - 2, after
        // their last use for this one.
        auto kb_copy = [&](int kb) __attribute__((always_inline)) {
            return (PERSIST && has_next) ? (kb + 2 < IB ? kb + 2 : kb + 2 - IB) : min(kb + 2, IB - 1);
        };
        auto copy_x = [&](int stage, int kb) __attribute__((always_inline)) {
            if (PERSIST && has_next && kb + 2 == IB) {
                consts(buf ^ 1, en, row0n, nrowsn, ntn);
#pragma unroll
                for (int i = 0; i < C::B_LD; ++i) b_off[i] = b_offset(i, en, ntn);
            }
            issue_b(stage, kb_copy(kb), b_off);
        };
        auto copy_y = [&](int stage, int kb) __attribute__((always_inline)) {
            if (PERSIST && has_next && kb + 2 == IB) {
#pragma unroll
                for (int i = 0; i < C::A_LD; ++i) a_off[i] = a_offset(i, row0n, nrowsn);
            }
            issue_a(stage, kb_copy(kb), a_off);
        };

        if (wm * 64 >= nrows) {
            // Rows past the expert (wave-uniform): copies and barriers only, in
            // step with the other waves (two barriers per k-block).
#pragma unroll 1
            for (int kb = 0; kb < IB; ++kb) {
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                copy_x(kb & 1, kb);
                asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                copy_y(kb & 1, kb);
            }
        } else {
            v4f acc[4][4];
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int n = 0; n < 4; ++n) acc[m][n] = zero;

            // k-block 0: raw weight fragments, activation fragments of row tile 0
            v4i blo[4], bhi[4], bq[4][4], acur[4], anx[4];
#pragma unroll
            for (int n = 0; n < 4; ++n) braw(smem, n, blo[n], bhi[n]);
            afrag(smem, 0, acur);

#pragma unroll 1
            for (int kb = 0; kb < IB; ++kb) {
                const int cur = kb & 1;
                uint8_t* const sc = smem + cur * C::STAGE;
                uint8_t* const sn = smem + (cur ^ 1) * C::STAGE;
                const float sb = s_sb[buf][sbcol][kb];
                auto pin_rows = [&](int m0, int m1) __attribute__((always_inline)) {
#pragma unroll
                    for (int m = m0; m < m1; ++m)
                        asm volatile("" : "+v"(acc[m][0]), "+v"(acc[m][1]), "+v"(acc[m][2]), "+v"(acc[m][3]));
                };
                v4f pr[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const int m = u >> 2, n = u & 3;
                    if (n == 0) asm volatile("" ::: "memory");
                    if (u == 4) {  // barrier X: every wave holds its weight fragments of kb
                        pin_rows(2, 4);
                        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                        copy_x(cur, kb);
                    }
                    if (u == 12) {  // barrier Y: kb+1 has landed; activations of kb all read
                        pin_rows(0, 2);
                        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                        copy_y(cur, kb);
                    }
                    // next row tile's activation fragment (row tile 0 of kb+1 once it has landed)
                    if (n == 0 && m < 3) afrag(sc, m + 1, anx);
                    if (u == 12) afrag(sn, 0, anx);
                    if (m == 0) widen(blo[n], bhi[n], bq[n]);  // weights of kb, widened at their first use
                    v4f t4 = zero;
                    t4 = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, acur[0]), __builtin_bit_cast(v8bf, bq[n][0]), t4);
                    t4 = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, acur[1]), __builtin_bit_cast(v8bf, bq[n][1]), t4);
                    t4 = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, acur[2]), __builtin_bit_cast(v8bf, bq[n][2]), t4);
                    t4 = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, acur[3]), __builtin_bit_cast(v8bf, bq[n][3]), t4);
                    pr[u] = t4;
                    if (m == 3) braw(sn, n, blo[n], bhi[n]);  // raw weights of kb+1
                    if (n == 3) {
#pragma unroll
                        for (int h = 0; h < 4; ++h) acur[h] = anx[h];
                    }
                    if (u >= 1) {  // the previous unit's scale-and-accumulate
                        const int pm = (u - 1) >> 2, pn = (u - 1) & 3;
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[pm][pn][v] += pr[u - 1][v] * sb;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[3][3][v] += pr[15][v] * sb;
            }

            // Epilogue: routing weight (kernel.py:364) and a bf16 (MODE G2_BF16) or
            // fp32 (G2_F32) row for the combine, as variant 3 writes them.
            const int n0 = nt * C::BN;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = wm * 64 + m * 16 + g * 4 + i;
                    if (row < nrows) {
                        const float w = w_lds[buf][row];
                        const size_t o = (size_t)(row0 + row) * H + n0 + wn * 64 + r;
#pragma unroll
                        for (int n = 0; n < 4; ++n) {
                            if constexpr (MODE == G2_F32)
                                p.part_f32[o + n * 16] = w * acc[m][n][i];
                            else
                                p.part[o + n * 16] = f2bf(w * acc[m][n][i]);
                        }
                    }
                }
            }
        }
        if (!PERSIST || !has_next) break;
        t += t_step;  // the copy offsets are the next tile's already
        e = en;
        row0 = row0n;
        nrows = nrowsn;
        nt = ntn;
        buf ^= 1;
    }
    wait_vmem();  // no copy into LDS may be pending when the workgroup ends
}

int persistent_grid() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8)
            n = 256;
        n = n / 8 * 8;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

hipError_t launch_gemm2_tile(const Plan& p, const uint8_t* w2, const float* w2s, int variant,
                             hipStream_t s) {
    const bool f32 = gemm2_mode(p) != G2_BF16;
    if (variant == 20) {
        using C = G2Tile<2, 4>;
        const int tiles = max_mtiles(p.T, C::BM) * C::NT;
        dim3 grid((tiles + 7) / 8 * 8);
        if (f32)
            hipLaunchKernelGGL((gemm2_tile_w_kernel<4, G2_F32, false>), grid, dim3(C::THREADS), 0, s, p, w2, w2s);
        else
            hipLaunchKernelGGL((gemm2_tile_w_kernel<4, G2_BF16, false>), grid, dim3(C::THREADS), 0, s, p, w2, w2s);
    } else if (variant == 21) {
        using C = G2Tile<2, 4>;
        const int tiles = (max_mtiles(p.T, C::BM) * C::NT + 7) / 8 * 8;
        dim3 grid(std::min(tiles, persistent_grid()));
        if (f32)
            hipLaunchKernelGGL((gemm2_tile_w_kernel<4, G2_F32, true>), grid, dim3(C::THREADS), 0, s, p, w2, w2s);
        else
            hipLaunchKernelGGL((gemm2_tile_w_kernel<4, G2_BF16, true>), grid, dim3(C::THREADS), 0, s, p, w2, w2s);
    } else if (variant == 3 || variant == 18) {
        using C = G2Tile<2, 4>;
        const int tiles = max_mtiles(p.T, C::BM) * C::NT;
        dim3 grid((tiles + 7) / 8 * 8);
        if (f32)
            hipLaunchKernelGGL((gemm2_tile_kernel<2, 4, 4, G2_F32>), grid, dim3(C::THREADS), 0, s, p, w2, w2s);
        else
            hipLaunchKernelGGL((gemm2_tile_kernel<2, 4, 4, G2_BF16>), grid, dim3(C::THREADS), 0, s, p, w2, w2s);
    } else {
        using C = G2Tile<1, 4>;
        const int tiles = max_mtiles(p.T, C::BM) * C::NT;
        dim3 grid((tiles + 7) / 8 * 8);
        if (f32)
            hipLaunchKernelGGL((gemm2_tile_kernel<1, 4, 4, G2_F32>), grid, dim3(C::THREADS), 0, s, p, w2, w2s);
        else
            hipLaunchKernelGGL((gemm2_tile_kernel<1, 4, 4, G2_BF16>), grid, dim3(C::THREADS), 0, s, p, w2, w2s);
    }
    return hipGetLastError();
}

}  // namespace mimoe
