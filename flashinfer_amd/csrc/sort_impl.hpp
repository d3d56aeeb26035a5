// One-wave pieces of the local-expert sort, shared by the sort kernels and by
// the decode GEMM1 kernel that derives its own row tile from the top-k ids.
//
// Slot order (solution/triton/kernel.py:460-516 groups a shard's slots by
// local expert; here the order inside an expert is token-ascending, which
// makes it deterministic): slot = expert_off[e] + rank of the token among the
// tokens that picked local expert e.
#pragma once

#include "common.hpp"

namespace mimoe {

// Largest T the one-wave sort takes (lane t = token t).
constexpr int SMALL_T = 64;

// A token's local experts: bit mask over the EL local ids, and per top-k
// position the local id (-1 if not local) and routing weight.
struct TokLocal {
    emask_t m;
    int lid[TOPK];
    float lw[TOPK];
};

__device__ __forceinline__ TokLocal make_local(const int ids[TOPK], const float ws[TOPK], int off) {
    TokLocal r;
    r.m = 0;
#pragma unroll
    for (int k = 0; k < TOPK; ++k) {
        const int l = ids[k] - off;
        const bool loc = (unsigned)l < (unsigned)EL;
        r.lid[k] = loc ? l : -1;
        r.lw[k] = ws[k];
        r.m |= loc ? ebit(l) : (emask_t)0;
    }
    return r;
}

__device__ __forceinline__ TokLocal load_local(const int* ids_base, const float* w_base, int t,
                                               bool valid, int off) {
    int ids[TOPK];
    float ws[TOPK];
    if (valid) {
        load_topk_ids(ids_base + (size_t)t * TOPK_LD, ids);
        load_topk_w(w_base + (size_t)t * TOPK_LD, ws);
    } else {
#pragma unroll
        for (int k = 0; k < TOPK; ++k) { ids[k] = -1 - EL; ws[k] = 0.f; }  // never local
    }
    return make_local(ids, ws, valid ? off : 0);
}

// Exclusive prefix of the per-expert slot counts held by lanes 0..EL-1 of the
// calling wave (every lane of the wave must call). Optionally writes the
// expert offsets and the row-tile prefixes for GEMM tiles of bm1 / bm2 rows.
__device__ __forceinline__ int scan_counts(const Plan& p, int lane, int c, int bm1, int bm2,
                                           bool write) {
    const int bm3 = p.g1_alt_bm > 0 ? p.g1_alt_bm : bm1;
    int v0 = c, v1 = (c + bm1 - 1) / bm1, v2 = (c + bm2 - 1) / bm2, v3 = (c + bm3 - 1) / bm3;
    const int own0 = v0, own1 = v1, own2 = v2, own3 = v3;
#pragma unroll
    for (int d = 1; d < EL; d <<= 1) {
        const int u0 = __shfl_up(v0, d), u1 = __shfl_up(v1, d), u2 = __shfl_up(v2, d),
                  u3 = __shfl_up(v3, d);
        if (lane >= d) { v0 += u0; v1 += u1; v2 += u2; v3 += u3; }
    }
    // Device-side GEMM1 choice (uniform: g1_alt_bm is a launch argument):
    // the alternative tile when the bm1-row tiling has at least
    // G1_SELECT_EXTRA_TILES more row tiles than active experts.
    int alt = 0;
    if (p.g1_alt_bm > 0) {
        const int active = __popcll(__ballot(lane < EL && c > 0));
        const int t1 = __shfl(v1, EL - 1);
        alt = t1 - active >= G1_SELECT_EXTRA_TILES ? 1 : 0;
    }
    if (write && lane < EL) {
        p.meta[META_EXPERT_OFF + lane] = v0 - own0;
        p.meta[META_MTILE1 + lane] = v1 - own1;
        p.meta[META_MTILE2 + lane] = v2 - own2;
        if (p.g1_alt_bm > 0) p.meta[META_MTILE1B + lane] = v3 - own3;
        if (lane == EL - 1) {
            p.meta[META_EXPERT_OFF + EL] = v0;
            p.meta[META_MTILE2 + EL] = v2;
            // the table of the kernel not chosen holds no tiles
            p.meta[META_MTILE1 + EL] = alt ? 0 : v1;
            if (p.g1_alt_bm > 0) {
                p.meta[META_MTILE1B + EL] = alt ? v3 : 0;
                p.meta[META_G1_SEL] = alt;
            }
        }
    }
    return v0 - own0;
}

// Exclusive prefix sum over the lanes of the wave of x in [0, 2^BITS): one
// ballot per bit plane, counted below the lane with mbcnt (no LDS traffic).
template <int BITS = 7>
__device__ __forceinline__ int excl_prefix_small(int x) {
    int s = 0;
#pragma unroll
    for (int k = 0; k < BITS; ++k) {
        const unsigned long long b = __ballot((x >> k) & 1);
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(
            (uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        s += (int)below << k;
    }
    return s;
}

// T <= 64: one wave holds every token (lane t = token t). The expert counts
// are popcounts of 32 ballots, the offsets bit-plane prefixes and the
// placement a second round of ballots: no LDS and no barrier. Writes expert_off, both
// row-tile prefixes, sorted_tok, sorted_w and tok_slot. UNROLL sets how far
// the two 32-expert loops unroll: fully in the sort kernels, not at all
// inside a GEMM kernel, where 32 ballots in flight would spill scalar
// registers into the GEMM's vector registers.
template <int UNROLL = EL>
__device__ inline void sort_one_wave(const Plan& p, const int* ids_base, const float* w_base,
                                     int bm1, int bm2, int lane) {
    const bool valid = lane < p.T;
    const TokLocal tl = load_local(ids_base, w_base, lane, valid, p.local_offset);
    int cnt = 0;
#pragma unroll UNROLL
    for (int e = 0; e < EL; ++e) {
        const unsigned long long bal = __ballot((tl.m >> e) & 1u);
        if (lane == e) cnt = __popcll(bal);
    }
    // offsets and both row-tile prefixes (counts <= 64: bit-plane prefixes)
    const int t1 = (cnt + bm1 - 1) / bm1, t2 = (cnt + bm2 - 1) / bm2;
    const int off = excl_prefix_small(cnt);
    const int o1 = excl_prefix_small(t1), o2 = excl_prefix_small(t2);
    if (lane < EL) {
        p.meta[META_EXPERT_OFF + lane] = off;
        p.meta[META_MTILE1 + lane] = o1;
        p.meta[META_MTILE2 + lane] = o2;
        if (lane == EL - 1) {
            p.meta[META_EXPERT_OFF + EL] = off + cnt;
            p.meta[META_MTILE1 + EL] = o1 + t1;
            p.meta[META_MTILE2 + EL] = o2 + t2;
        }
    }
    const unsigned long long lower = (1ull << lane) - 1ull;
    int j = 0;
#pragma unroll UNROLL
    for (int e = 0; e < EL; ++e) {
        const bool hit = (tl.m >> e) & 1;
        const unsigned long long bal = __ballot(hit);
        const int base = __builtin_amdgcn_readlane(off, e);
        if (hit) {
            const int pos = base + __popcll(bal & lower);
            float w = 0.f;
#pragma unroll
            for (int k = 0; k < TOPK; ++k) w = (tl.lid[k] == e) ? tl.lw[k] : w;
            p.sorted_tok[pos] = lane;
            p.sorted_w[pos] = w;
            p.tok_slot[(size_t)lane * TOPK_LD + j] = pos;
            ++j;
        }
    }
    if (valid)
        for (; j < TOPK_LD; ++j) p.tok_slot[(size_t)lane * TOPK_LD + j] = -1;
}

// Writes the slots of one chunk given wcnt[wave][e] = first slot of expert e
// for the wave's tokens (every thread of the workgroup calls it). Lane e
// keeps expert e's token ballot and first slot; each token then walks its
// own (at most 8) local experts in top-k order and fetches those with lane
// shuffles, so no LDS read or weight search sits inside a per-expert loop.
// A slot's place in the token's list is the number of its local experts
// below it (ascending local expert order).
__device__ __forceinline__ void place_with_prefix(const Plan& p, int t, bool valid,
                                                  const TokLocal& tl, int (*wcnt)[EL], int lane,
                                                  int wave) {
    uint32_t bal_lo = 0, bal_hi = 0;
#pragma unroll
    for (int e = 0; e < EL; ++e) {
        const unsigned long long bal = __ballot((tl.m >> e) & 1);
        if (lane == e) { bal_lo = (uint32_t)bal; bal_hi = (uint32_t)(bal >> 32); }
    }
    const int base_e = wcnt[wave][lane & (EL - 1)];
    const uint32_t lower_lo = lane >= 32 ? 0xffffffffu : (1u << lane) - 1u;
    const uint32_t lower_hi = lane >= 32 ? (1u << (lane - 32)) - 1u : 0u;
#pragma unroll
    for (int k = 0; k < TOPK; ++k) {
        const int l = tl.lid[k];
        const int src = l < 0 ? 0 : l;
        const uint32_t blo = (uint32_t)__shfl((int)bal_lo, src);
        const uint32_t bhi = (uint32_t)__shfl((int)bal_hi, src);
        const int base = __shfl(base_e, src);
        if (l >= 0) {
            const int pos = base + __popc(blo & lower_lo) + __popc(bhi & lower_hi);
            const int j = epopc(tl.m & (ebit(l) - 1));
            p.sorted_tok[pos] = t;
            p.sorted_w[pos] = tl.lw[k];
            p.tok_slot[(size_t)t * TOPK_LD + j] = pos;
        }
    }
    if (valid)
        for (int j = epopc(tl.m); j < TOPK_LD; ++j) p.tok_slot[(size_t)t * TOPK_LD + j] = -1;
}

// Position of the k-th set bit (k counted from 0) of a 64-bit mask; k must be
// below the mask's popcount. Binary search over halves with popcounts.
__device__ __forceinline__ int nth_set_bit(unsigned long long mask, int k) {
    int pos = 0;
#pragma unroll
    for (int step = 32; step > 0; step >>= 1) {
        const unsigned long long seg = (mask >> pos) & ((1ull << step) - 1ull);
        const int c = __popcll(seg);
        if (k >= c) { k -= c; pos += step; }
    }
    return pos;
}

// Row tiles of bm rows in the slot order of sort_one_wave, for kernels that
// find their row tiles from the top-k ids alone (T <= 64): every wave builds
// the table in its registers (wave_table: the one-wave sort's counts and
// scans; lane t holds token t's local-expert mask, lane e < EL expert e's
// slot count, exclusive slot prefix and inclusive row-tile prefix) and reads
// a tile's entry with readlanes (table_tile).
struct WaveTable {
    emask_t m;     // lane t: local experts of token t
    int cnt, s0;   // lane e: slots of expert e, exclusive prefix (expert_off[e])
    int v1;        // lane e: inclusive prefix of the row tiles
};

// ids_base: [T, TOPK_LD], global or LDS. Every lane of the wave calls. Up to
// SMALL_TABLE_T tokens the expert counts come from the tokens' masks read
// with readlane instead of one ballot per local expert.
constexpr int SMALL_TABLE_T = 4;
__device__ __forceinline__ WaveTable wave_table(const Plan& p, const int* ids_base, int lane, int bm) {
    WaveTable w;
    w.m = 0;
    if (lane < p.T) {
        int ids[TOPK];
        load_topk_ids(ids_base + (size_t)lane * TOPK_LD, ids);
#pragma unroll
        for (int k = 0; k < TOPK; ++k) {
            const int l = ids[k] - p.local_offset;
            w.m |= (unsigned)l < (unsigned)EL ? ebit(l) : (emask_t)0;
        }
    }
    int cnt = 0;
    if (p.T <= SMALL_TABLE_T) {
        // a few tokens: lane e counts expert e's bit in each token's mask
#pragma unroll
        for (int t = 0; t < SMALL_TABLE_T; ++t) {
            emask_t mt;
            if constexpr (EL > 32) {
                const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)w.m, t);
                const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(w.m >> 32), t);
                mt = ((emask_t)hi << 32) | lo;
            } else {
                mt = (emask_t)__builtin_amdgcn_readlane((uint32_t)w.m, t);
            }
            cnt += (t < p.T && lane < EL) ? (int)((mt >> (lane & (EL - 1))) & 1) : 0;
        }
    } else {
#pragma unroll
        for (int e = 0; e < EL; ++e) {
            const unsigned long long bal = __ballot((w.m >> e) & 1);
            if (lane == e) cnt = __popcll(bal);
        }
    }
    const int tiles = (cnt + bm - 1) / bm;
    w.cnt = cnt;
    w.s0 = excl_prefix_small(cnt);
    w.v1 = excl_prefix_small(tiles) + tiles;
    return w;
}

__device__ __forceinline__ int table_tiles(const WaveTable& w) {
    return __builtin_amdgcn_readlane(w.v1, EL - 1);
}

// Row tile mt (0 <= mt < table_tiles) of the table: expert e, first slot
// row0 = expert_off[e] + rank0, rows, and the mask of tokens (bit t = token
// t) that picked e.
struct WaveTile {
    int e, row0, nrows, rank0;
    unsigned long long hits;
};

__device__ __forceinline__ WaveTile table_tile(const WaveTable& w, int lane, int mt, int bm) {
    // experts wholly before tile mt
    const int ee = __popcll(__ballot(lane < EL && w.v1 <= mt));
    const int ce = __builtin_amdgcn_readlane(w.cnt, ee);
    const int t0 = __builtin_amdgcn_readlane(w.v1, ee) - (ce + bm - 1) / bm;
    WaveTile t;
    t.e = ee;
    t.rank0 = (mt - t0) * bm;
    t.row0 = __builtin_amdgcn_readlane(w.s0, ee) + t.rank0;
    t.nrows = min(bm, ce - t.rank0);
    t.hits = __ballot((w.m >> ee) & 1);
    return t;
}

}  // namespace mimoe
