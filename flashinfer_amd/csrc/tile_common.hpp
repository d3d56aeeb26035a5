// Helpers shared by the LDS-tiled GEMM kernels (prefill shapes).
#pragma once

#include "common.hpp"

namespace mimoe {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(size_t)(lds_ptr_t)p;
}

// 16-byte global -> LDS copy: lane l's 16 bytes land at lds_base + 16 * l
// (lds_base must be wave-uniform; gfx950 global_load_lds_dwordx4).
//
// Written as inline asm on purpose: the compiler cannot tell that a copy into
// one LDS stage does not alias reads of the other stage, and would put a
// vmcnt(0) wait in front of every LDS read, serialising copy and compute.
// The kernels using these place their own vmcnt waits before each barrier.
// One wait state between the M0 write and the LDS DMA is required.
__device__ __forceinline__ void g2l16(const void* gsrc, void* lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gsrc), "s"(lds_addr(lds_base))
                 : "memory", "m0");
}

// 4-byte global -> LDS copy: lane l's dword lands at lds_base + 4 * l.
__device__ __forceinline__ void g2l4(const void* gsrc, void* lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(gsrc), "s"(lds_addr(lds_base))
                 : "memory", "m0");
}

// The same two copies with a wave-uniform 64-bit base in SGPRs and a 32-bit
// per-lane byte offset (the saddr form: address = sbase + voff): one VGPR per
// copy instead of a 64-bit address per lane.
__device__ __forceinline__ void g2l16s(const void* sbase, uint32_t voff, void* lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_addr(lds_base))
                 : "memory", "m0");
}

__device__ __forceinline__ void g2l4s(const void* sbase, uint32_t voff, void* lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_addr(lds_base))
                 : "memory", "m0");
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// XOR swizzle of the 16-byte chunk index inside a 128-byte LDS row: 16
// consecutive rows reading the same logical chunk hit 16 distinct 16-byte
// bank groups (conflict-free for 32- and 64-bank LDS).
__device__ __forceinline__ int swz8(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// Swizzle of a 128-byte row whose reads are also conflict-free when 32 lanes
// (16 rows x two adjacent chunks) are serviced together: for the four rows
// r, r+4, r+8, r+12 that share a bank group the values differ in their upper
// two bits, so chunks c and c^1 of those rows land on 8 distinct positions;
// 16 rows at one chunk still take 16 distinct bank groups. A copy of 8 rows
// x 8 chunks still reads each row's 128 bytes whole.
__device__ __forceinline__ int swzq(int row) { return (((row >> 2) & 3) << 1) | ((row >> 1) & 1); }

// Same for a 256-byte row of 16 chunks.
__device__ __forceinline__ int swz16(int row) { return row & 15; }

__device__ __forceinline__ v4i lds16(const uint8_t* p) { return *reinterpret_cast<const v4i*>(p); }

// Logical tile order shared by the tiled GEMMs. Tiles of one expert are
// visited in groups of GM row tiles; inside a group every n tile is swept
// with the GM row tiles innermost, so the tiles running at the same time
// on one XCD share weight and activation tiles in that XCD's L2. Each XCD
// (workgroup b runs on XCD b % 8) takes one contiguous eighth of the order.
// tile_at returns the coordinates of logical tile t < total.
template <int NT, int GM>
__device__ __forceinline__ void tile_at(const int* meta, int mtile_base, int bm, int t, int& e,
                                        int& row0, int& nrows, int& nt) {
    const int mt = t / NT;  // NT tiles per row tile: find the expert by row-tile index
    int ee = 0;
#pragma unroll
    for (int k = 0; k < EL; ++k) ee += (meta[mtile_base + k + 1] <= mt) ? 1 : 0;
    e = ee;
    const int mt0 = meta[mtile_base + ee];
    const int mts = meta[mtile_base + ee + 1] - mt0;  // row tiles of this expert
    const int u = t - mt0 * NT;                        // tile index inside the expert
    const int grp = u / (GM * NT);
    const int gm = min(GM, mts - grp * GM);            // row tiles in this group
    const int v = u - grp * GM * NT;
    nt = v / gm;
    const int mtl = grp * GM + (v - nt * gm);
    row0 = meta[META_EXPERT_OFF + ee] + mtl * bm;
    nrows = min(bm, meta[META_EXPERT_OFF + ee + 1] - row0);
}

// The tile of workgroup blockIdx.x in a grid of one workgroup per tile.
template <int NT, int GM>
__device__ __forceinline__ bool tile_coords(const int* meta, int mtile_base, int bm, int& e,
                                            int& row0, int& nrows, int& nt) {
    const int total = meta[mtile_base + EL] * NT;
    const int per_xcd = (total + 7) >> 3;
    const int b = blockIdx.x;
    const int idx = b >> 3;
    if (idx >= per_xcd) return false;
    const int t = (b & 7) * per_xcd + idx;
    if (t >= total) return false;
    tile_at<NT, GM>(meta, mtile_base, bm, t, e, row0, nrows, nt);
    return true;
}

}  // namespace mimoe
