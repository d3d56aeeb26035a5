// Shared constants, device helpers and the launch plan of the fused MoE.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mimoe {

// Definition of the layer (solution/triton/kernel.py:615-625 hard-codes
// H=7168, I=2048, 256 experts in 8 groups, top-4 groups, top-8, 32 local
// experts; its routing kernel takes them as constexpr parameters,
// kernel.py:371-389). Each library build fixes them at compile time:
// -DMI_MOE_HIDDEN / -DMI_MOE_INTER / -DMI_MOE_E_LOCAL / -DMI_MOE_E_GLOBAL /
// -DMI_MOE_N_GROUP / -DMI_MOE_TOPK_GROUP / -DMI_MOE_TOP_K. The scale blocks
// stay 128 elements.
#ifndef MI_MOE_HIDDEN
#define MI_MOE_HIDDEN 7168
#endif
#ifndef MI_MOE_INTER
#define MI_MOE_INTER 2048
#endif
#ifndef MI_MOE_E_LOCAL
#define MI_MOE_E_LOCAL 32
#endif
#ifndef MI_MOE_E_GLOBAL
#define MI_MOE_E_GLOBAL 256
#endif
#ifndef MI_MOE_N_GROUP
#define MI_MOE_N_GROUP 8
#endif
#ifndef MI_MOE_TOPK_GROUP
#define MI_MOE_TOPK_GROUP 4
#endif
#ifndef MI_MOE_TOP_K
#define MI_MOE_TOP_K 8
#endif
constexpr int H = MI_MOE_HIDDEN;  // hidden size
constexpr int I = MI_MOE_INTER;   // intermediate size
// combine: 1024-column chunks; GEMM1 K split over 4 waves of 2-deep rings:
// 8 | H/128. GEMM2 rings at least 2 deep, tiles of 128 columns: 2 | I/128.
static_assert(H % 1024 == 0 && I % 256 == 0, "supported shapes: H % 1024 == 0, I % 256 == 0");
constexpr int N1 = 2 * I;                // GEMM1 output width (gate | up)
constexpr int EG = MI_MOE_E_GLOBAL;      // global experts
constexpr int EL = MI_MOE_E_LOCAL;       // local experts per shard
constexpr int TOPK = MI_MOE_TOP_K;       // experts per token
constexpr int NGROUP = MI_MOE_N_GROUP;   // routing groups
constexpr int KGROUP = MI_MOE_TOPK_GROUP;  // groups a token may pick from
constexpr int GSIZE = EG / NGROUP;       // experts per group
// Routing: one wave64 per token, lane l owns experts EPL*l .. EPL*l+EPL-1;
// a group is LPG adjacent lanes, reduced by DPP exchanges within 16 lanes.
constexpr int EPL = EG / 64;
constexpr int LPG = GSIZE / (EPL > 0 ? EPL : 1);
static_assert(EG % 64 == 0 && EG <= 256, "global experts: 64, 128, 192 or 256");
static_assert(EG % NGROUP == 0 && GSIZE % EPL == 0, "groups of whole lanes");
static_assert(LPG == 2 || LPG == 4 || LPG == 8 || LPG == 16, "2 to 16 lanes per routing group");
static_assert(KGROUP >= 1 && KGROUP <= NGROUP, "topk_group within the groups");
static_assert(TOPK >= 1 && TOPK <= 8 && TOPK <= KGROUP * GSIZE, "top-k of 1..8 from the kept groups");
// Local experts: one lane (and one ballot bit plane) per expert.
static_assert(EL == 16 || EL == 32 || EL == 64, "16, 32 or 64 local experts");
// Row stride of the per-token top-k tables and slot lists in the workspace:
// always 8, entries past TOPK are padding, so every kernel loads a token's
// row as two 16-byte vectors.
constexpr int TOPK_LD = 8;
// Bit mask over the local experts.
typedef __typeof__(EL > 32 ? 0ull : 0u) emask_t;
__device__ __forceinline__ emask_t ebit(int l) { return (emask_t)1 << l; }
__device__ __forceinline__ int epopc(emask_t m) {
    if constexpr (EL > 32) return __popcll(m); else return __popc((uint32_t)m);
}
// The LDS-tiled GEMMs address weight rows of the shard with 32-bit signed
// offsets ((e * N1 + row) * H for W1, (e * H + row) * I for W2).
static_assert((long long)EL * N1 * H < (1LL << 31), "gemm1_weights of the shard exceed 2^31 bytes");
static_assert((long long)EL * H * I < (1LL << 31), "gemm2_weights of the shard exceed 2^31 bytes");
constexpr int BLK = 128;            // scale block
constexpr int HB = H / BLK;         // k-blocks of GEMM1 (56 at H=7168)
constexpr int IB = I / BLK;         // k-blocks of GEMM2 (16 at I=2048)
constexpr int N1B = N1 / BLK;       // n-blocks of GEMM1 (32 at I=2048)

// Device pointers into the caller's workspace plus the call's scalars.
struct Plan {
    int T;
    int local_offset;          // clamped into int range by the host
    float rsf;
    int* topk_ids;             // [T, TOPK_LD]
    float* topk_w;             // [T, TOPK_LD]
    int* meta;                 // expert_off[EL+1] | mtile_off1[EL+1] | mtile_off2[EL+1]
    int* sorted_tok;           // [TOPK*T]
    float* sorted_w;           // [TOPK*T]
    int* tok_slot;             // [T, TOPK_LD]
    int* chunk_cnt;            // [ceil(T/1024), EL] per-chunk expert totals (large-T sort)
    uint16_t* act;             // bf16 [TOPK*T, I]
    uint16_t* part;            // bf16 [TOPK*T, H]: routing weight x GEMM2 row of each slot
    // part_f32 (the same bytes as part), when set: GEMM2 writes the weighted
    // rows in fp32 there and the combine sums those, as the reference's
    // fp32 partials (kernel.py:364-368).
    float* part_f32;           // fp32 [TOPK*T, H] or null
    // act_lo (only with part_f32), when set: GEMM1 also writes
    // bf16(x - bf16(x)) of each SwiGLU value x there, and GEMM2 multiplies
    // act + act_lo, 16 mantissa bits (the reference's fp32 -> TF32 operand
    // keeps 10, kernel.py:272-278).
    uint16_t* act_lo;          // bf16 [TOPK*T, I] or null
    // GEMM1 kernel chosen on the device from the expert counts (0: off). When
    // set, the sort also writes the row-tile prefix for tiles of g1_alt_bm rows
    // (META_MTILE1B) and zeroes the total of the table it does not choose, so
    // of the two GEMM1 launches only the chosen one finds tiles.
    int g1_alt_bm;
    int g1_mtile;              // META_MTILE1 or META_MTILE1B: the LDS-tile GEMM1's row-tile table
};

// What a GEMM2 kernel reads and writes (template argument, picked per call).
constexpr int G2_BF16 = 0;   // act; bf16 rows to part
constexpr int G2_F32 = 1;    // act; fp32 rows to part_f32
constexpr int G2_SPLIT = 2;  // act + act_lo; fp32 rows to part_f32
inline int gemm2_mode(const Plan& p) {
    return p.act_lo ? G2_SPLIT : (p.part_f32 ? G2_F32 : G2_BF16);
}

constexpr int META_STRIDE = EL < 64 ? 64 : 128;  // holds EL + 1 entries
constexpr int META_EXPERT_OFF = 0;
constexpr int META_MTILE1 = META_STRIDE;
constexpr int META_MTILE2 = 2 * META_STRIDE;
constexpr int META_MTILE1B = 3 * META_STRIDE;  // GEMM1 row tiles of g1_alt_bm rows
constexpr int META_G1_SEL = 4 * META_STRIDE;   // 1: the alternative GEMM1 tile was chosen
constexpr int META_INTS = 4 * META_STRIDE + 64;

// Device-side GEMM1 choice (Plan::g1_alt_bm): the LDS tile of g1_alt_bm rows
// runs instead of the 64-row wide kernel when the 64-row tiling would stream
// at least this many expert weight sets beyond one per active expert (sum_e
// ceil(c_e / 64) - active experts). Measured on 24 batches of T = 384 ...
// 1536 at four shard offsets (per call, one process, three alternating
// passes): thresholds of 11 and 12 came within 23.6 us in total of the
// better kernel on every batch, against 218 us for the wide kernel alone.
constexpr int G1_SELECT_EXTRA_TILES = 11;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f2bf(float f) {
    __bf16 b = (__bf16)f;  // round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950)
    return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ float bf2f(uint16_t u) {
    return __builtin_bit_cast(float, (uint32_t)u << 16);
}

// 16x16x128 fp8(e4m3) x fp8(e4m3) -> fp32, unit block scales (E8M0 127 = 2^0).
__device__ __forceinline__ v4f mfma_f8_16x16x128(v8i a, v8i b, v4f c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

__device__ __forceinline__ v4f mfma_bf16_16x16x32(v8bf a, v8bf b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Two fp8 e4m3 values (low or high 16 bits of w) -> two bf16, exact.
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
    v2bf r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI);
    return __builtin_bit_cast(uint32_t, r);
}

// Eight fp8 (two dwords) -> eight bf16 (four dwords), exact.
__device__ __forceinline__ v4i fp8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
    v4i r;
    r.x = (int)fp8x2_to_bf16x2<false>(w0);
    r.y = (int)fp8x2_to_bf16x2<true>(w0);
    r.z = (int)fp8x2_to_bf16x2<false>(w1);
    r.w = (int)fp8x2_to_bf16x2<true>(w1);
    return r;
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

// One SwiGLU value into act (bf16, round to nearest even) and, for the
// exact-input GEMM2, the remainder into act_lo.
__device__ __forceinline__ void store_act(const Plan& p, size_t idx, float v) {
    const uint16_t hi = f2bf(v);
    p.act[idx] = hi;
    if (p.act_lo) p.act_lo[idx] = f2bf(v - bf2f(hi));
}


__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Loads 16 bytes through the vector memory path.
__device__ __forceinline__ v4i ld16(const void* p) { return *reinterpret_cast<const v4i*>(p); }

// Weight operand of one 16-row x 128-byte k-block, read as whole lines.
// Lane l (n = l % 16, q = l / 16) loads 16 bytes at wl_off from row n % 8
// (x) and from row 8 + n % 8 (y), bytes [32q + 16(n / 8), +16): each load
// instruction covers 8 complete 128-byte lines, which non-temporal loads
// stream from HBM about 15% faster than the 16 half lines of a row-per-lane
// layout (measured on MI355X: 7.1 against 6.2 TB/s plain, and 5.7 TB/s for
// half lines with the non-temporal hint). Rotating each 16-lane row by 8
// (DPP; lanes 8-15 take y of lane n - 8, lanes 0-7 x of lane n + 8) leaves
// lane l with row n, bytes [32q, 32q + 32): the MFMA operand in its own k
// order, which the activation side reads with ld_afrag (fp8) or as 32
// consecutive bf16.
__device__ __forceinline__ size_t wl_off(int lane, size_t row_stride) {
    return (size_t)(lane & 7) * row_stride + (lane >> 4) * 32 + ((lane >> 3) & 1) * 16;
}

// Buffer resource over `bytes` bytes at a uniform `base`: raw buffer loads
// through it are range-checked (an offset past the end reads 0) and carry
// their cache policy as an immediate.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wrsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// The two loads of a weight k-block (off = row base + wl_off, stride8 = 8
// rows), kept raw in a prefetch ring: the exchange (wl_frag) runs where the
// operand is consumed, so the loads stay in flight until then.
// NT: non-temporal loads. They stream weights that no other row tile of the
// launch reads again ~12 % faster; where several row tiles of an expert
// re-read its weights, plain loads keep them in L2 / MALL for the others
// (with the hint each tile fetched them from HBM again: T=1024 with up to 8
// row tiles per expert, GEMM1 564 against 475 us). The policy is a template
// argument: per workgroup from its expert's row count in the wide GEMM1 and
// the stream GEMM2 (two copies of the k loop, BoolC below); per launch from
// T (wt_nt) in the stream GEMM1, whose two-copy form took 69 -> 96 VGPRs
// (108 without the sort folded in), and in the GEMM2 + combine kernel.
struct WRaw {
    v4i x, y;
};
template <bool NT>
__device__ __forceinline__ WRaw ld_wraw(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t stride8) {
    constexpr int AUX = NT ? 2 : 0;  // cache policy: nt
    WRaw w;
    w.x = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX));
    w.y = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off + stride8), 0, AUX));
    return w;
}

// Weight load policy of a launch with T tokens and `bm`-row tiles: non-
// temporal while an expert holds about one row tile or less on average
// (T * top_k <= bm * global experts / 4: T <= 128 for 16-row tiles, 512 for
// 64-row tiles with the default routing; a shard's experts can hold twice
// the uniform share, as at T = 1024 offset 0). Measured per GEMM with random
// routing at T = 16 / 64 / 100 / 256 / 512: 9-12 % faster with the hint;
// with every token on the same 8 experts (T = 64 / 256: 4 row tiles each)
// 5-7 % slower, the price of not knowing the counts on the host.
inline bool wt_nt(int64_t T, int bm) { return T * TOPK <= (int64_t)bm * EG / 4; }

// Compile-time bool for `body(BoolC<NT>{})`: a kernel whose register budget
// allows it runs one of two copies of its k loop per workgroup, picking the
// load policy from its expert's row count.
template <bool B>
struct BoolC {
    static constexpr bool value = B;
};
template <int V>
struct IntC {
    static constexpr int value = V;
};

__device__ __forceinline__ v8i wl_frag(const WRaw& w) {
    constexpr int ROR8 = 0x128;  // DPP row_ror:8
    v8i r;
    r.s0 = __builtin_amdgcn_update_dpp(w.x.x, w.y.x, ROR8, 0xF, 0xC, false);
    r.s1 = __builtin_amdgcn_update_dpp(w.x.y, w.y.y, ROR8, 0xF, 0xC, false);
    r.s2 = __builtin_amdgcn_update_dpp(w.x.z, w.y.z, ROR8, 0xF, 0xC, false);
    r.s3 = __builtin_amdgcn_update_dpp(w.x.w, w.y.w, ROR8, 0xF, 0xC, false);
    r.s4 = __builtin_amdgcn_update_dpp(w.y.x, w.x.x, ROR8, 0xF, 0x3, false);
    r.s5 = __builtin_amdgcn_update_dpp(w.y.y, w.x.y, ROR8, 0xF, 0x3, false);
    r.s6 = __builtin_amdgcn_update_dpp(w.y.z, w.x.z, ROR8, 0xF, 0x3, false);
    r.s7 = __builtin_amdgcn_update_dpp(w.y.w, w.x.w, ROR8, 0xF, 0x3, false);
    return r;
}

// The fp8 activation operand matching wl_frag: bytes [32q, 32q + 32) of the
// k-block (p = row + k-block + 32q).
__device__ __forceinline__ v8i ld_afrag(const uint8_t* p) {
    const v4i lo = ld16(p);
    const v4i hi = ld16(p + 16);
    v8i r;
    r.s0 = lo.x; r.s1 = lo.y; r.s2 = lo.z; r.s3 = lo.w;
    r.s4 = hi.x; r.s5 = hi.y; r.s6 = hi.z; r.s7 = hi.w;
    return r;
}

// A token's top-k row in a TOPK_LD-strided table (workspace or LDS, 16-byte
// aligned): stored as two 16-byte vectors, entries past TOPK as id -1,
// weight 0; loaded the same way, keeping the first TOPK.
__device__ __forceinline__ void store_topk_row(int* ids_row, float* w_row, const int ids[TOPK],
                                               const float w[TOPK]) {
    int iv[TOPK_LD];
    float wv[TOPK_LD];
#pragma unroll
    for (int k = 0; k < TOPK_LD; ++k) {
        iv[k] = k < TOPK ? ids[k < TOPK ? k : 0] : -1;
        wv[k] = k < TOPK ? w[k < TOPK ? k : 0] : 0.f;
    }
    reinterpret_cast<int4*>(ids_row)[0] = make_int4(iv[0], iv[1], iv[2], iv[3]);
    reinterpret_cast<int4*>(ids_row)[1] = make_int4(iv[4], iv[5], iv[6], iv[7]);
    reinterpret_cast<float4*>(w_row)[0] = make_float4(wv[0], wv[1], wv[2], wv[3]);
    reinterpret_cast<float4*>(w_row)[1] = make_float4(wv[4], wv[5], wv[6], wv[7]);
}

__device__ __forceinline__ void load_topk_ids(const int* ids_row, int ids[TOPK]) {
    const int4 i0 = reinterpret_cast<const int4*>(ids_row)[0];
    const int4 i1 = reinterpret_cast<const int4*>(ids_row)[1];
    const int iv[TOPK_LD] = {i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w};
#pragma unroll
    for (int k = 0; k < TOPK; ++k) ids[k] = iv[k];
}

__device__ __forceinline__ void load_topk_w(const float* w_row, float w[TOPK]) {
    const float4 w0 = reinterpret_cast<const float4*>(w_row)[0];
    const float4 w1 = reinterpret_cast<const float4*>(w_row)[1];
    const float wv[TOPK_LD] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int k = 0; k < TOPK; ++k) w[k] = wv[k];
}

// Locate the expert and first row of row tile `mt` (prefix table in meta).
__device__ __forceinline__ bool find_tile(const int* meta, int mtile_base, int mt, int bm, int& e,
                                          int& row0, int& nrows) {
    const int total = meta[mtile_base + EL];
    if (mt >= total) return false;
    int ee = 0;
#pragma unroll
    for (int k = 0; k < EL; ++k) ee += (meta[mtile_base + k + 1] <= mt) ? 1 : 0;
    e = ee;
    row0 = meta[META_EXPERT_OFF + ee] + (mt - meta[mtile_base + ee]) * bm;
    nrows = min(bm, meta[META_EXPERT_OFF + ee + 1] - row0);
    return true;
}

// Upper bound on the row tiles of all experts: sum_e ceil(c_e / bm) with
// sum_e c_e <= TOPK*T, c_e <= T and at most min(EL, TOPK*T) experts holding
// slots (each adds under one tile of rounding).
inline int max_mtiles(int T, int bm) {
    const long long st = (long long)TOPK * T;
    const long long a = (st + bm - 1) / bm + (st < EL ? st : EL);
    const long long b = (long long)EL * ((T + bm - 1) / bm);
    return (int)(a < b ? a : b);
}

// Host-side launchers (one per kernel family); return hipError_t of the launch.
// packed: rows of TOPK entries (the public routing entry point), else the
// workspace's TOPK_LD-wide rows.
hipError_t launch_route(const float* logits, const void* bias, int bias_is_f32, int T, float rsf,
                        int* topk_ids, float* topk_w, hipStream_t s, bool packed = false);
hipError_t launch_sort(const Plan& p, int bm1, int bm2, hipStream_t s);
// [T, TOPK] top-k rows -> TOPK_LD-wide rows (padding: id -1, weight 0).
hipError_t launch_repack_topk(const int* ids, const float* w, int T, int* out_ids, float* out_w,
                              hipStream_t s);
// Routing + sort in one single-workgroup launch (small T only).
bool route_sort_supported(int T);
// Tokens per chunk of the large-T sort (one 1024-thread workgroup each).
constexpr int SORT_CHUNK = 1024;
#ifndef MI_MOE_SORT_CHUNK_L
#define MI_MOE_SORT_CHUNK_L 256
#endif
// Tokens per workgroup of the two-pass sort above T = SORT_CHUNK. Chunks of
// 256 keep more CUs placing than chunks of 1024 (place pass, measured by
// kernel trace on MI355X: T=2048 6.0 against 10.0 us, T=8192 7.6 against
// 11.1, T=14000 8.1 against 12.1; 512-token chunks in between; the count
// pass stays at 4.6 us).
constexpr int SORT_CHUNK_L = MI_MOE_SORT_CHUNK_L;
static_assert(SORT_CHUNK_L % 64 == 0 && SORT_CHUNK_L <= SORT_CHUNK && SORT_CHUNK_L >= EL,
              "large-T sort chunk: whole waves, at most one workgroup, a thread per expert");
constexpr int sort_chunks(int T) { return (T + SORT_CHUNK_L - 1) / SORT_CHUNK_L; }
hipError_t launch_route_sort(const Plan& p, const float* logits, const void* bias, int bias_is_f32,
                             int bm1, int bm2, hipStream_t s);
hipError_t launch_gemm1(const Plan& p, const uint8_t* hs, const float* hs_scale, const uint8_t* w1,
                        const float* w1s, int variant, hipStream_t s);
// Front-end work a GEMM1 stream kernel can do itself at decode sizes: none
// (it reads the sort's tables), the sort (from the top-k ids in the
// workspace), or routing and the sort (from the logits).
constexpr int FRONT_NONE = 0;
constexpr int FRONT_SORT = 1;
constexpr int FRONT_ROUTE = 2;
struct FrontArgs {
    const float* logits;  // [T, 256] (FRONT_ROUTE)
    const void* bias;     // [256] bf16 or fp32 (FRONT_ROUTE)
    int bias_is_f32;
    int bm1, bm2;         // row-tile heights of the GEMM1 / GEMM2 kernels for the tables
};
// GEMM1 stream variants 16 and 5 with FRONT_SORT or FRONT_ROUTE (T <= 64),
// and the wide variant 15 with FRONT_SORT (T <= 256): they find their row
// tiles themselves and write the sort's tables (and, with FRONT_ROUTE, the
// top-k) for the kernels after them, so no sort (or routing) launch precedes
// them.
bool gemm1_sorts_supported(int T, int variant);
bool gemm1_routes_supported(int T, int variant);
bool gemm1_wide_sorts_supported(int T);
hipError_t launch_gemm1_wide_sorting(const Plan& p, const uint8_t* hs, const float* hs_scale,
                                     const uint8_t* w1, const float* w1s, int bm2, hipStream_t s);
hipError_t launch_gemm1_front(const Plan& p, const uint8_t* hs, const float* hs_scale,
                              const uint8_t* w1, const float* w1s, int variant, int front,
                              const FrontArgs& fa, hipStream_t s);
hipError_t launch_gemm2(const Plan& p, const uint8_t* w2, const float* w2s, int variant,
                        hipStream_t s);
hipError_t launch_combine(const Plan& p, uint16_t* out, hipStream_t s);
hipError_t launch_quant_fp8(const void* x, int T, uint8_t* q, float* scale, hipStream_t s);
// The quantiser and the routing kernel's work in one launch.
hipError_t launch_quant_route(const void* x, int T, uint8_t* q, float* scale, const float* logits,
                              const void* bias, int bias_is_f32, float rsf, int* topk_ids,
                              float* topk_w, hipStream_t s);
bool gemm2_combine_supported(int T);
// The same with the 16 k-blocks split over the 4 waves (every wave runs every
// row tile): more waves in flight when there are fewer than 4 row tiles.
hipError_t launch_gemm2_combine_ks(const Plan& p, const uint8_t* w2, const float* w2s,
                                   uint16_t* out, hipStream_t s);
hipError_t launch_gemm2_combine(const Plan& p, const uint8_t* w2, const float* w2s, uint16_t* out,
                                hipStream_t s);
hipError_t launch_gemm1_tile(const Plan& p, const uint8_t* hs, const float* hs_scale,
                             const uint8_t* w1, const float* w1s, int variant, hipStream_t s);
hipError_t launch_gemm2_tile(const Plan& p, const uint8_t* w2, const float* w2s, int variant,
                             hipStream_t s);
hipError_t launch_gemm1_wide(const Plan& p, const uint8_t* hs, const float* hs_scale,
                             const uint8_t* w1, const float* w1s, hipStream_t s);
hipError_t launch_gemm2_wide(const Plan& p, const uint8_t* w2, const float* w2s, hipStream_t s);

// GEMM kernel variants: 0/1/2 weight-streaming with 16/32/64-row tiles and
// 4-wave workgroups, 3 LDS-tiled large (GEMM1 256 rows, GEMM2 128 rows),
// 4 LDS-tiled medium (GEMM1 128 rows, GEMM2 64 rows), 5..14 weight-streaming
// shapes with 1-, 2-, 4- or 8-wave workgroups and 16/32/64 columns per wave
// (see the launchers), 10 GEMM2 fused with the combine, 15 "wide" tiles
// (64 rows for GEMM1, 32 for GEMM2; weights through a per-wave register
// ring, activations through LDS) for medium row counts, 16 streaming with K
// split over 4 waves of a workgroup (and, for GEMM2, 9: the same with 64
// columns per wave), 17 GEMM2 fused with the combine
// with K split over its 4 waves, 18 the GEMM1 LDS tile of variant 3 with the MFMA
// operands swapped (one scale factor per lane and tile) and the scale FMAs
// software-pipelined behind later MFMAs (for GEMM2, the tile of variant 3),
// 19 the GEMM1 LDS tile whose waves hold a k-block's weight fragments in
// registers so that each weight copy has two k-blocks to arrive.
// An id without a kernel of its own in one GEMM (9, 10 and 17 for GEMM1, 19
// for GEMM2) runs that GEMM's default stream shape.
constexpr int NUM_VARIANTS = 22;
// GEMM2 variants that also perform the combine (decode sizes only): tiles
// dealt to the 4 waves, or k-blocks split over them.
constexpr int VARIANT_GEMM2_COMBINE = 10;
constexpr int VARIANT_GEMM2_COMBINE_KS = 17;

// Row-tile height of each GEMM variant (rows of one expert per workgroup).
int gemm1_bm(int variant);
int gemm2_bm(int variant);
// Workgroups of the tile kernels that walk their tiles one workgroup per CU:
// the current device's CU count (a multiple of its 8 XCDs).
int persistent_grid();

}  // namespace mimoe
