// extern "C" boundary of the fused MoE (declared in include/mi_moe.h).
//
// mi_moe_run replaces solution/triton/kernel.py::run (kernel.py:600-825).
// Every argument is checked before the first launch, so a bad call enqueues
// nothing and reports why through mi_moe_last_error(). The call enqueues
// route -> sort -> GEMM1+SwiGLU -> GEMM2 -> combine on the caller's stream
// with grids sized from T alone: no device-to-host copy, no host sync
// (the reference syncs three times, kernel.py:572, :718, :773). Routing and
// the sort fold into GEMM1 up to T = 4, the sort alone up to T = 512 (the
// stream GEMM1 kernels up to 64, the wide one above); see pick_front.
#include <dlfcn.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/mi_moe.h"
#include "common.hpp"

using namespace mimoe;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

// The LDS-tiled GEMMs address gathered rows with 32-bit byte offsets (token
// * H into hidden_states, slot * 2I into the bf16 activations, with at most
// 8 slots per token), so T is capped where those stay below 2^32.
constexpr int64_t kMaxTokens = MI_MOE_MAX_TOKENS;
static_assert((uint64_t)kMaxTokens * H <= (1ull << 32), "GEMM1 tile row offsets fit 32 bits");
static_assert((uint64_t)kMaxTokens * TOPK * I * 2 <= (1ull << 32), "GEMM2 tile row offsets fit 32 bits");

constexpr size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

// Largest T whose GEMM2 writes fp32 partial rows: the workspace reserves
// 4-byte partials for these T. Measured per call on MI355X against bf16 rows
// (same box, interleaved): under 1% up to T = 256, where weights stream from
// HBM; +2.4% at T = 1024 (combine reads twice the bytes); +4.0% at T = 8192
// and +7.9% at T = 14000 with every token on 8 experts, which keep bf16 rows.
#ifndef MI_MOE_F32_PART_MAX_T
#define MI_MOE_F32_PART_MAX_T 1024
#endif
constexpr int64_t F32_PART_MAX_T = MI_MOE_F32_PART_MAX_T;
// Largest T for which the workspace reserves act_lo (the split activation
// act + act_lo that MI_MOE_SPLIT_ACT=1 asks for; the LDS tiles have no split
// path, so it stops where they take over).
constexpr int64_t SPLIT_ACT_MAX_T = 256;
static_assert(SPLIT_ACT_MAX_T <= F32_PART_MAX_T, "the split activation writes fp32 rows");

constexpr mi_moe_layout make_layout(int64_t T) {
    mi_moe_layout L{};
    const size_t t = (size_t)(T < 0 ? 0 : T);
    const size_t s_max = (size_t)TOPK * t;  // local slots: at most TOPK per token
    size_t o = 0;
    L.topk_ids = o;   o = align_up(o + t * TOPK_LD * 4);
    L.topk_w = o;     o = align_up(o + t * TOPK_LD * 4);
    L.expert_off = o; o = align_up(o + META_INTS * 4);
    L.sorted_tok = o; o = align_up(o + s_max * 4);
    L.sorted_w = o;   o = align_up(o + s_max * 4);
    L.tok_slot = o;   o = align_up(o + t * TOPK_LD * 4);
    L.chunk_cnt = o;  o = align_up(o + (size_t)sort_chunks((int)t) * EL * 4);
    const bool f32 = (int64_t)t <= F32_PART_MAX_T;
    const bool split = (int64_t)t <= SPLIT_ACT_MAX_T;
    L.act = o;        o = align_up(o + s_max * I * 2);
    L.part = o;       o = align_up(o + s_max * H * (f32 ? 4 : 2));
    L.act_lo = o;     o = align_up(o + (split ? s_max * I * 2 : 0));
    L.total = o;
    return L;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Scratch of the no-allocation entry point (mi_moe_run_noalloc): the
// workspace of MI_MOE_NOALLOC_MAX_TOKENS tokens, one copy per GPU the library
// runs on, held until the process ends. Host code never passes `scratch`
// itself (on the host it names a stand-in, not device memory): it uses the
// device address hipGetSymbolAddress returns for the device in question.
constexpr size_t kScratchBytes = make_layout(MI_MOE_NOALLOC_MAX_TOKENS).total;
static_assert(kScratchBytes % 256 == 0, "scratch is a whole number of 256-byte blocks");
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the device `stream` belongs to, looked up
// once per device (with that device current) and kept.
int scratch_address(hipStream_t stream, void** out) {
    int dev = -1;
    hipError_t e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess)
        return fail(MI_MOE_ERR_HIP, "mi_moe_run_noalloc: hipStreamGetDevice failed: %s",
                    hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_run_noalloc: device %d beyond the %d supported",
                    dev, kMaxDevices);
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p) {
        *out = p;
        return MI_MOE_OK;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
        int cur = -1;
        e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != dev) {
            const hipError_t r = hipSetDevice(cur);
            if (e == hipSuccess) e = r;
        }
        if (e != hipSuccess || !p)
            return fail(MI_MOE_ERR_HIP, "mi_moe_run_noalloc: scratch address on device %d: %s",
                        dev, hipGetErrorString(e));
        g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return MI_MOE_OK;
}

// Device pointers of one call into the caller's workspace.
Plan make_plan(void* workspace, const mi_moe_layout& L, int64_t T, int64_t local_expert_offset,
               float rsf) {
    // Offsets outside [-2^30, 2^30] select no expert; clamp so int math stays exact.
    int64_t off = local_expert_offset;
    if (off > (1 << 30)) off = 1 << 30;
    if (off < -(1 << 30)) off = -(1 << 30);
    uint8_t* ws = (uint8_t*)workspace;
    Plan p;
    p.T = (int)T;
    p.local_offset = (int)off;
    p.rsf = rsf;
    p.topk_ids = (int*)(ws + L.topk_ids);
    p.topk_w = (float*)(ws + L.topk_w);
    p.meta = (int*)(ws + L.expert_off);
    p.sorted_tok = (int*)(ws + L.sorted_tok);
    p.sorted_w = (float*)(ws + L.sorted_w);
    p.tok_slot = (int*)(ws + L.tok_slot);
    p.chunk_cnt = (int*)(ws + L.chunk_cnt);
    p.act = (uint16_t*)(ws + L.act);
    p.part = (uint16_t*)(ws + L.part);
    p.part_f32 = nullptr;
    p.act_lo = nullptr;
    p.g1_alt_bm = 0;
    p.g1_mtile = META_MTILE1;
    return p;
}

// Named ranges for profilers, as the reference's _profile_region gives its
// phases (kernel.py:10-24, :678-823): with FIB_PROFILE_PHASES=1 in the
// environment at the first call, each phase's launches sit in a roctx range
// named as the reference names that phase (route + sort ->
// phase1_route_permute, GEMM1 with its SwiGLU -> phase3_gemm1, phase5_gemm2,
// the combine with its bf16 cast -> phase6_scatter), inside an "mi_moe_run"
// range, so `rocprofv3 --marker-trace` attributes the kernels. The roctx
// library is looked up at run time, so the operator does not link against it.
struct Roctx {
    int (*push)(const char*);
    int (*pop)();
};

const Roctx* roctx() {
    static const Roctx r = [] {
        Roctx x{nullptr, nullptr};
        const char* f = getenv("FIB_PROFILE_PHASES");
        if (!f || f[0] != '1' || f[1] != 0) return x;
        void* h = dlopen("librocprofiler-sdk-roctx.so.1", RTLD_NOW | RTLD_LOCAL);
        if (!h) h = dlopen("libroctx64.so.4", RTLD_NOW | RTLD_LOCAL);
        if (!h) return x;
        x.push = reinterpret_cast<int (*)(const char*)>(dlsym(h, "roctxRangePushA"));
        x.pop = reinterpret_cast<int (*)()>(dlsym(h, "roctxRangePop"));
        if (!x.push || !x.pop) x = Roctx{nullptr, nullptr};
        return x;
    }();
    return r.push ? &r : nullptr;
}

// GEMM variants by token count. MI_MOE_VARIANT="v" or "v1,v2" overrides
// (0..NUM_VARIANTS-1, for tests and tuning).
struct Variants {
    int g1, g2;
    int g1_alt = -1;  // >= 0: GEMM1 variant that the device may choose instead of g1
};

// Which launches do routing and the sort (decode sizes fold them into
// others). MI_MOE_FUSE_FRONT, MI_MOE_ROUTE_IN_GEMM1 and MI_MOE_SORT_IN_GEMM1
// (=0/1) override the defaults, in that order of precedence.
enum class Front {
    KERNELS,         // routing kernel, sort kernel(s)
    FUSED,           // one single-workgroup routing + sort kernel
    SORT_IN_GEMM1,   // routing kernel; GEMM1 sorts (FRONT_SORT)
    ROUTE_IN_GEMM1,  // GEMM1 routes and sorts (FRONT_ROUTE)
};

// Largest T whose routing every GEMM1 workgroup repeats by default. Each
// workgroup routes all T tokens (one per wave) before its first weight load;
// with 8 workgroup rows at T <= 4 that beats the routing launch it saves up
// to T = 4 (measured per call on MI355X: T=2 21.0 against 22.4 us, T=4 33.8
// against 35.5) and loses beyond (T=16 126.8 against 100.4).
constexpr int64_t ROUTE_IN_GEMM1_MAX_T = 4;

int env_flag(const char* name) {  // -1 unset, else 0 / 1
    const char* v = getenv(name);
    return (v && *v) ? (atoi(v) != 0) : -1;
}

// GEMM2's inputs and outputs (G2_*): fp32 partial rows up to F32_PART_MAX_T
// tokens (MI_MOE_F32_PARTIALS=0 turns them off); the split activation only
// up to SPLIT_ACT_MAX_T, with a kernel other than the LDS tiles, and when
// MI_MOE_SPLIT_ACT=1 asks for it (measured on MI355X it adds 5-9% at T = 1,
// 4, 64 and 256, 1.6% at T = 16: the second operand's loads and registers
// cost occupancy).
int gemm2_mode_for(int64_t T, int g2) {
    if (T > F32_PART_MAX_T) return G2_BF16;
    const bool tile = g2 == 3 || g2 == 4 || g2 == 18 || g2 == 20 || g2 == 21;
    if (!tile && T <= SPLIT_ACT_MAX_T && env_flag("MI_MOE_SPLIT_ACT") == 1) return G2_SPLIT;
    return env_flag("MI_MOE_F32_PARTIALS") == 0 ? G2_BF16 : G2_F32;
}

Front pick_front(int64_t T, int g1) {
    const int fuse = env_flag("MI_MOE_FUSE_FRONT");
    const int route = env_flag("MI_MOE_ROUTE_IN_GEMM1");
    const int sort = env_flag("MI_MOE_SORT_IN_GEMM1");
    const bool g1_can = gemm1_sorts_supported((int)T, g1);
    const bool fused_ok = route_sort_supported((int)T);
    if (fuse == 1 && fused_ok) return Front::FUSED;
    if (gemm1_routes_supported((int)T, g1) && (route == -1 ? T <= ROUTE_IN_GEMM1_MAX_T : route == 1))
        return Front::ROUTE_IN_GEMM1;
    // Routing as its own launch plus the sort inside the K-split GEMM1 beats
    // the fused routing + sort kernel from T = 2 when the shard has slots
    // (measured per call, four seeds at T = 3..4: 1.5-4 us; T = 5..8: 2-3 us;
    // 2.5 us slower only when no token is local), so the fused kernel runs
    // only when asked for.
    if (g1_can && sort != 0) return Front::SORT_IN_GEMM1;
    return Front::KERNELS;
}

// Layers smaller than 7168 x 2048 keep the stream kernels (K-split GEMM1,
// 64-column GEMM2 waves) while T * top_k <= 8 * global experts (about 8 slots
// per local expert), at 7168 x 2048 only to T = 64 (about 2). Measured per
// call at H = 4096, I = 1536 with 32 of 256 experts, top-8: T = 80 104.2
// against 127.5 us with the wide GEMM1, T = 160 104.0 against 123.5, T = 256
// 113.9 against 130.1, T = 384 153.0 against 140.5 (the wide kernels win);
// with 16 of 128 experts, top-6: T = 128 54.3 against 61.8, T = 256 88.6
// against 74.9 (wide); at 7168 x 2048 the wide kernels lead from T = 96.
constexpr bool kSmallLayer = (int64_t)H * I < (int64_t)7168 * 2048;
constexpr int64_t kStreamMaxSlotsPerExpert = 8;

Variants pick_variants(int64_t T) {
    Variants v;
    // Measured on MI355X: streaming workgroups (GEMM1 with K split over 4
    // waves) while an expert has at most a few row tiles, 64-column GEMM2 waves from T = 64, the
    // wide kernels (register-ring weights, LDS activations) for roughly 5 to
    // 70 rows per expert (GEMM2 from ~10 to ~15), the LDS-tiled kernels beyond.
    // GEMM2 with the combine (K split over its 4 waves, which keeps them all
    // busy with fewer than 4 row tiles): one launch fewer where launches
    // dominate (T <= 4). From T = 1 on the K-split GEMM1 (per call with two
    // local slots: 27.9 against 35.6 us for single-wave workgroups, 0.4 us
    // slower with none); at 7168 x 2048 the K-split 32-column GEMM2 waves up
    // to T = 16: with random routing T = 12 30.8 against 37.0 us for 64-column
    // waves, T = 16 77.1 against 79.3; with every token on the same 8 experts
    // (16 activation rows per tile, which 32-column waves re-read twice as
    // often) T = 16 83.9 against 77.0, T = 32 158.6 against 139.0.
    if (T <= 4) v = {16, VARIANT_GEMM2_COMBINE_KS};
    else if (T <= 8 && kSmallLayer) v = {16, 5};
    else if (T <= 16 && !kSmallLayer) v = {16, 16};
    else if (T <= 64) v = {16, 14};
    else if (kSmallLayer && T * TOPK <= kStreamMaxSlotsPerExpert * EG) v = {16, 14};
    else if (T <= 128) v = {15, 14};  // the wide GEMM1 folds in the sort from T = 65
    else if (T <= 176) v = {15, 13};  // wide GEMM2 ahead by 3.5 us at T = 192, behind by ~2 at 160
    // The wide GEMM2 (32-row tiles) to T = 640, the LDS tile above: per call
    // (one process, three alternating passes, four shard offsets) the wide
    // kernel is 6-18 us faster at T = 320, 1-28 at 448 and 512, level on
    // average at 640, and 10-23 us slower at 768.
    else if (T <= 640) v = {15, 15};
    // GEMM2 LDS tile as one software pipeline (variant 20): bitwise equal to
    // variant 3, per call (one process, three alternating passes) T=1024
    // 367.6 against 372.7 us, T=1536 299.8 against 305.4, T=2048 336-337
    // against 343-345, T=3072 448.4 against 454.3, T=8192 level to 7 us
    // faster; 0.3 % slower at T=14000 with every token on 8 experts. The
    // same kernel run by one workgroup per CU (variant 21), which copies the
    // next tile's first k-blocks during the last ones of the current tile, is
    // bitwise equal and faster again (per call, one process, alternating
    // passes: T=8192 866.3 against 885.6 us, T=14000 skewed 6,633 against
    // 6,649, T=4096 358.3 against 362.0, T=2048 334.2 against 337.4, T=1536
    // 419.4 against 422.6, T=1024 364.6 against 370.5 and 221.0 against
    // 224.1 at two shard offsets).
    else if (T <= 1536) v = {15, 21};
    // GEMM1 LDS tile as one software pipeline (barriers inside the MFMA
    // stream, weight fragments held in registers): bitwise equal to variant
    // 18 and faster at every T (GEMM1 per launch, one process: T=8192 401-420
    // against 436-509 us, T=14000 skewed 2972 against 3151, T=3072 287
    // against 308); level with the wide kernel at T=2048.
    else v = {19, 21};
    // From T = 640 to 1536 the GEMM1 kernel is chosen on the device from the
    // expert counts (G1_SELECT_EXTRA_TILES): the wide kernel streams an
    // expert's weights once per 64-row tile, the LDS tile once per 256 rows,
    // so experts with hundreds of rows favour the tile (T=1024 offset 0 with
    // 1,966 slots: 337 against 368 us per call) and evenly spread slots the
    // wide kernel (T=1024 offset 64: 223 against 255). Both are launched; the
    // one not chosen finds no tiles. MI_MOE_G1_SELECT=0 keeps the wide kernel.
    // The same rule picks the faster kernel with 64 local experts (T = 768 to
    // 1536: the tile 17-85 us faster at 15-34 extra tiles, the wide kernel 9
    // us faster at 6); at H = 4096, I = 1536 the wide kernel wins to T = 1536
    // at up to 18 extra tiles, so smaller layers keep it.
    if (T >= 640 && T <= 1536 && !kSmallLayer) v.g1_alt = 19;
    const char* env = getenv("MI_MOE_VARIANT");
    if (env && *env) {
        int a = -1, b = -1;
        const int n = sscanf(env, "%d,%d", &a, &b);
        if (n >= 1 && a >= 0 && a < NUM_VARIANTS) v.g1 = a;
        if (n == 2 && b >= 0 && b < NUM_VARIANTS) v.g2 = b;
        else if (n == 1 && a >= 0 && a < NUM_VARIANTS) v.g2 = a;
        v.g1_alt = -1;  // a forced variant runs as asked
    }
    if (env_flag("MI_MOE_G1_SELECT") == 0) v.g1_alt = -1;
    return v;
}

}  // namespace

extern "C" {

size_t mi_moe_workspace_size(int64_t num_tokens) { return make_layout(num_tokens).total; }

int mi_moe_workspace_layout(int64_t num_tokens, mi_moe_layout* out) {
    if (!out) return fail(MI_MOE_ERR_INVALID, "mi_moe_workspace_layout: out is NULL");
    if (num_tokens < 0 || num_tokens > kMaxTokens)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_workspace_layout: num_tokens %lld out of range",
                    (long long)num_tokens);
    *out = make_layout(num_tokens);
    return MI_MOE_OK;
}

const char* mi_moe_last_error(void) { return g_last_error.c_str(); }

#define MI_MOE_STR2(x) #x
#define MI_MOE_STR(x) MI_MOE_STR2(x)
const char* mi_moe_version(void) {
    return "mi_moe 0.2.0 gfx950 h" MI_MOE_STR(MI_MOE_HIDDEN) " i" MI_MOE_STR(MI_MOE_INTER) " e" MI_MOE_STR(
        MI_MOE_E_LOCAL) " g" MI_MOE_STR(MI_MOE_E_GLOBAL) " ng" MI_MOE_STR(MI_MOE_N_GROUP) " kg" MI_MOE_STR(
        MI_MOE_TOPK_GROUP) " k" MI_MOE_STR(MI_MOE_TOP_K);
}

int mi_moe_route(const float* routing_logits, const void* routing_bias, int32_t bias_dtype,
                 int64_t num_tokens, float routed_scaling_factor, int32_t* topk_ids,
                 float* topk_weights, void* stream) {
    g_last_error.clear();
    if (num_tokens < 0 || num_tokens > kMaxTokens)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_route: num_tokens %lld out of range",
                    (long long)num_tokens);
    if (bias_dtype != MI_MOE_DTYPE_BF16 && bias_dtype != MI_MOE_DTYPE_F32)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_route: unknown bias_dtype %d", bias_dtype);
    if (!isfinite(routed_scaling_factor))
        return fail(MI_MOE_ERR_INVALID, "mi_moe_route: routed_scaling_factor is not finite");
    if (num_tokens == 0) return MI_MOE_OK;
    if (!routing_logits || !routing_bias || !topk_ids || !topk_weights)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_route: NULL pointer argument");
    if (!aligned(routing_logits, 16) || !aligned(routing_bias, bias_dtype ? 16 : 8) ||
        !aligned(topk_ids, 4) || !aligned(topk_weights, 4))
        return fail(MI_MOE_ERR_INVALID, "mi_moe_route: misaligned pointer");
    hipError_t err = launch_route(routing_logits, routing_bias, bias_dtype == MI_MOE_DTYPE_F32,
                                  (int)num_tokens, routed_scaling_factor, topk_ids, topk_weights,
                                  (hipStream_t)stream, /*packed=*/true);
    if (err != hipSuccess)
        return fail(MI_MOE_ERR_HIP, "mi_moe_route: launch failed: %s", hipGetErrorString(err));
    return MI_MOE_OK;
}

int mi_moe_get_definition(mi_moe_definition* out) {
    g_last_error.clear();
    if (!out) return fail(MI_MOE_ERR_INVALID, "mi_moe_get_definition: out is NULL");
    out->hidden_size = H;
    out->intermediate_size = I;
    out->num_local_experts = EL;
    out->num_experts = EG;
    out->n_group = NGROUP;
    out->topk_group = KGROUP;
    out->top_k = TOPK;
    return MI_MOE_OK;
}

int mi_moe_shape(int32_t* hidden_size, int32_t* intermediate_size) {
    g_last_error.clear();
    if (!hidden_size || !intermediate_size)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_shape: NULL pointer argument");
    *hidden_size = H;
    *intermediate_size = I;
    return MI_MOE_OK;
}

int mi_moe_sort(const int32_t* topk_ids, const float* topk_weights, int64_t num_tokens,
                int64_t local_expert_offset, void* workspace, size_t workspace_bytes, void* stream) {
    g_last_error.clear();
    if (num_tokens < 0 || num_tokens > kMaxTokens)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_sort: num_tokens %lld out of range",
                    (long long)num_tokens);
    if (num_tokens == 0) return MI_MOE_OK;
    if (!topk_ids || !topk_weights || !workspace)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_sort: NULL pointer argument");
    const bool direct = TOPK == TOPK_LD;  // rows already in the workspace's stride
    if (!aligned(topk_ids, direct ? 16 : 4) || !aligned(topk_weights, direct ? 16 : 4) ||
        !aligned(workspace, 256))
        return fail(MI_MOE_ERR_INVALID, "mi_moe_sort: misaligned pointer");
    const mi_moe_layout L = make_layout(num_tokens);
    if (workspace_bytes < L.total)
        return fail(MI_MOE_ERR_WORKSPACE, "mi_moe_sort: workspace has %zu bytes, needs %zu",
                    workspace_bytes, L.total);
    Plan p = make_plan(workspace, L, num_tokens, local_expert_offset, 0.f);
    hipError_t err = hipSuccess;
    if (direct) {
        p.topk_ids = const_cast<int*>(topk_ids);  // read only
        p.topk_w = const_cast<float*>(topk_weights);
    } else {  // [T, TOPK] rows -> the workspace's TOPK_LD-wide rows
        err = launch_repack_topk(topk_ids, topk_weights, (int)num_tokens, p.topk_ids, p.topk_w,
                                 (hipStream_t)stream);
    }
    const Variants var = pick_variants(num_tokens);
    if (err == hipSuccess)
        err = launch_sort(p, gemm1_bm(var.g1), gemm2_bm(var.g2), (hipStream_t)stream);
    if (err != hipSuccess)
        return fail(MI_MOE_ERR_HIP, "mi_moe_sort: launch failed: %s", hipGetErrorString(err));
    return MI_MOE_OK;
}

int mi_moe_quantize_fp8(const void* hidden_bf16, int64_t num_tokens, uint8_t* hidden_states,
                        float* hidden_states_scale, void* stream) {
    g_last_error.clear();
    if (num_tokens < 0 || num_tokens > kMaxTokens)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_quantize_fp8: num_tokens %lld out of range",
                    (long long)num_tokens);
    if (num_tokens == 0) return MI_MOE_OK;
    if (!hidden_bf16 || !hidden_states || !hidden_states_scale)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_quantize_fp8: NULL pointer argument");
    if (!aligned(hidden_bf16, 16) || !aligned(hidden_states, 16) || !aligned(hidden_states_scale, 4))
        return fail(MI_MOE_ERR_INVALID, "mi_moe_quantize_fp8: misaligned pointer");
    hipError_t err = launch_quant_fp8(hidden_bf16, (int)num_tokens, hidden_states,
                                      hidden_states_scale, (hipStream_t)stream);
    if (err != hipSuccess)
        return fail(MI_MOE_ERR_HIP, "mi_moe_quantize_fp8: launch failed: %s",
                    hipGetErrorString(err));
    return MI_MOE_OK;
}

// hidden_bf16 != nullptr: quantise it into a->hidden_states / scale first
// (mi_moe_run_bf16), in the same launch as routing.
static int run_impl(const mi_moe_args* a, hipStream_t s, hipEvent_t const* ev,
                    const void* hidden_bf16 = nullptr) {
    g_last_error.clear();
    if (!a) return fail(MI_MOE_ERR_INVALID, "mi_moe_run: args is NULL");
    const int64_t T = a->num_tokens;
    if (T < 0 || T > kMaxTokens)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_run: num_tokens %lld out of range [0, %lld]",
                    (long long)T, (long long)kMaxTokens);
    if (a->bias_dtype != MI_MOE_DTYPE_BF16 && a->bias_dtype != MI_MOE_DTYPE_F32)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_run: unknown bias_dtype %d", a->bias_dtype);
    if (a->reserved != 0) return fail(MI_MOE_ERR_INVALID, "mi_moe_run: reserved must be 0");
    if (!isfinite(a->routed_scaling_factor))
        return fail(MI_MOE_ERR_INVALID, "mi_moe_run: routed_scaling_factor is not finite");
    if (T == 0) {
        if (ev) {
            for (int i = 0; i <= MI_MOE_NUM_PHASES; ++i) {
                hipError_t e = hipEventRecord(ev[i], s);
                if (e != hipSuccess)
                    return fail(MI_MOE_ERR_HIP, "mi_moe_run: event record failed: %s",
                                hipGetErrorString(e));
            }
        }
        return MI_MOE_OK;
    }

    const void* ptrs[] = {a->routing_logits, a->routing_bias, a->hidden_states,
                          a->hidden_states_scale, a->gemm1_weights, a->gemm1_weights_scale,
                          a->gemm2_weights, a->gemm2_weights_scale, a->output, a->workspace};
    const char* names[] = {"routing_logits", "routing_bias", "hidden_states",
                           "hidden_states_scale", "gemm1_weights", "gemm1_weights_scale",
                           "gemm2_weights", "gemm2_weights_scale", "output", "workspace"};
    const size_t align[] = {16, (size_t)(a->bias_dtype == MI_MOE_DTYPE_F32 ? 16 : 8), 16, 4, 16,
                            4, 16, 4, 8, 256};
    if (hidden_bf16 && !aligned(hidden_bf16, 16))
        return fail(MI_MOE_ERR_INVALID, "mi_moe_run_bf16: hidden_bf16 is not 16-byte aligned");
    for (int i = 0; i < 10; ++i) {
        if (!ptrs[i]) return fail(MI_MOE_ERR_INVALID, "mi_moe_run: %s is NULL", names[i]);
        if (!aligned(ptrs[i], align[i]))
            return fail(MI_MOE_ERR_INVALID, "mi_moe_run: %s is not %zu-byte aligned", names[i],
                        align[i]);
    }
    const mi_moe_layout L = make_layout(T);
    if (a->workspace_bytes < L.total)
        return fail(MI_MOE_ERR_WORKSPACE, "mi_moe_run: workspace has %zu bytes, needs %zu",
                    a->workspace_bytes, L.total);

    Plan p = make_plan(a->workspace, L, T, a->local_expert_offset, a->routed_scaling_factor);

    const Variants var = pick_variants(T);
    const int g2_mode = gemm2_mode_for(T, var.g2);
    if (g2_mode != G2_BF16) p.part_f32 = (float*)p.part;
    if (g2_mode == G2_SPLIT) p.act_lo = (uint16_t*)((uint8_t*)a->workspace + L.act_lo);
    hipError_t err = hipSuccess;
    // mark(i) opens phase i (0 route, 1 sort, 2 GEMM1, 3 GEMM2, 4 combine)
    // and closes phase i - 1; the named ranges join route and sort.
    const Roctx* rx = roctx();
    auto mark = [&](int i) {
        if (ev && err == hipSuccess) err = hipEventRecord(ev[i], s);
        if (!rx) return;
        switch (i) {
            case 0: rx->push("mi_moe_run"); rx->push("phase1_route_permute"); break;
            case 2: rx->pop(); rx->push("phase3_gemm1"); break;
            case 3: rx->pop(); rx->push("phase5_gemm2"); break;
            case 4: rx->pop(); rx->push("phase6_scatter"); break;
            case 5: rx->pop(); rx->pop(); break;
            default: break;
        }
    };
    const int bias_f32 = a->bias_dtype == MI_MOE_DTYPE_F32;
    Front front = pick_front(T, var.g1);
    if (hidden_bf16)  // routing runs with the quantiser; GEMM1 needs its output
        front = (gemm1_sorts_supported((int)T, var.g1) && env_flag("MI_MOE_SORT_IN_GEMM1") != 0)
                    ? Front::SORT_IN_GEMM1
                    : Front::KERNELS;
    // the device-side GEMM1 choice needs the sort launch's counts
    const bool g1_choice = var.g1_alt >= 0 && front == Front::KERNELS;
    if (g1_choice) p.g1_alt_bm = gemm1_bm(var.g1_alt);
    const FrontArgs fa{a->routing_logits, a->routing_bias, bias_f32, gemm1_bm(var.g1),
                       gemm2_bm(var.g2)};
    mark(0);
    if (hidden_bf16) {
        if (err == hipSuccess)
            err = launch_quant_route(hidden_bf16, (int)T, (uint8_t*)a->hidden_states,
                                     (float*)a->hidden_states_scale, a->routing_logits,
                                     a->routing_bias, bias_f32, p.rsf, p.topk_ids, p.topk_w, s);
    } else if (front == Front::FUSED) {
        if (err == hipSuccess)
            err = launch_route_sort(p, a->routing_logits, a->routing_bias, bias_f32, fa.bm1, fa.bm2,
                                    s);
    } else if (front != Front::ROUTE_IN_GEMM1) {
        if (err == hipSuccess)
            err = launch_route(a->routing_logits, a->routing_bias, bias_f32, p.T, p.rsf,
                               p.topk_ids, p.topk_w, s);
    }
    mark(1);
    if (err == hipSuccess && front == Front::KERNELS) err = launch_sort(p, fa.bm1, fa.bm2, s);
    mark(2);
    if (err == hipSuccess) {
        if (front == Front::SORT_IN_GEMM1 || front == Front::ROUTE_IN_GEMM1)
            err = launch_gemm1_front(p, a->hidden_states, a->hidden_states_scale, a->gemm1_weights,
                                     a->gemm1_weights_scale, var.g1,
                                     front == Front::ROUTE_IN_GEMM1 ? FRONT_ROUTE : FRONT_SORT, fa,
                                     s);
        else
            err = launch_gemm1(p, a->hidden_states, a->hidden_states_scale, a->gemm1_weights,
                               a->gemm1_weights_scale, var.g1, s);
        if (err == hipSuccess && g1_choice) {
            // the alternative kernel, on its own row-tile table (empty unless chosen)
            Plan q = p;
            q.g1_mtile = META_MTILE1B;
            err = launch_gemm1(q, a->hidden_states, a->hidden_states_scale, a->gemm1_weights,
                               a->gemm1_weights_scale, var.g1_alt, s);
        }
    }
    mark(3);
    const bool fused_ks = var.g2 == VARIANT_GEMM2_COMBINE_KS && gemm2_combine_supported(p.T);
    const bool fused =
        fused_ks || (var.g2 == VARIANT_GEMM2_COMBINE && gemm2_combine_supported(p.T));
    if (err == hipSuccess) {
        if (fused_ks)
            err = launch_gemm2_combine_ks(p, a->gemm2_weights, a->gemm2_weights_scale,
                                          (uint16_t*)a->output, s);
        else if (fused)
            err = launch_gemm2_combine(p, a->gemm2_weights, a->gemm2_weights_scale,
                                       (uint16_t*)a->output, s);
        else
            err = launch_gemm2(p, a->gemm2_weights, a->gemm2_weights_scale,
                               (var.g2 == VARIANT_GEMM2_COMBINE ||
                                var.g2 == VARIANT_GEMM2_COMBINE_KS) ? 0 : var.g2, s);
    }
    mark(4);
    if (err == hipSuccess && !fused) err = launch_combine(p, (uint16_t*)a->output, s);
    mark(5);
    if (err != hipSuccess)
        return fail(MI_MOE_ERR_HIP, "mi_moe_run: launch failed: %s", hipGetErrorString(err));
    return MI_MOE_OK;
}

int mi_moe_run(const mi_moe_args* a, void* stream) {
    return run_impl(a, (hipStream_t)stream, nullptr);
}

int mi_moe_run_bf16(const mi_moe_args* a, const void* hidden_bf16, void* stream) {
    if (!hidden_bf16) {
        g_last_error.clear();
        return fail(MI_MOE_ERR_INVALID, "mi_moe_run_bf16: hidden_bf16 is NULL");
    }
    return run_impl(a, (hipStream_t)stream, nullptr, hidden_bf16);
}

int mi_moe_run_noalloc(const mi_moe_args* a, void* stream) {
    g_last_error.clear();
    if (!a) return fail(MI_MOE_ERR_INVALID, "mi_moe_run_noalloc: args is NULL");
    if (a->workspace || a->workspace_bytes)
        return fail(MI_MOE_ERR_INVALID,
                    "mi_moe_run_noalloc: workspace must be NULL and workspace_bytes 0 (the "
                    "library's per-GPU scratch holds the intermediates)");
    if (a->num_tokens > MI_MOE_NOALLOC_MAX_TOKENS)
        return fail(MI_MOE_ERR_INVALID,
                    "mi_moe_run_noalloc: num_tokens %lld exceeds MI_MOE_NOALLOC_MAX_TOKENS (%d); "
                    "use mi_moe_run with a workspace",
                    (long long)a->num_tokens, MI_MOE_NOALLOC_MAX_TOKENS);
    void* ws = nullptr;
    const int rc = scratch_address((hipStream_t)stream, &ws);
    if (rc != MI_MOE_OK) return rc;
    mi_moe_args b = *a;
    b.workspace = ws;
    b.workspace_bytes = kScratchBytes;
    return run_impl(&b, (hipStream_t)stream, nullptr);
}

int mi_moe_run_profiled(const mi_moe_args* a, void* stream, void* const* events, int32_t n_events) {
    g_last_error.clear();
    if (!events || n_events != MI_MOE_NUM_PHASES + 1)
        return fail(MI_MOE_ERR_INVALID, "mi_moe_run_profiled: needs %d events, got %d",
                    MI_MOE_NUM_PHASES + 1, (int)n_events);
    for (int i = 0; i < n_events; ++i)
        if (!events[i]) return fail(MI_MOE_ERR_INVALID, "mi_moe_run_profiled: event %d is NULL", i);
    return run_impl(a, (hipStream_t)stream, (hipEvent_t const*)events);
}

}  // extern "C"
