/*
 * mi_moe: MI355X (gfx950) fused Mixture-of-Experts operator, C ABI.
 *
 * One call computes the DeepSeek-routed, FP8 block-scaled MoE layer for one
 * expert-parallel shard of 32 local experts, definition
 * moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048
 * (H = 7168, I = 2048, 256 global experts in 8 groups of 32, top-4 groups,
 * top-8 experts, 128-element scale blocks). The shapes below are written for
 * that definition; a library built for another one (mi_moe_get_definition:
 * hidden size H, intermediate size I, E local experts, G global experts in
 * n_group groups, topk_group groups kept, top_k experts per token) takes the
 * same layouts with 7168 -> H, 2048 -> I, 4096 -> 2I, 56 -> H/128,
 * 32 (GEMM1 n-blocks) -> 2I/128, 16 -> I/128, 32 (experts) -> E, 256 -> G
 * and 8 (top-k) -> top_k.
 *
 * All pointers are device pointers; the caller owns every buffer, including
 * the workspace. The library never allocates device memory, never
 * synchronises the host, and enqueues all work on the given stream.
 */
#ifndef MI_MOE_H_
#define MI_MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define MI_MOE_OK 0
#define MI_MOE_ERR_INVALID 1   /* bad pointer, size, alignment or scalar */
#define MI_MOE_ERR_WORKSPACE 2 /* workspace_bytes < mi_moe_workspace_size(T) */
#define MI_MOE_ERR_HIP 3       /* a HIP launch failed */

/* Element type of routing_bias. */
#define MI_MOE_DTYPE_BF16 0
#define MI_MOE_DTYPE_F32 1

/* Largest num_tokens any entry point accepts (larger T is MI_MOE_ERR_INVALID):
 * the row-gathering GEMM kernels keep byte offsets in 32 bits. */
#define MI_MOE_MAX_TOKENS 131072

/* Arguments of one call. Field order and meaning follow the reference entry
 * point solution/triton/kernel.py:600-613 (run(routing_logits, routing_bias,
 * hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
 * gemm2_weights, gemm2_weights_scale, local_expert_offset,
 * routed_scaling_factor, output)); shapes are those of kernel.py:615-627.
 * Every tensor is dense, row-major, 16-byte aligned. */
typedef struct mi_moe_args {
    const float* routing_logits;       /* fp32 [T, 256] */
    const void* routing_bias;          /* bf16 or fp32 [256] (bias_dtype) */
    const uint8_t* hidden_states;      /* fp8 e4m3fn [T, 7168] */
    const float* hidden_states_scale;  /* fp32 [56, T] (block-major) */
    const uint8_t* gemm1_weights;      /* fp8 e4m3fn [32, 4096, 7168] */
    const float* gemm1_weights_scale;  /* fp32 [32, 32, 56] */
    const uint8_t* gemm2_weights;      /* fp8 e4m3fn [32, 7168, 2048] */
    const float* gemm2_weights_scale;  /* fp32 [32, 56, 16] */
    int64_t local_expert_offset;       /* first global expert id of this shard */
    float routed_scaling_factor;
    void* output;                      /* bf16 [T, 7168], fully overwritten */
    int64_t num_tokens;                /* 0 <= T <= MI_MOE_MAX_TOKENS */
    int32_t bias_dtype;                /* MI_MOE_DTYPE_* */
    int32_t reserved;                  /* must be 0 */
    void* workspace;                   /* >= mi_moe_workspace_size(T) bytes, 256-B aligned */
    size_t workspace_bytes;
} mi_moe_args;

/* Byte offsets of the intermediate buffers inside the workspace, for staged
 * parity checks. Layout of each buffer (k = top_k, rows of the [T, 8] tables
 * are 8 wide whatever k is; entries past k are padding):
 *   topk_ids   int32 [T, 8]   global expert ids in selection order
 *   topk_w     fp32  [T, 8]   routing weights (kernel.py:450)
 *   expert_off int32 [E+1]    exclusive prefix of local slot counts (S = [E]),
 *                             followed by the row-tile prefixes of the default
 *                             GEMM kernels at int offsets 64 and 128 (E <= 32)
 *                             or 128 and 256 (E = 64); from T = 640 to 1536
 *                             also the 256-row GEMM1 prefix at 192 and the
 *                             device's GEMM1 choice at 256 (1: the 256-row
 *                             tile, whose prefix then holds the tiles; 0: the
 *                             64-row one, the prefix at 64). The prefix of the
 *                             kernel not chosen has a total of 0.
 *   sorted_tok int32 [kT]     token of each slot, expert-major, token-ascending
 *   sorted_w   fp32  [kT]     routing weight of each slot
 *   tok_slot   int32 [T, 8]   slots of each token, ascending local expert, -1 pad
 *   chunk_cnt  int32 [ceil(T/256), E]   per-256-token-chunk local expert counts
 *   act        bf16  [kT, 2048]  SwiGLU(GEMM1) per slot, rounded to bf16
 *   part       bf16  [kT, 7168]  routing weight x GEMM2 row per slot; fp32
 *                             (same offset, twice the bytes) at T <= 1024
 *   act_lo     bf16  [kT, 2048]  SwiGLU(GEMM1) - act, reserved at T <= 256
 *                             (empty above) and written when the environment
 *                             sets MI_MOE_SPLIT_ACT=1: GEMM2 then multiplies
 *                             act + act_lo, 16 mantissa bits, wider than the
 *                             reference's TF32 operand (kernel.py:272-278) */
typedef struct mi_moe_layout {
    size_t topk_ids, topk_w, expert_off, sorted_tok, sorted_w, tok_slot, chunk_cnt, act, part;
    size_t act_lo;
    size_t total;
} mi_moe_layout;

/* Workspace bytes needed for T tokens. Replaces the reference's per-call
 * torch allocations (kernel.py:535-536, :576-581, :710, :747, :769, :801). */
size_t mi_moe_workspace_size(int64_t num_tokens);

/* Fills *out with the workspace layout for T tokens. Returns MI_MOE_OK. */
int mi_moe_workspace_layout(int64_t num_tokens, mi_moe_layout* out);

/* The fused MoE forward pass; replaces kernel.py::run (kernel.py:600-825).
 * Validates everything before the first launch; on error nothing is
 * enqueued. stream is a hipStream_t (NULL = default stream). */
int mi_moe_run(const mi_moe_args* args, void* stream);

/* mi_moe_run plus phase timing: records the caller's HIP events
 * (hipEvent_t, n_events == MI_MOE_NUM_PHASES + 1) on the stream before the
 * first kernel and after each of the phases route, sort, gemm1 (+SwiGLU),
 * gemm2, combine. A phase whose work another launch does (routing and the
 * sort inside GEMM1 at T = 1, the sort inside GEMM1 up to T = 64, the combine
 * inside GEMM2 at T <= 4) records its two events back to back. Counterpart of the
 * reference's env-gated phase events (kernel.py:634-672, phase names
 * :677-823). */
#define MI_MOE_NUM_PHASES 5
int mi_moe_run_profiled(const mi_moe_args* args, void* stream, void* const* events,
                        int32_t n_events);

/* mi_moe_run from bf16 activations: quantises hidden_bf16 (bf16 [T, 7168],
 * 16-byte aligned) into args->hidden_states and args->hidden_states_scale,
 * which are written (same formula and layout as mi_moe_quantize_fp8), and
 * routes the tokens in that same first launch; then the call continues as
 * mi_moe_run. No counterpart in the reference, whose inputs arrive quantised:
 * it equals mi_moe_quantize_fp8 followed by mi_moe_run, one launch shorter,
 * for callers that start from bf16 hidden states. */
int mi_moe_run_bf16(const mi_moe_args* args, const void* hidden_bf16, void* stream);

/* Routing only (kernel.py:371-457 without the local filter): writes global
 * top-k ids (int32 [T, top_k], selection order) and weights (fp32
 * [T, top_k]); 4-byte aligned. */
int mi_moe_route(const float* routing_logits, const void* routing_bias, int32_t bias_dtype,
                 int64_t num_tokens, float routed_scaling_factor, int32_t* topk_ids,
                 float* topk_weights, void* stream);

/* Local-expert sort only (kernel.py:460-516 and the scan at :572-581), for
 * staged parity: from global top-k ids (int32 [T, top_k]) and weights (fp32
 * [T, top_k]), e.g. those of mi_moe_route, writes into the workspace (offsets
 * from mi_moe_workspace_layout) what mi_moe_run's sort writes: expert_off
 * int32[E+1] (followed by the row-tile prefixes of T's default GEMM kernels),
 * sorted_tok / sorted_w [S] (slots grouped by local expert, token-ascending
 * inside an expert) and tok_slot int32 [T, 8] (a token's slots in ascending
 * local expert, then -1). Ids outside [local_expert_offset,
 * local_expert_offset + E) are not local. topk pointers 16-byte aligned when
 * top_k = 8, else 4-byte; workspace 256-byte aligned and at least
 * mi_moe_workspace_size(T) bytes. */
int mi_moe_sort(const int32_t* topk_ids, const float* topk_weights, int64_t num_tokens,
                int64_t local_expert_offset, void* workspace, size_t workspace_bytes, void* stream);

/* FP8 activation quantiser feeding mi_moe_run: bf16 hidden states [T, 7168]
 * -> hidden_states fp8 e4m3fn [T, 7168] and hidden_states_scale fp32 [56, T]
 * (block-major, the layout kernel.py:169 reads). Per token and 128-element
 * block: s = max(amax, 1e-10) / 448, q = e4m3(clamp(x / s, -448, 448)),
 * round to nearest even, IEEE fp32 division. Inputs must be finite.
 * No counterpart in the reference, whose inputs arrive already quantised; it
 * produces exactly the hidden_states / hidden_states_scale pair of
 * kernel.py:600-613. Pointers 16-byte aligned (scale: 4-byte). */
int mi_moe_quantize_fp8(const void* hidden_bf16, int64_t num_tokens, uint8_t* hidden_states,
                        float* hidden_states_scale, void* stream);

/* The definition this library is compiled for: the reference hard-codes it
 * (kernel.py:615-625) and its routing kernel takes E_GLOBAL, N_GROUP,
 * TOPK_GROUP and TOP_K as constexpr parameters (kernel.py:371-389);
 * libmi_moe.so is moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048,
 * the other builds are named by their fields. */
typedef struct mi_moe_definition {
    int32_t hidden_size;        /* H */
    int32_t intermediate_size;  /* I */
    int32_t num_local_experts;  /* E: 16, 32 or 64 */
    int32_t num_experts;        /* G: 64, 128 or 256 */
    int32_t n_group;            /* routing groups of G / n_group experts */
    int32_t topk_group;         /* groups kept per token */
    int32_t top_k;              /* experts per token, <= 8 */
} mi_moe_definition;
int mi_moe_get_definition(mi_moe_definition* out);

/* Hidden size H and expert intermediate size I this library is compiled for
 * (kernel.py:615-625 hard-codes 7168 and 2048; libmi_moe.so is that shape,
 * libmi_moe_h<H>_i<I>.so others). Every tensor shape of mi_moe_args follows
 * from them; no counterpart in the reference. */
int mi_moe_shape(int32_t* hidden_size, int32_t* intermediate_size);

/* Largest num_tokens mi_moe_run_noalloc accepts. */
#define MI_MOE_NOALLOC_MAX_TOKENS 256

/* mi_moe_run without a caller workspace and without any allocation, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. args->workspace must be NULL and args->workspace_bytes 0:
 * the intermediates live in the library's static device array (one per GPU,
 * mi_moe_workspace_size(MI_MOE_NOALLOC_MAX_TOKENS) bytes, about 76 MB at
 * H = 7168, I = 2048, held until the process ends), so num_tokens is at most
 * MI_MOE_NOALLOC_MAX_TOKENS (larger T: MI_MOE_ERR_INVALID, nothing enqueued).
 * The first call on a device looks up that array's address there. The
 * kernels, results and every other check are those of mi_moe_run; the array
 * keeps the previous call's contents and nothing in it needs to start at zero.
 * Calls that overlap on one GPU (two streams, two threads, or a replayed
 * graph and another call) share the array and race: serialise them. */
int mi_moe_run_noalloc(const mi_moe_args* args, void* stream);

/* Message of the last error on the calling thread ("" if none). */
const char* mi_moe_last_error(void);

/* Library version string. */
const char* mi_moe_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MI_MOE_H_ */
