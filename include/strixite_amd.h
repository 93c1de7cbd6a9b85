/* strixite_amd: MI355X (gfx950, CDNA4, wave64) kernels for strixite's MTP verify path, behind a C ABI.
 *
 * Every entry point is asynchronous on the caller's HIP stream (passed as `sx_stream`, a hipStream_t) unless it says
 * otherwise, takes plain device pointers and sizes, and returns SX_OK (0) or an error code; sx_last_error() returns the
 * calling thread's message for the last failure. Preconditions are checked on the host before any launch (the
 * reference's STRIX_CHECK set); data-dependent failures go to 3-word device error slots (first writer wins) and NaN
 * outputs, as in the reference. Nothing here allocates device memory: callers pass workspaces sized by the
 * *_workspace_bytes functions.
 *
 * Each declaration names the reference interface it replaces (file:line in TheBeaninator/strixite). The C++ shim that
 * gives the reference's own kernels/ *.hpp signatures on top of these is strixite_amd/integration/strix_kernels_shim.cpp.
 */
#ifndef STRIXITE_AMD_H
#define STRIXITE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *sx_stream; /* hipStream_t */

enum sx_status { SX_OK = 0, SX_EINVAL = 1, SX_EHIP = 2, SX_EUNSUPPORTED = 3 };

/* Activation dtype: strix::kernels::Act (kernels/norm.hpp:20), F32 or BF16 raw bits. */
enum sx_act { SX_ACT_F32 = 0, SX_ACT_BF16 = 1 };

/* strix::kernels::MoeMath (kernels/moe_grouped.hpp:35). On gfx950 all three run the MFMA path on exact codes with
 * FP32 accumulation (F32 semantics: the tightest of the three); the value is accepted for API compatibility. */
enum sx_moe_math { SX_MOE_F32 = 0, SX_MOE_WMMA_BF16 = 1, SX_MOE_WMMA_F16 = 2 };

/* Q4DeviceView (runtime/q4_device.hpp:13-18) / Q8DeviceView (runtime/q8_device.hpp:12-17): non-owning device views of
 * a [N, K] weight in the formats/q4.hpp:3-6 / q8.hpp:3-11 layout. q: N*K/2 (q4, low nibble = even k) or N*K (q8) bytes,
 * 16-byte aligned; scale, minv: [N, K/G] BF16 bits; G in {32, 64, 128}; w = code * scale + min. */
typedef struct sx_qview {
    const uint8_t *q;
    const uint16_t *scale;
    const uint16_t *minv;
    int64_t N, K, G;
} sx_qview;

const char *sx_last_error(void);
const char *sx_version(void);

/* ---- dense dequantizing GEMV/GEMM: y[M, N] = x[M, K] * deq(W)^T, FP32 accumulation, one rounding at the store ----
 * kernels/linear_q4.hpp:26-30 and kernels/linear_q8.hpp:13-14. out_act == act, or BF16 x -> F32 y. */
int sx_linear_q4(const void *x, const sx_qview *w, void *y, int64_t M, int act, int out_act, sx_stream stream);
int sx_linear_q8(const void *x, const sx_qview *w, void *y, int64_t M, int act, int out_act, sx_stream stream);

/* ---- per-slot MoE experts (decode / short verify), kernels/linear_q4.hpp:32-58 ----
 * w: E experts stacked [E*N, K]; ids [M, A] int32 device. err: >= 3 zeroed uint32 (device).
 *   gather:         y[m, a, :] = x[m, :] * W[ids[m, a]]^T                          (linear_q4.hpp:42-43)
 *   gather_swiglu:  h[m, a, j] = silu(g) * u over rows [gate (I) | up (I)]          (linear_q4.hpp:55-56)
 *   combine:        y[m, :] = sum_a coef[m, a] * (h[m, a, :] * W[ids[m, a]]^T)      (linear_q4.hpp:44-46) */
int sx_linear_q4_experts_gather(const void *x, const sx_qview *w, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                                void *y, int act, uint32_t *err, sx_stream stream);
int sx_linear_q4_experts_gather_swiglu(const void *x, const sx_qview *w, int64_t E, const int32_t *ids, int64_t M,
                                       int64_t A, void *h, int act, uint32_t *err, sx_stream stream);
int sx_linear_q4_experts_combine(const void *h, const sx_qview *w, int64_t E, const int32_t *ids, const float *coef,
                                 int64_t M, int64_t A, void *y, int act, uint32_t *err, sx_stream stream);
/* report_expert_error (kernels/linear_q4.hpp:61): the 3 words already on the host; SX_EINVAL + message if set. */
int sx_report_expert_error(const uint32_t e[3], const char *what);

/* ---- MoE router, kernels/moe_router.hpp:33-43 ----
 * Top k of E logits per token (value desc, lower index on a tie), coef = softmax over the k (FP32); optional shared
 * slot k with id shared_id and coef sigmoid(shared logit). Non-finite logit: ids -1, coef NaN, err {1, token, expert}.
 * k in 1..min(E, 32); E in 1..1024. */
int sx_moe_router(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const void *shared_logit,
                  int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, int act, uint32_t *err,
                  sx_stream stream);
/* report_router_error (kernels/moe_router.hpp:43). */
int sx_report_router_error(const uint32_t e[3], const char *what);
/* moe_shared_add / moe_shared_add_inject (kernels/moe_router.hpp:53-63). */
int sx_moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                      uint32_t gate_index, int act, uint32_t *err, sx_stream stream);
int sx_moe_shared_add_inject(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                             uint32_t gate_index, void *x, const float *w_in, int64_t H, int act, uint32_t *err,
                             sx_stream stream);

/* ---- grouped MoE experts (verify width and prefill), kernels/moe_grouped.hpp:42-62 ----
 * moe_group_routes buckets the M*A slots by expert into ws (int32 layout of moe_grouped.hip:63-81: header [n_tiles,
 * S, E, n_wtiles], offsets [E+2], slots [S], 16-slot tiles, 64-slot tiles); slot order within a bucket is unspecified
 * and no output depends on it. Bad ids go to bucket E and set err {1, id, slot}. */
int sx_moe_route_workspace_bytes(int64_t M, int64_t A, int64_t E, size_t *bytes);
int sx_moe_group_routes(const int32_t *ids, int64_t M, int64_t A, int64_t E, void *ws, size_t ws_bytes, uint32_t *err,
                        sx_stream stream);
/* moe_router (no shared slot) then moe_group_routes in one launch, for M*k <= 2048: the same ids, coef, error words
 * and workspace as those two calls (kernels/moe_router.hpp:38-40 + kernels/moe_grouped.hpp:47-49, the sequence
 * runtime/qwen4exp.cpp:1139-1147 runs at verify width). No reference counterpart as one call. */
int sx_moe_router_group(const void *logits, int64_t ld, int64_t M, int64_t E, int64_t k, int act, int32_t *ids,
                        float *coef, uint32_t *router_err, void *ws, size_t ws_bytes, uint32_t *expert_err,
                        sx_stream stream);
/* ---- verify-width MoE FFN in two launches (after the router projection) ----
 * The sequence runtime/qwen4exp.cpp:1139-1163 runs below kGroupedMinTokens - moe_router (moe_router.hpp:38-40),
 * linear_q4_experts_gather_swiglu (linear_q4.hpp:55-56), linear_q4_experts_combine (linear_q4.hpp:44-46) - with the
 * same ids, coef, h, y and error words; no reference counterpart as two calls. q4 G = 128, BF16 activations;
 * M <= 16, M * A <= 64 (A = k + 1 with a shared slot), gate_up K in {512 .. 4096}, down K in {1024, 2048};
 * sx_moe_verify_supported says whether a shape qualifies (SX_OK) or why not. Ew: experts stacked in the weights
 * (E, or E + 1 with the shared expert stacked). A repeated id within a token counts as an invalid slot. */
int sx_moe_verify_supported(int64_t M, int64_t A, int64_t E, int64_t k, int64_t Ew, const sx_qview *gate_up,
                            const sx_qview *down, int act);
/* route (ids, coef [M, A]; router_err) + h [M, A, I] = silu(x W_gate^T) * (x W_up^T) per slot (expert_err, NaN rows
 * for invalid slots). shared_logit nullable. h_sums (nullable, 16-byte aligned): FP32 [M * A, ceil(I / 16)], the sum
 * of each 16-feature run of the valid slots' h rows as stored, for sx_moe_verify_down. sync (nullable): a buffer of
 * sx_moe_verify_layer_sync_bytes bytes as sx_moe_verify_layer takes it (zeroed once, one per stream, may be the same
 * buffer): with K = 4096 each compute unit then streams a fixed run of about 4/5 of an equal share of the weight
 * tiles and takes the rest from a shared pool, so faster ones take more (without it each takes a fixed equal
 * share); the outputs are the same either way. plan (nullable): a device buffer of SX_VERIFY_PLAN_BYTES bytes,
 * 16-byte aligned, that receives the launch's routing in the form sx_moe_verify_down takes it. */
#define SX_VERIFY_PLAN_BYTES 4096
int sx_moe_verify_gate_up(const void *x, int64_t M, const float *logits, int64_t ld, int64_t E, int64_t k,
                          const float *shared_logit, int64_t shared_ld, int32_t shared_id, const sx_qview *gate_up,
                          int64_t Ew, int32_t *ids, float *coef, void *h, float *h_sums, int act,
                          uint32_t *router_err, uint32_t *expert_err, void *sync, void *plan, sx_stream stream);
/* y [M, N] = sum_a coef[m, a] * (h[m, a] W_down[ids[m, a]]^T); NaN rows for tokens with an invalid slot. h_sums
 * (nullable): the h_sums sx_moe_verify_gate_up wrote with this h (saves the kernel summing h itself). plan
 * (nullable): the plan sx_moe_verify_gate_up wrote with these ids and coef; the launch then takes the routing from
 * it (ids and coef are not read) instead of rebuilding the expert list, so its first weight loads go out sooner. */
int sx_moe_verify_down(const void *h, const float *h_sums, int64_t M, int64_t A, const int32_t *ids,
                       const float *coef, const sx_qview *down, int64_t Ew, void *y, int act, uint32_t *expert_err,
                       const void *plan, sx_stream stream);
/* ---- the whole verify-width MoE sublayer in one launch ----
 * runtime/qwen4exp.cpp:1132-1163 below kGroupedMinTokens - the router projection (linear_bf16w, kernels/linear.hpp:19-24,
 * or an FP32 weight), moe_router (moe_router.hpp:38-40), linear_q4_experts_gather_swiglu (linear_q4.hpp:55-56) and
 * linear_q4_experts_combine (linear_q4.hpp:44-46) - as one kernel whose phases hand over through counters in `sync`
 * instead of kernel boundaries; no reference counterpart as one call. wr: router weight [rows, d], FP32 (wr_act F32)
 * or BF16 bits; logits [M, rows] FP32 are written; shared != 0: slot k is expert shared_id with coefficient
 * sigmoid(logits[m, E]) (rows >= E + 1). ids, coef, h, h_sums, y, router_err, expert_err as sx_moe_verify_gate_up /
 * sx_moe_verify_down. Shapes: those sx_moe_verify_supported takes, with d = 4096 and E <= 1024. sync: a device buffer
 * of sx_moe_verify_layer_sync_bytes bytes, 16-byte aligned, zeroed once by the caller; one per stream: launches that
 * overlap in time must not share it. The launch runs one block per compute unit and needs them resident together; a
 * phase that waits more than 20 ms for another (another kernel holding compute units that long) gives up and sets
 * expert_err {1, 0xFFFFFFFE, phase} instead of hanging. */
int sx_moe_verify_layer_sync_bytes(size_t *bytes);
/* Diagnostic: a device buffer of (compute units x 16) uint64 that later sx_moe_verify_layer launches (any thread) fill
 * with each block's phase timestamps (s_memrealtime, 100 MHz): [0] start, [1] projection items done, [2] logits
 * fresh (wave 0), [8] tokens routed, [9] expert list built, [3] first gate_up weight loads issued, [4] gate_up done,
 * [5] h complete, [6] h staged, [7] end; and two counts: [10] polls of the logits, [11] gate_up rounds taken. NULL
 * turns it off (the default). No reference counterpart: the
 * reference's tracing (common/trace.hpp) marks host-side launch ranges, which cannot show phases inside a launch. */
int sx_moe_verify_layer_trace(uint64_t *buf);
int sx_moe_verify_layer(const void *x, int64_t M, const void *wr, int wr_act, int64_t rows, int64_t E, int64_t k,
                        int shared, int32_t shared_id, const sx_qview *gate_up, const sx_qview *down, int64_t Ew,
                        float *logits, int32_t *ids, float *coef, void *h, float *h_sums, void *y, int act,
                        uint32_t *router_err, uint32_t *expert_err, void *sync, sx_stream stream);
/* y [M, A, N] (linear_q4_experts_gather_grouped, moe_grouped.hpp:53-55). */
int sx_linear_q4_experts_gather_grouped(const void *x, const sx_qview *w, int64_t E, const void *ws, size_t ws_bytes,
                                        int64_t M, int64_t A, void *y, int act, int math, sx_stream stream);
/* y [M, N]; partial: M*A*N FP32 scratch (linear_q4_experts_combine_grouped, moe_grouped.hpp:60-62). */
int sx_linear_q4_experts_combine_grouped(const void *h, const sx_qview *w, int64_t E, const int32_t *ids,
                                         const float *coef, const void *ws, size_t ws_bytes, float *partial, int64_t M,
                                         int64_t A, void *y, int act, int math, sx_stream stream);
/* Grouped gather with the SwiGLU epilogue: h [M, A, N/2] = swiglu(gather_grouped(x)), bit-identical to
 * sx_linear_q4_experts_gather_grouped followed by sx_swiglu. No single reference counterpart: it fuses the two calls
 * runtime/qwen4exp.cpp:1154-1156 makes. */
int sx_linear_q4_experts_gather_swiglu_grouped(const void *x, const sx_qview *w, int64_t E, const void *ws,
                                               size_t ws_bytes, int64_t M, int64_t A, void *h, int act,
                                               sx_stream stream);

/* ---- SwiGLU, kernels/swiglu.hpp:21: gu [rows, 2I] -> h [rows, I]; BF16: h = bf16(bf16(silu(g)) * u). ---- */
int sx_swiglu(const void *gu, void *h, int64_t rows, int64_t I, int act, sx_stream stream);

/* ---- dense FP32-weight projection: y[M, N] (F32) = x[M, K] (act) * W[N, K]^T. The router logits of the
 * benchmark's MoE layers (fp32 Wr); plays the role kernels/linear.hpp linear_bf16w plays at runtime/qwen4exp.cpp:1132-1137. ---- */
int sx_linear_f32w(const void *x, const float *W, int64_t N, int64_t K, float *y, int64_t M, int act,
                   sx_stream stream);

/* ---- BF16-weight linear, kernels/linear.hpp:14-24 (linear_bf16w) and kernels/linear_wmma.hpp:25-28
 * (linear_bf16w_wmma): y[M, N] = x[M, K] * W^T, W [N, K] raw BF16 bits row-major, FP32 accumulation, one rounding at
 * the store; out_act == act, or BF16 x -> F32 y (the router logits of the served model: W [E + 1, d], the shared
 * expert's gate in the last row, runtime/qwen4exp.cpp:1132-1137). y must not overlap x. _wmma: x rounded to BF16
 * before the products, K % 64 == 0 and 16-byte aligned x and W (its prefill contract). ---- */
int sx_linear_bf16w(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, int act, int out_act,
                    sx_stream stream);
int sx_linear_bf16w_wmma(const void *x, const uint16_t *w, void *y, int64_t M, int64_t N, int64_t K, int act,
                         int out_act, sx_stream stream);

/* ---- logits top-k, kernels/logits_topk.hpp:26-46 ----
 * Per row the best k (value desc, lower id on a tie; -0 ties +0) of ids [0, n_valid); NaN left out and flagged in
 * nan[row]; optional allow mask [rows, mask_words]; padding (-inf, INT32_MAX). k in 1..64 (the reference: 20). */
typedef struct sx_logit_cand {
    float v;
    int32_t id;
} sx_logit_cand; /* LogitCand, kernels/logits_topk.hpp:29-33 */
int sx_logits_topk_workspace_bytes(int64_t rows, int64_t n_valid, int64_t k, size_t *bytes);
int sx_logits_topk(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, int64_t k, sx_logit_cand *out,
                   uint32_t *nan, void *workspace, size_t workspace_bytes, const uint32_t *mask, int64_t mask_words,
                   sx_stream stream);
/* sx_logits_topk without a workspace argument and without allocating: the level candidates live in a fixed scratch
 * array of SX_TOPK_SCRATCH_BYTES the library holds on each device it runs on (until the process ends). No counterpart
 * in the reference: it is for callers that cannot allocate (HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The same outputs as sx_logits_topk; SX_EINVAL when sx_logits_topk_workspace_bytes for the shape
 * exceeds the scratch (e.g. 64 rows of 248,320 logits at k = 64 still fit). Calls on one device share the scratch:
 * two that overlap in time (different streams) race. */
#define SX_TOPK_SCRATCH_BYTES (4u << 20)
int sx_logits_topk_noalloc(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, int64_t k,
                           sx_logit_cand *out, uint32_t *nan, const uint32_t *mask, int64_t mask_words,
                           sx_stream stream);

/* ---- the MTP draft head's Q4 copy of the Q8 LM head: formats/q4_from_q8.hpp:17-27 (quantize_q4_from_q8), which
 * runtime/qwen4exp.cpp:192-238 runs on the host at load; here on the device, from the resident Q8 rows ----
 * src: a Q8 view [N, K] (its first N rows: a row prefix of the head); G: the Q4 group (32, 64, 128; the served draft
 * head uses 64); q [N, K/2], scale / minv [N, K/G] BF16: the Q4 weight, byte-identical to the reference's. A
 * non-finite dequantized value (the reference throws) sets err {1, row, first k of its group} and that group's scale,
 * min and codes to zero. */
int sx_quantize_q4_from_q8(const sx_qview *src, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv,
                           uint32_t *err, sx_stream stream);

/* ---- MTP draft pick, kernels/mtp_pick.hpp:20-33: top-2 + NaN flag + the forward's error words, one 64-byte block.
 * emb_err points at the 8-byte EmbeddingError slot (kernels/embedding.hpp:26-28). ---- */
typedef struct sx_mtp_pick_s {
    int32_t best;
    float best_v, second_v;
    uint32_t nan;
    uint32_t err[9];
    uint32_t pad;
    unsigned long long emb;
} sx_mtp_pick_t;
int sx_mtp_pick(const float *logits, int64_t n, const uint32_t *router_err, const uint32_t *expert_err,
                const uint32_t *attn_err, const unsigned long long *emb_err, sx_mtp_pick_t *out, sx_stream stream);
/* The same pick (kernels/mtp_pick.hpp:20-33, the same output bit for bit) read by many blocks at once, one launch:
 * each block reduces its run of the logits to a top-2 in `workspace` and the last block to finish merges them.
 * workspace: device, 16-byte aligned, sx_mtp_pick_ws_bytes long, ZEROED before its first use (it holds a counter that
 * every call leaves ready for the next). Calls that share a workspace must be ordered on one stream. */
int sx_mtp_pick_ws_bytes(int64_t n, size_t *bytes);
/* The MTP draft head's LM head and pick in one launch (runtime/qwen4exp.cpp:1408-1413: the head's logits, then
 * kernels::mtp_pick over them): logits[N] = x[1, K] (BF16) . deq(w)^T in FP32 as sx_linear_q4 / q8 write them, and
 * `out` the pick of those logits, bit-identical to sx_mtp_pick's. bits 4 or 8; workspace as sx_mtp_pick_ws's (zeroed
 * before its first use). Shapes the fused GEMV does not take run sx_linear_q4 / q8 and then sx_mtp_pick_ws. */
int sx_mtp_head_pick(const void *x, const sx_qview *w, int bits, float *logits, const uint32_t *router_err,
                     const uint32_t *expert_err, const uint32_t *attn_err, const unsigned long long *emb_err,
                     sx_mtp_pick_t *out, void *workspace, size_t workspace_bytes, sx_stream stream);
int sx_mtp_pick_ws(const float *logits, int64_t n, const uint32_t *router_err, const uint32_t *expert_err,
                   const uint32_t *attn_err, const unsigned long long *emb_err, sx_mtp_pick_t *out, void *workspace,
                   size_t workspace_bytes, sx_stream stream);

/* ---- logits top-k and acceptance in one launch (the verify tail after the LM head) ----
 * sx_logits_topk (kernels/logits_topk.hpp:35-46) followed by sx_mtp_accept (serve/engine.cpp:592-653 with
 * serve/sampler.cpp:183-248), as one kernel whose blocks hand over through counters in `workspace`; no reference
 * counterpart as one call. cands / nan: as sx_logits_topk's out / nan (k = kc), for every row. out (nullable: top-k
 * only): as sx_mtp_accept's, for drafts [k] (rows >= k + 1). workspace: sx_verify_tail_workspace_bytes bytes, 8-byte
 * aligned, ZEROED before its first use (it holds counters each launch leaves at zero); one per stream. Rows of more
 * than 262,144 logits are refused (sx_logits_topk takes them). */
int sx_verify_tail_workspace_bytes(int64_t rows, int64_t n_valid, int64_t kc, size_t *bytes);
int sx_verify_tail(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, int64_t kc, sx_logit_cand *cands,
                   uint32_t *nan, const uint32_t *mask, int64_t mask_words, const int32_t *drafts, int64_t k,
                   const double *u, double temperature, int64_t top_k, double top_p, int32_t *out, void *workspace,
                   size_t workspace_bytes, sx_stream stream);
/* ---- draft acceptance on the device: serve/engine.cpp:592-610 with Sampler semantics (serve/sampler.cpp:183-248) ----
 * cands [k+1, kc] (from sx_logits_topk, value desc), nan [k+1], drafts [k] (device). Row j is sampled (greedy:
 * candidate 0; else temperature -> top_k (<= kc) -> top_p -> draw r = u[j] * kept, u[j] a host draw of
 * std::generate_canonical<double, 53> from the engine's mt19937_64, in order), accepting while the sample equals
 * drafts[j]. Writes out[0] = j (0..k), out[1] = status (0, or 1 + the row whose sampling failed: NaN or non-finite top
 * logit), out[2 .. 2+j] = the j+1 tokens committed (the accepted drafts, then row j's sample: the correction, or row
 * k's when all were accepted). Draws consumed on the host side: 0 (greedy) or j+1 (j on failure). */
int sx_mtp_accept(const sx_logit_cand *cands, const uint32_t *nan, int64_t kc, const int32_t *drafts, int64_t k,
                  const double *u, double temperature, int64_t top_k, double top_p, int64_t n_valid, int32_t *out,
                  sx_stream stream);

/* ---- strixw weight files: formats/strixw.hpp (the reader, StrixwFile :86-112) and runtime/strixw_loader.hpp (the
 * upload, StrixwDevice :22-52) ----
 * A file is a 128-byte header (magic "STRIXWT\0", format version 1..4, index and data-region offsets, file size, the
 * index's and the header's own strix_hash64), an index (metadata key/value pairs; one record per tensor: name,
 * encoding, shape, group size, experts, source parts, and each component's role, absolute offset, size and hash) and
 * a data region on a 4096-byte boundary: tensors start on 4096-byte boundaries, components on 256-byte ones.
 * Encodings and component roles carry the file's own numbering (formats/strixw.hpp:17-19). */
enum sx_strixw_encoding {
    SX_STRIXW_Q4 = 1, SX_STRIXW_Q4_CHUNK_MAJOR = 2, SX_STRIXW_BF16 = 3, SX_STRIXW_F32 = 4, SX_STRIXW_I64 = 5,
    SX_STRIXW_Q8 = 6, SX_STRIXW_Q8_CHUNK_MAJOR = 7, SX_STRIXW_Q6 = 8, SX_STRIXW_Q5 = 9
};
enum sx_strixw_role { SX_STRIXW_DATA = 0, SX_STRIXW_Q = 1, SX_STRIXW_SCALE = 2, SX_STRIXW_MIN = 3 };

typedef struct sx_strixw sx_strixw; /* an open, validated file (read-only mapping) */

/* StrixwComponent (formats/strixw.hpp:30-33): offset absolute in the file. */
typedef struct sx_strixw_component {
    uint8_t role;
    uint64_t offset, bytes, hash;
} sx_strixw_component;

/* StrixwTensor (formats/strixw.hpp:35-44); name points into the open file and lives as long as it. */
typedef struct sx_strixw_tensor {
    const char *name;
    int32_t encoding, ndim;
    int64_t shape[8];
    int64_t group_size, experts;
    int32_t nparts, ncomp;
    sx_strixw_component comp[4];
} sx_strixw_tensor;

/* strix_hash64 (formats/strixw.hpp:50): the file's 64-bit checksum of n bytes (host memory). */
uint64_t sx_strix_hash64(const void *data, uint64_t n);
/* StrixwFile::StrixwFile (formats/strixw.hpp:88): maps path and validates the header, the index and every record
 * (the same checks, in the same order, as formats/strixw.cpp:398-500); on failure SX_EINVAL with a message naming the
 * file and the problem ("bad magic", "header hash mismatch", "truncated", "components overlap", ...), *out NULL.
 * Host only: no HIP call. */
int sx_strixw_open(const char *path, sx_strixw **out);
void sx_strixw_close(sx_strixw *f);
/* version, file_bytes, data_offset, tensor and metadata counts (any pointer may be NULL). */
int sx_strixw_summary(const sx_strixw *f, uint32_t *version, uint64_t *file_bytes, uint64_t *data_offset,
                      int64_t *tensors, int64_t *meta);
/* StrixwFile::meta() (formats/strixw.hpp:95-96): the i-th pair in the file's key order, or the value of `key`
 * (SX_EINVAL naming the file when absent). Strings live as long as the file. */
int sx_strixw_meta_at(const sx_strixw *f, int64_t i, const char **key, const char **value);
int sx_strixw_meta(const sx_strixw *f, const char *key, const char **value);
/* StrixwFile::find / tensors() (formats/strixw.hpp:97-98): *index = the record's position, or -1 when absent. */
int sx_strixw_find(const sx_strixw *f, const char *name, int64_t *index);
int sx_strixw_tensor_at(const sx_strixw *f, int64_t i, sx_strixw_tensor *out);
/* StrixwPart (formats/strixw.hpp:25-28) of a record: the checkpoint tensor and the rows it fills. */
int sx_strixw_part_at(const sx_strixw *f, int64_t tensor, int64_t part, const char **source, int64_t *row_offset,
                      int64_t *rows);
/* StrixwFile::verify_hashes (formats/strixw.hpp:102): rehashes every component on `threads` host threads; SX_EINVAL
 * naming the first corrupt component in file order. */
int sx_strixw_verify_hashes(const sx_strixw *f, int threads);
/* StrixwDevice::StrixwDevice (runtime/strixw_loader.hpp:27): copies the data region (file_bytes - data_offset bytes)
 * to dst (device memory of at least that size, 256-byte aligned, owned by the caller) through pinned staging slots
 * filled by read_threads (1..64) concurrent pread()s, the copies queued on `stream`. Synchronous: returns once the
 * region is on the device; *seconds (may be NULL) = wall time. Component hashes are not rechecked (the header and
 * index hashes were, at open). */
int sx_strixw_load(const sx_strixw *f, void *dst, uint64_t dst_bytes, int read_threads, double *seconds,
                   sx_stream stream);
/* StrixwDevice::q4 / q8 / qw (runtime/strixw_loader.hpp:36-41): the view of a row-major q4 (bits 4), q8 (8) or either
 * (0) tensor of shape [N, K], checked, with pointers into the region loaded at `base` (base + offset - data_offset),
 * or into the file's mapping when base is NULL. */
int sx_strixw_qview(const sx_strixw *f, const void *base, const char *name, int bits, int64_t N, int64_t K,
                    sx_qview *out);
/* StrixwDevice::bf16 / f32 (runtime/strixw_loader.hpp:46-47), and i64: a dense tensor's data, encoding and shape
 * checked; base as for sx_strixw_qview. */
int sx_strixw_data(const sx_strixw *f, const void *base, const char *name, int encoding, const int64_t *shape,
                   int ndim, const void **out);

/* ---------------- measurement probes (no counterpart in the reference: the ceilings the roofline fractions are
 * judged against, measured on the part) ---------------- */
/* A streaming read of `bytes` (16-byte aligned) by `blocks` blocks of 512 threads, 16-byte loads, nothing stored
 * (sink: 4 bytes, written only in a case the data practically never gives). */
int sx_probe_stream_read(const void *buf, uint64_t bytes, int blocks, uint32_t *sink, sx_stream stream);
/* `blocks` blocks of 4 waves, each wave `iters` x 4 independent v_mfma_f32_32x32x16_bf16; *flops (may be NULL) = the
 * launch's dense BF16 flops. */
int sx_probe_mfma(int blocks, int iters, float *sink, double *flops, sx_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* STRIXITE_AMD_H */
