/* CPU oracle for strixite's MTP verify path: a plain restatement of the reference's algorithms, used ONLY as the
 * checker (tests/, __graft_entry__.smoke, bench.py's cpu_baseline leg). Nothing in the product library calls it.
 *
 * Every function cites the reference file:line it restates. Floating-point outputs are computed in double (the
 * closed form sum_k x_k * deq(w)_k) and rounded once at the store, so they differ from the GPU only by summation
 * order; integer outputs (expert ids, token ids, accepted lengths) are exact.
 *
 * Parity pins (tests/test_oracle.py): dequant vs fixtures from the compiled reference formats/q4.cpp + q8.cpp;
 * linear vs brute force and basis vectors; router / top-k vs a full stable sort; top2 and the sampler / accept loop
 * vs fixtures from the compiled reference serve/sampler.cpp. */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_ACT_F32 = 0, OR_ACT_BF16 = 1 };

float or_bf16_to_f32(uint16_t b);
uint16_t or_f32_to_bf16(float f);

/* formats/q4.cpp:121-134, formats/q8.cpp:117-127: w = code * scale + min, each step rounded (no FMA). */
void or_dequant(int bits, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K,
                int64_t G, float *out);

/* formats/q4.cpp:44-86 quantize_q4 on finite FP32 w [N, K]: per group lo/hi, s = bf16((hi - lo) / 15),
 * m = bf16(lo), code = clamp(nearbyint((w - m) / s), 0, 15) (0 when s = 0). Returns 0, or 1 on a non-finite weight. */
int or_quantize_q4(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv);

/* formats/q4_from_q8.cpp:34-86: a Q8 weight's rows dequantized exactly (q8.cpp:117-127), then quantize_q4 with group
 * G4. Returns 0, or 1 on a non-finite dequantized value. */
int or_q4_from_q8(const uint8_t *q8, const uint16_t *s8, const uint16_t *m8, int64_t N, int64_t K, int64_t G8,
                  int64_t G4, uint8_t *q4, uint16_t *s4, uint16_t *m4, int threads);

/* kernels/linear_q4.hpp:26-30, linear_q8.hpp:13-14: y[M,N] = x[M,K] * deq(W)^T, x in act, y in out_act.
 * threads <= 0: all hardware threads. */
void or_linear_q(int bits, const void *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N,
                 int64_t K, int64_t G, void *y, int64_t M, int act, int out_act, int threads);

/* Dense FP32-weight projection (the router logits of the MoE configs): y[M,N] f32 = x[M,K] (act) * W[N,K]^T. */
void or_linear_f32w(const void *x, const float *W, int64_t N, int64_t K, float *y, int64_t M, int act, int threads);

/* kernels/linear.hpp:14-24 (linear_bf16w; kernels/linear.hip:176-204): y[M,N] = x[M,K] (act) * W^T, W BF16 bits [N, K],
 * FP32-or-better accumulation (here double), one rounding to out_act (act, or BF16 -> F32). */
void or_linear_bf16w(const void *x, const uint16_t *W, int64_t N, int64_t K, void *y, int64_t M, int act,
                     int out_act, int threads);

/* kernels/moe_router.hpp:45-63, moe_router.hip:127-180: y[m,:] = stored(fma(sigmoid(gate_logit[m*gate_ld]), s, y)); a
 * non-finite gate logit: the row NaN, err {1, m, gate_index} (first wins). x != NULL: then each of the H streams
 * x[m, st*N + n] = fma(w_in[m*H + st], y_stored, x) rounded once (moe_shared_add_inject). */
void or_moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                       uint32_t gate_index, void *x, const float *w_in, int64_t H, int act, uint32_t *err);

/* kernels/moe_router.hpp:11-40: per token the top k of E logits (value desc, index asc), coef = softmax over the k;
 * optional shared slot (sigmoid). Non-finite logit: ids -1, coef NaN, err {1, token, expert}. Returns err[0]. */
int or_moe_router(const float *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const float *shared,
                  int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, uint32_t *err);

/* kernels/linear_q4.hpp:53-56 + swiglu.hip:22-37: h[m,a,j] = silu(g) * u over expert rows [gate | up];
 * BF16 act rounds g, u, silu(g) and h as the stores do. Bad id: err {1, id, slot}, that slot's h NaN. */
void or_experts_gather_swiglu(int bits, const void *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv,
                              int64_t Nall, int64_t K, int64_t G, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                              void *h, int act, uint32_t *err, int threads);

/* kernels/linear_q4.hpp:36-38 gather: y[m,a,:] = x[m,:] * W[ids[m,a]]^T (act dtype). */
void or_experts_gather(int bits, const void *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv,
                       int64_t Nall, int64_t K, int64_t G, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                       void *y, int act, uint32_t *err, int threads);

/* kernels/linear_q4.hpp:37-38 combine: y[m,:] = sum_a coef[m,a] * (h[m,a,:] * W[ids[m,a]]^T). A bad id in a
 * token's slots: that token's row NaN, err {1, id, slot}. */
void or_experts_combine(int bits, const void *h, const uint8_t *q, const uint16_t *scale, const uint16_t *minv,
                        int64_t Nall, int64_t K, int64_t G, int64_t E, const int32_t *ids, const float *coef,
                        int64_t M, int64_t A, void *y, int act, uint32_t *err, int threads);

/* kernels/swiglu.hpp:21, swiglu.hip:22-37. */
void or_swiglu(const void *gu, void *h, int64_t rows, int64_t I, int act);

/* kernels/logits_topk.hpp:3-9, 35-46 (k candidates instead of the fixed 20): per row the best k of ids [0, n_valid)
 * by (value desc, id asc), NaN left out and flagged, -0 ties +0, optional allow mask, padding (-inf, INT32_MAX). */
void or_logits_topk(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, int64_t k, const uint32_t *mask,
                    int64_t mask_words, float *out_v, int32_t *out_id, uint32_t *nan);

/* kernels/mtp_pick.hpp:3-8, mtp_pick.hip:17-74: over the non-NaN logits the best (lowest id on a tie), its value,
 * the multiset runner-up (-inf if none), and a NaN flag. Equal to serve/sampler.cpp:79-101 top2 on NaN-free rows. */
void or_top2(const float *x, int64_t n, int32_t *best, float *best_v, float *second_v, uint32_t *nan);

/* serve/sampler.cpp:103-161 + 216-248: Sampler::sample on a full row (temperature > 0 with top_k in 1..n-1, or
 * temperature 0), driving the caller's mt19937_64 state. Returns the id, or -1 on a sampler error (NaN row or
 * non-finite top logit). */
typedef struct or_rng or_rng;
or_rng *or_rng_new(uint64_t seed);
void or_rng_free(or_rng *r);
double or_rng_canonical(or_rng *r); /* std::generate_canonical<double, 53> as uniform_real_distribution draws it */
int32_t or_sample_row(or_rng *r, const float *logits, int64_t n_valid, double temperature, int64_t top_k,
                      double top_p);

/* serve/engine.cpp:592-610: accept drafts while the sampled token equals the draft. rows = k + 1 logits rows of
 * row_len floats, drafts [k]. Writes the sampled ids of the rows visited to sampled[] and returns the accepted
 * length j (0..k); *status = 0, or 1 + the row whose sampling failed (NaN). */
int64_t or_accept(or_rng *r, const float *logits, int64_t k, int64_t row_len, int64_t n_valid, const int32_t *drafts,
                  double temperature, int64_t top_k, double top_p, int32_t *sampled, int32_t *status);

// strix_hash64 (formats/strixw.cpp:253-274), restated word by word: the n / 8 whole little-endian 8-byte words go, in
// order, to lane (word index mod 4) - the reference's 32-byte blocks and then its leftover words land on the same
// lanes - each absorbed as lane = ((lane ^ w*A) ^ ((lane ^ w*A) >> 31)) * B; the 1..7 trailing bytes, zero-padded,
// with their count in the top byte, go to lane 0; the lanes start from n and ~n xor A / B and fold 0..3 in order,
// then r ^= r >> 33, r *= A, r ^= r >> 29.
uint64_t or_strix_hash64(const uint8_t *p, uint64_t n);

#ifdef __cplusplus
}
#endif
