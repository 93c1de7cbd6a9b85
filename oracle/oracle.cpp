// CPU oracle (test infrastructure only): a restatement of the reference's verify-path algorithms. See oracle.h for
// what each function follows; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this.
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <random>
#include <thread>
#include <utility>
#include <vector>

namespace {

float bf16f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Round to nearest even, NaN kept quiet (the store rounding of formats/q4.cpp:12-19 and the kernels).
uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0x007fffffu) ? 0x0040u : 0u));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float load_act(const void *p, int64_t i, int act) {
    return act == OR_ACT_F32 ? static_cast<const float *>(p)[i] : bf16f(static_cast<const uint16_t *>(p)[i]);
}
void store_act(void *p, int64_t i, float v, int act) {
    if (act == OR_ACT_F32) static_cast<float *>(p)[i] = v;
    else static_cast<uint16_t *>(p)[i] = to_bf16(v);
}
float as_stored(float v, int act) { return act == OR_ACT_F32 ? v : bf16f(to_bf16(v)); }

int hw_threads(int threads) {
    if (threads > 0) return threads;
    unsigned n = std::thread::hardware_concurrency();
    return n ? (int)n : 1;
}

// Runs f(i) for i in [0, n) over `threads` threads (dynamic chunks).
template <typename F>
void parallel_for(int64_t n, int threads, F f) {
    threads = hw_threads(threads);
    if (threads <= 1 || n < 2) {
        for (int64_t i = 0; i < n; ++i) f(i);
        return;
    }
    std::atomic<int64_t> next{0};
    const int64_t chunk = std::max<int64_t>(1, n / (threads * 16));
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t)
        pool.emplace_back([&] {
            for (;;) {
                const int64_t b = next.fetch_add(chunk);
                if (b >= n) break;
                const int64_t e = std::min(n, b + chunk);
                for (int64_t i = b; i < e; ++i) f(i);
            }
        });
    for (auto &th : pool) th.join();
}

int code_at(int bits, const uint8_t *q, int64_t K, int64_t n, int64_t k) {
    if (bits == 8) return q[n * K + k];
    return (q[(n * K + k) / 2] >> ((k & 1) ? 4 : 0)) & 0xF;  // formats/q4.hpp:4: low nibble = even k
}

// One dequantized row, exactly as formats/q4.cpp:121-134 / q8.cpp:117-127 compute it: (float)code * s, then + m,
// two separately rounded FP32 operations.
void dequant_row(int bits, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t K, int64_t G,
                 int64_t n, float *w) {
    const int64_t groups = K / G;
    for (int64_t k = 0; k < K; ++k) {
        const int64_t gi = n * groups + k / G;
        volatile float prod = (float)code_at(bits, q, K, n, k) * bf16f(scale[gi]);  // volatile: no contraction
        w[k] = prod + bf16f(minv[gi]);
    }
}

// sum_k x_k * w_k in double (the closed form; differs from any FP32 kernel only by rounding).
double dot_d(const double *x, const float *w, int64_t K) {
    double s = 0;
    for (int64_t k = 0; k < K; ++k) s += x[k] * (double)w[k];
    return s;
}

std::vector<double> widen(const void *x, int64_t off, int64_t K, int act) {
    std::vector<double> v((size_t)K);
    for (int64_t k = 0; k < K; ++k) v[(size_t)k] = load_act(x, off + k, act);
    return v;
}

float silu(float v) { return v / (1.0f + std::exp(-v)); }  // kernels/swiglu.hip:19's form

bool id_ok(int32_t id, int64_t E) { return id >= 0 && id < E; }

void flag(uint32_t *err, uint32_t a, uint32_t b) {
    if (err && err[0] == 0) err[0] = 1, err[1] = a, err[2] = b;
}

const float kNaN = std::numeric_limits<float>::quiet_NaN();
const float kInf = std::numeric_limits<float>::infinity();

// Candidate order of serve/sampler.cpp:114-116 and kernels/logits_topk.hpp:5: value descending, lower id first.
bool better(const std::pair<float, int32_t> &a, const std::pair<float, int32_t> &b) {
    return a.first != b.first ? a.first > b.first : a.second < b.second;
}

}  // namespace

struct or_rng {
    std::mt19937_64 g;
};

extern "C" {

float or_bf16_to_f32(uint16_t b) { return bf16f(b); }
uint16_t or_f32_to_bf16(float f) { return to_bf16(f); }

void or_dequant(int bits, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K,
                int64_t G, float *out) {
    for (int64_t n = 0; n < N; ++n) dequant_row(bits, q, scale, minv, K, G, n, out + n * K);
}

int or_quantize_q4(const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale, uint16_t *minv) {
    const int64_t groups = K / G;
    std::memset(q, 0, (size_t)(N * K / 2));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t g = 0; g < groups; ++g) {
            const float *grp = w + n * K + g * G;
            float lo = grp[0], hi = grp[0];
            for (int64_t i = 0; i < G; ++i) {
                if (!std::isfinite(grp[i])) return 1;
                lo = std::fmin(lo, grp[i]);
                hi = std::fmax(hi, grp[i]);
            }
            const uint16_t sb = to_bf16((hi - lo) / 15.0f), mb = to_bf16(lo);
            const float s = bf16f(sb), m = bf16f(mb);
            scale[n * groups + g] = sb, minv[n * groups + g] = mb;
            for (int64_t i = 0; i < G; ++i) {
                int code = 0;
                if (s > 0.0f) code = (int)std::fmin(std::fmax(std::nearbyint((grp[i] - m) / s), 0.0f), 15.0f);
                const int64_t k = g * G + i;
                q[(n * K + k) / 2] |= (uint8_t)(code << ((k & 1) ? 4 : 0));
            }
        }
    return 0;
}

int or_q4_from_q8(const uint8_t *q8, const uint16_t *s8, const uint16_t *m8, int64_t N, int64_t K, int64_t G8,
                  int64_t G4, uint8_t *q4, uint16_t *s4, uint16_t *m4, int threads) {
    std::atomic<int> bad{0};
    parallel_for(N, threads, [&](int64_t n) {
        std::vector<float> w((size_t)K);
        dequant_row(8, q8, s8, m8, K, G8, n, w.data());
        // row n of the result: its own slice of each output array (groups run along K inside a row)
        if (or_quantize_q4(w.data(), 1, K, G4, q4 + n * K / 2, s4 + n * (K / G4), m4 + n * (K / G4))) bad = 1;
    });
    return bad.load();
}

void or_linear_q(int bits, const void *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N,
                 int64_t K, int64_t G, void *y, int64_t M, int act, int out_act, int threads) {
    std::vector<std::vector<double>> xs;
    for (int64_t m = 0; m < M; ++m) xs.push_back(widen(x, m * K, K, act));
    parallel_for(N, threads, [&](int64_t n) {
        std::vector<float> w((size_t)K);
        dequant_row(bits, q, scale, minv, K, G, n, w.data());
        for (int64_t m = 0; m < M; ++m) store_act(y, m * N + n, (float)dot_d(xs[(size_t)m].data(), w.data(), K), out_act);
    });
}

void or_linear_f32w(const void *x, const float *W, int64_t N, int64_t K, float *y, int64_t M, int act, int threads) {
    std::vector<std::vector<double>> xs;
    for (int64_t m = 0; m < M; ++m) xs.push_back(widen(x, m * K, K, act));
    parallel_for(N, threads, [&](int64_t n) {
        for (int64_t m = 0; m < M; ++m) y[m * N + n] = (float)dot_d(xs[(size_t)m].data(), W + n * K, K);
    });
}

void or_linear_bf16w(const void *x, const uint16_t *W, int64_t N, int64_t K, void *y, int64_t M, int act,
                     int out_act, int threads) {
    std::vector<std::vector<double>> xs;
    for (int64_t m = 0; m < M; ++m) xs.push_back(widen(x, m * K, K, act));
    parallel_for(N, threads, [&](int64_t n) {
        std::vector<float> w((size_t)K);
        for (int64_t k = 0; k < K; ++k) w[(size_t)k] = bf16f(W[n * K + k]);
        for (int64_t m = 0; m < M; ++m) store_act(y, m * N + n, (float)dot_d(xs[(size_t)m].data(), w.data(), K), out_act);
    });
}

void or_moe_shared_add(void *y, const void *s, const float *gate_logit, int64_t gate_ld, int64_t M, int64_t N,
                       uint32_t gate_index, void *x, const float *w_in, int64_t H, int act, uint32_t *err) {
    for (int64_t m = 0; m < M; ++m) {
        const float gl = gate_logit[m * gate_ld];
        const bool ok = std::isfinite(gl);
        if (!ok) flag(err, (uint32_t)m, gate_index);
        const float g = ok ? 1.f / (1.f + std::exp(-gl)) : kNaN;
        for (int64_t n = 0; n < N; ++n) {
            // y + g * s as one fused multiply-add (the kernel's expression under HIP's default contraction)
            const float v = as_stored(std::fma(g, load_act(s, m * N + n, act), load_act(y, m * N + n, act)), act);
            store_act(y, m * N + n, v, act);
            if (x != nullptr)
                for (int64_t st = 0; st < H; ++st) {
                    const int64_t xi = (m * H + st) * N + n;
                    store_act(x, xi, std::fma(w_in[m * H + st], v, load_act(x, xi, act)), act);
                }
        }
    }
}

int or_moe_router(const float *logits, int64_t ld, int64_t M, int64_t E, int64_t k, const float *shared,
                  int64_t shared_ld, int32_t shared_id, int32_t *ids, float *coef, uint32_t *err) {
    const int64_t A = k + (shared ? 1 : 0);
    for (int64_t m = 0; m < M; ++m) {
        const float *row = logits + m * ld;
        // moe_router.hip:40-68: the lowest non-finite expert index (E = the shared gate) fails the token.
        int64_t bad = -1;
        for (int64_t e = 0; e < E && bad < 0; ++e)
            if (!std::isfinite(row[e])) bad = e;
        if (bad < 0 && shared && !std::isfinite(shared[m * shared_ld])) bad = E;
        if (bad >= 0) {
            flag(err, (uint32_t)m, (uint32_t)bad);
            for (int64_t a = 0; a < A; ++a) ids[m * A + a] = -1, coef[m * A + a] = kNaN;
            continue;
        }
        std::vector<std::pair<float, int32_t>> c((size_t)E);
        for (int64_t e = 0; e < E; ++e) c[(size_t)e] = {row[e], (int32_t)e};
        std::stable_sort(c.begin(), c.end(), better);
        const float top = c[0].first;
        float sum = 0;
        std::vector<float> ex((size_t)k);
        for (int64_t j = 0; j < k; ++j) sum += ex[(size_t)j] = std::exp(c[(size_t)j].first - top);
        for (int64_t j = 0; j < k; ++j) ids[m * A + j] = c[(size_t)j].second, coef[m * A + j] = ex[(size_t)j] / sum;
        if (shared) ids[m * A + k] = shared_id, coef[m * A + k] = 1.0f / (1.0f + std::exp(-shared[m * shared_ld]));
    }
    return err ? (int)err[0] : 0;
}

void or_experts_gather(int bits, const void *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv,
                       int64_t Nall, int64_t K, int64_t G, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                       void *y, int act, uint32_t *err, int threads) {
    const int64_t N = Nall / E;
    for (int64_t s = 0; s < M * A; ++s)
        if (!id_ok(ids[s], E)) flag(err, (uint32_t)ids[s], (uint32_t)s);
    parallel_for(M * A, threads, [&](int64_t s) {
        const int32_t id = ids[s];
        if (!id_ok(id, E)) {
            for (int64_t n = 0; n < N; ++n) store_act(y, s * N + n, kNaN, act);
            return;
        }
        const std::vector<double> xv = widen(x, (s / A) * K, K, act);
        std::vector<float> w((size_t)K);
        for (int64_t n = 0; n < N; ++n) {
            dequant_row(bits, q, scale, minv, K, G, (int64_t)id * N + n, w.data());
            store_act(y, s * N + n, (float)dot_d(xv.data(), w.data(), K), act);
        }
    });
}

void or_experts_gather_swiglu(int bits, const void *x, const uint8_t *q, const uint16_t *scale, const uint16_t *minv,
                              int64_t Nall, int64_t K, int64_t G, int64_t E, const int32_t *ids, int64_t M, int64_t A,
                              void *h, int act, uint32_t *err, int threads) {
    const int64_t N = Nall / E, I = N / 2;
    for (int64_t s = 0; s < M * A; ++s)
        if (!id_ok(ids[s], E)) flag(err, (uint32_t)ids[s], (uint32_t)s);
    parallel_for(M * A, threads, [&](int64_t s) {
        const int32_t id = ids[s];
        if (!id_ok(id, E)) {
            for (int64_t j = 0; j < I; ++j) store_act(h, s * I + j, kNaN, act);
            return;
        }
        const std::vector<double> xv = widen(x, (s / A) * K, K, act);
        std::vector<float> wg((size_t)K), wu((size_t)K);
        for (int64_t j = 0; j < I; ++j) {
            dequant_row(bits, q, scale, minv, K, G, (int64_t)id * N + j, wg.data());
            dequant_row(bits, q, scale, minv, K, G, (int64_t)id * N + I + j, wu.data());
            // linear_q4.hip:227-231: g and u as stored, then swiglu's rounding points.
            const float g = as_stored((float)dot_d(xv.data(), wg.data(), K), act);
            const float u = as_stored((float)dot_d(xv.data(), wu.data(), K), act);
            store_act(h, s * I + j, as_stored(silu(g), act) * u, act);
        }
    });
}

void or_experts_combine(int bits, const void *h, const uint8_t *q, const uint16_t *scale, const uint16_t *minv,
                        int64_t Nall, int64_t K, int64_t G, int64_t E, const int32_t *ids, const float *coef,
                        int64_t M, int64_t A, void *y, int act, uint32_t *err, int threads) {
    const int64_t N = Nall / E;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t a = 0; a < A; ++a)
            if (!id_ok(ids[m * A + a], E)) {
                flag(err, (uint32_t)ids[m * A + a], (uint32_t)(m * A + a));
                break;
            }
    parallel_for(M, threads, [&](int64_t m) {
        bool ok = true;
        for (int64_t a = 0; a < A; ++a) ok = ok && id_ok(ids[m * A + a], E);
        if (!ok) {
            for (int64_t n = 0; n < N; ++n) store_act(y, m * N + n, kNaN, act);
            return;
        }
        std::vector<std::vector<double>> hs;
        for (int64_t a = 0; a < A; ++a) hs.push_back(widen(h, (m * A + a) * K, K, act));
        std::vector<float> w((size_t)K);
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0;
            for (int64_t a = 0; a < A; ++a) {
                dequant_row(bits, q, scale, minv, K, G, (int64_t)ids[m * A + a] * N + n, w.data());
                acc += (double)coef[m * A + a] * dot_d(hs[(size_t)a].data(), w.data(), K);
            }
            store_act(y, m * N + n, (float)acc, act);
        }
    });
}

void or_swiglu(const void *gu, void *h, int64_t rows, int64_t I, int act) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < I; ++j) {
            const float g = load_act(gu, r * 2 * I + j, act), u = load_act(gu, r * 2 * I + I + j, act);
            store_act(h, r * I + j, as_stored(silu(g), act) * u, act);
        }
}

void or_logits_topk(const float *logits, int64_t rows, int64_t ld, int64_t n_valid, int64_t k, const uint32_t *mask,
                    int64_t mask_words, float *out_v, int32_t *out_id, uint32_t *nan) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = logits + r * ld;
        std::vector<std::pair<float, int32_t>> c;
        uint32_t f = 0;
        for (int64_t i = 0; i < n_valid; ++i) {
            const float v = row[i];
            if (v != v) {
                f = 1;  // flagged whether the id is allowed or not (logits_topk.hip:118-121)
                continue;
            }
            if (mask && !((mask[r * mask_words + (i >> 5)] >> (i & 31)) & 1u)) continue;
            c.push_back({v, (int32_t)i});  // -0 == +0 under better(): the lower id wins the tie
        }
        std::stable_sort(c.begin(), c.end(), better);
        for (int64_t j = 0; j < k; ++j) {
            const bool real = j < (int64_t)c.size();
            out_v[r * k + j] = real ? c[(size_t)j].first : -kInf;
            out_id[r * k + j] = real ? c[(size_t)j].second : std::numeric_limits<int32_t>::max();
        }
        nan[r] = f;
    }
}

void or_top2(const float *x, int64_t n, int32_t *best, float *best_v, float *second_v, uint32_t *nan) {
    int32_t b = -1;
    float b1 = -kInf, b2 = -kInf;
    uint32_t f = 0;
    for (int64_t i = 0; i < n; ++i) {
        const float v = x[i];
        if (v != v) {
            f = 1;
            continue;
        }
        if (b < 0 || v > b1) b2 = b < 0 ? -kInf : b1, b1 = v, b = (int32_t)i;
        else if (v > b2) b2 = v;
    }
    *best = b < 0 ? 0 : b;  // every logit NaN: 0, flagged (mtp_pick.hip:99)
    *best_v = b1, *second_v = b2, *nan = f;
}

or_rng *or_rng_new(uint64_t seed) { return new or_rng{std::mt19937_64(seed)}; }
void or_rng_free(or_rng *r) { delete r; }
double or_rng_canonical(or_rng *r) { return std::generate_canonical<double, 53>(r->g); }

}  // extern "C"

namespace {

// serve/sampler.cpp:216-248: softmax at the temperature over the sorted candidates c[0, k), top-p, then the draw.
// Returns -1 when the top logit is not finite.
int32_t draw(or_rng *r, const std::vector<std::pair<float, int32_t>> &c, int64_t k, double T, double top_p) {
    if (!std::isfinite(c[0].first)) return -1;
    std::vector<double> prob((size_t)k);
    const double top = c[0].first / T;
    double sum = 0;
    for (int64_t i = 0; i < k; ++i) sum += prob[(size_t)i] = std::exp(c[(size_t)i].first / T - top);
    int64_t keep = k;
    if (top_p < 1) {
        double acc = 0;
        for (int64_t i = 0; i < k; ++i) {
            acc += prob[(size_t)i] / sum;
            if (acc >= top_p) {
                keep = i + 1;
                break;
            }
        }
    }
    double kept = 0;
    for (int64_t i = 0; i < keep; ++i) kept += prob[(size_t)i];
    const double u = std::uniform_real_distribution<double>(0, kept)(r->g);
    double acc = 0;
    for (int64_t i = 0; i < keep; ++i) {
        acc += prob[(size_t)i];
        if (u < acc) return c[(size_t)i].second;
    }
    return c[(size_t)(keep - 1)].second;
}

// serve/sampler.cpp:276-328 (top_k off): every id a candidate, the sorted order's prefix sums, the index-order sum.
int32_t draw_all(or_rng *r, const float *x, int64_t n, double T, double top_p) {
    float top = -kInf;
    for (int64_t i = 0; i < n; ++i) top = std::max(top, x[i]);
    if (!std::isfinite(top)) return -1;
    std::vector<double> p((size_t)n);
    const double t_top = top / T;
    double sum = 0;
    for (int64_t i = 0; i < n; ++i) sum += p[(size_t)i] = std::exp(x[i] / T - t_top);
    std::vector<std::pair<float, int32_t>> c((size_t)n);
    for (int64_t i = 0; i < n; ++i) c[(size_t)i] = {x[i], (int32_t)i};
    std::stable_sort(c.begin(), c.end(), better);
    if (top_p < 1) {
        size_t keep = c.size();
        double acc = 0;
        for (size_t j = 0; j < c.size(); ++j) {
            acc += p[(size_t)c[j].second] / sum;
            if (acc >= top_p) {
                keep = j + 1;
                break;
            }
        }
        double kept = 0;
        for (size_t j = 0; j < keep; ++j) kept += p[(size_t)c[j].second];
        const double u = std::uniform_real_distribution<double>(0, kept)(r->g);
        acc = 0;
        for (size_t j = 0; j < keep; ++j) {
            acc += p[(size_t)c[j].second];
            if (u < acc) return c[j].second;
        }
        return c[keep - 1].second;
    }
    const double u = std::uniform_real_distribution<double>(0, sum)(r->g);
    double acc = 0;
    for (size_t j = 0; j < c.size(); ++j) {
        acc += p[(size_t)c[j].second];
        if (u < acc) return c[j].second;
    }
    return c.back().second;
}

}  // namespace

extern "C" {

int32_t or_sample_row(or_rng *r, const float *x, int64_t n, double T, int64_t top_k, double top_p) {
    for (int64_t i = 0; i < n; ++i)
        if (x[i] != x[i]) return -1;  // sampler.cpp:109, 155, 263, 286: a NaN anywhere fails the row
    if (T == 0) {
        int32_t b;
        float bv, sv;
        uint32_t f;
        or_top2(x, n, &b, &bv, &sv, &f);
        return b;
    }
    const int64_t k = top_k > 0 ? std::min<int64_t>(top_k, n) : n;
    if (k == n) return draw_all(r, x, n, T, top_p);
    std::vector<std::pair<float, int32_t>> c((size_t)n);
    for (int64_t i = 0; i < n; ++i) c[(size_t)i] = {x[i], (int32_t)i};
    std::partial_sort(c.begin(), c.begin() + k, c.end(), better);  // total order: same head as a full stable sort
    return draw(r, c, k, T, top_p);
}

int64_t or_accept(or_rng *r, const float *logits, int64_t k, int64_t row_len, int64_t n_valid, const int32_t *drafts,
                  double temperature, int64_t top_k, double top_p, int32_t *sampled, int32_t *status) {
    *status = 0;
    // serve/engine.cpp:592-598: sample row j, stop at the first draft that differs. Row k (all accepted) is the next
    // token's row: its sample (engine.cpp:540 on the next step) is drawn here too, so j + 1 tokens come out.
    for (int64_t j = 0; j <= k; ++j) {
        const int32_t v = or_sample_row(r, logits + j * row_len, n_valid, temperature, top_k, top_p);
        if (v < 0) {
            *status = (int32_t)(1 + j);
            return j;
        }
        sampled[j] = v;
        if (j == k || v != drafts[j]) return j;
    }
    return k;
}

}  // extern "C"

uint64_t or_strix_hash64(const uint8_t *p, uint64_t n) {
    const uint64_t A = 0x9e3779b97f4a7c15ull, B = 0xd6e8feb86659fd93ull;
    auto absorb = [&](uint64_t h, uint64_t w) {
        const uint64_t x = h ^ (w * A);
        return (x ^ (x >> 31)) * B;
    };
    uint64_t lanes[4] = {n ^ A, n ^ B, ~n ^ A, ~n ^ B};
    const uint64_t words = n / 8;
    for (uint64_t i = 0; i < words; ++i) {
        uint64_t w = 0;
        for (int b = 7; b >= 0; --b) w = (w << 8) | p[8 * i + b];
        lanes[i % 4] = absorb(lanes[i % 4], w);
    }
    const uint64_t rest = n - 8 * words;
    if (rest) {
        uint64_t w = rest << 56;
        for (uint64_t b = 0; b < rest; ++b) w ^= (uint64_t)p[8 * words + b] << (8 * b);
        lanes[0] = absorb(lanes[0], w);
    }
    uint64_t r = lanes[0];
    for (int l = 1; l < 4; ++l) r = absorb(r, lanes[l]);
    r ^= r >> 33;
    r *= A;
    return r ^ (r >> 29);
}
