// extern "C" entry points over the reference's own host code (formats/q4.cpp, q8.cpp, q4_from_q8.cpp, serve/sampler.cpp),
// compiled from /root/reference by oracle/Makefile into oracle/_ref/libstrix_ref.so. Test infrastructure only: it is
// the reference itself, used to pin the oracle restatement and to write the fixtures under tests/golden/.
#include "formats/q4.hpp"
#include "formats/q4_from_q8.hpp"
#include "formats/q8.hpp"
#include "serve/sampler.hpp"

#include <cstring>
#include <exception>

extern "C" {

// formats/q4.hpp:35 / q8.hpp:31 quantize, then :45 / :39 dequantize. Returns 0, or 1 if the reference threw.
int ref_quantize(int bits, const float *w, int64_t N, int64_t K, int64_t G, uint8_t *q, uint16_t *scale,
                 uint16_t *minv, float *deq) {
    try {
        if (bits == 4) {
            const strix::Q4Weight r = strix::quantize_q4(w, N, K, G);
            std::memcpy(q, r.q.data(), r.q.size());
            std::memcpy(scale, r.scale.data(), 2 * r.scale.size());
            std::memcpy(minv, r.minv.data(), 2 * r.minv.size());
            const std::vector<float> d = strix::dequantize_q4(r);
            std::memcpy(deq, d.data(), 4 * d.size());
        } else {
            const strix::Q8Weight r = strix::quantize_q8(w, N, K, G);
            std::memcpy(q, r.q.data(), r.q.size());
            std::memcpy(scale, r.scale.data(), 2 * r.scale.size());
            std::memcpy(minv, r.minv.data(), 2 * r.minv.size());
            const std::vector<float> d = strix::dequantize_q8(r);
            std::memcpy(deq, d.data(), 4 * d.size());
        }
        return 0;
    } catch (const std::exception &) {
        return 1;
    }
}

// formats/q4_from_q8.hpp:23 quantize_q4_from_q8 on a caller-supplied Q8 weight; the Q4 result's arrays into q4, s4,
// m4. Returns 0, or 1 if the reference threw.
int ref_q4_from_q8(const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K, int64_t G8,
                   int64_t G4, int threads, uint8_t *q4, uint16_t *s4, uint16_t *m4) {
    try {
        strix::Q8Weight w;
        w.N = N, w.K = K, w.G = G8;
        const size_t groups = (size_t)(N * (K / G8));
        w.q.assign(q, q + N * K), w.scale.assign(scale, scale + groups), w.minv.assign(minv, minv + groups);
        const strix::Q4Weight r = strix::quantize_q4_from_q8(w, G4, threads);
        std::memcpy(q4, r.q.data(), r.q.size());
        std::memcpy(s4, r.scale.data(), 2 * r.scale.size());
        std::memcpy(m4, r.minv.data(), 2 * r.minv.size());
        return 0;
    } catch (const std::exception &) {
        return 1;
    }
}

// formats dequantize on caller-supplied codes (no quantize step).
int ref_dequantize(int bits, const uint8_t *q, const uint16_t *scale, const uint16_t *minv, int64_t N, int64_t K,
                   int64_t G, float *deq) {
    try {
        const size_t groups = (size_t)(N * (K / G));
        std::vector<float> d;
        if (bits == 4) {
            strix::Q4Weight w;
            w.N = N, w.K = K, w.G = G;
            w.q.assign(q, q + N * K / 2), w.scale.assign(scale, scale + groups), w.minv.assign(minv, minv + groups);
            d = strix::dequantize_q4(w);
        } else {
            strix::Q8Weight w;
            w.N = N, w.K = K, w.G = G;
            w.q.assign(q, q + N * K), w.scale.assign(scale, scale + groups), w.minv.assign(minv, minv + groups);
            d = strix::dequantize_q8(w);
        }
        std::memcpy(deq, d.data(), 4 * d.size());
        return 0;
    } catch (const std::exception &) {
        return 1;
    }
}

// serve/sampler.hpp:29 top2.
void ref_top2(const float *x, int64_t n, int32_t *best, float *best_v, float *second_v, uint32_t *nan) {
    const strix::Top2 t = strix::top2(x, n);
    *best = t.best, *best_v = t.best_v, *second_v = t.second_v, *nan = t.nan ? 1u : 0u;
}

void *ref_sampler_new(double temperature, int64_t top_k, double top_p, uint64_t seed, int64_t n_valid) {
    try {
        return new strix::Sampler(strix::SamplingParams{temperature, top_k, top_p, seed}, n_valid);
    } catch (const std::exception &) {
        return nullptr;
    }
}
void ref_sampler_free(void *s) { delete static_cast<strix::Sampler *>(s); }

// Sampler::sample on a full row; -1 if it threw (NaN row, non-finite top logit).
int32_t ref_sampler_sample(void *s, const float *logits, int64_t size) {
    try {
        return static_cast<strix::Sampler *>(s)->sample(logits, (size_t)size);
    } catch (const std::exception &) {
        return -1;
    }
}

// Sampler::sample_candidates (top_k <= kCandidates); -1 if it threw.
int32_t ref_sampler_sample_candidates(void *s, const float *v, const int32_t *id, int64_t m, int nan) {
    try {
        return static_cast<strix::Sampler *>(s)->sample_candidates(v, id, m, nan != 0);
    } catch (const std::exception &) {
        return -1;
    }
}

}  // extern "C"
