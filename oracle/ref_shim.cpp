// extern "C" entry points over the reference's own host code (formats/q4.cpp, q8.cpp, q4_from_q8.cpp, strixw.cpp,
// serve/sampler.cpp),
// compiled from /root/reference by oracle/Makefile into oracle/_ref/libstrix_ref.so. Test infrastructure only: it is
// the reference itself, used to pin the oracle restatement and to write the fixtures under tests/golden/.
#include "formats/q4.hpp"
#include "formats/q4_from_q8.hpp"
#include "formats/q8.hpp"
#include "formats/strixw.hpp"
#include "serve/sampler.hpp"

#include <cstring>
#include <exception>
#include <map>
#include <sstream>
#include <stdexcept>
#include <string>

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

// ---- formats/strixw.cpp ----

uint64_t ref_strix_hash64(const void *p, uint64_t n) { return strix::strix_hash64(p, (size_t)n); }

namespace {
void put_msg(const std::string &m, char *msg, int64_t cap) {
    if (msg && cap > 0) {
        const size_t n = std::min<size_t>(m.size(), (size_t)cap - 1);
        std::memcpy(msg, m.data(), n);
        msg[n] = 0;
    }
}
std::vector<std::string> split_tabs(const std::string &line) {
    std::vector<std::string> f;
    size_t a = 0;
    for (size_t b; (b = line.find('\t', a)) != std::string::npos; a = b + 1) f.push_back(line.substr(a, b - a));
    f.push_back(line.substr(a));
    return f;
}
}  // namespace

// StrixwWriter on a plan given as text, one line each:
//   M <key> <value>
//   T <name> <encoding> <group> <experts> <ndim> <dims...> <nparts> (<source> <row_offset> <rows>)...
// (fields tab-separated), then each planned component written from `data` in plan order. Returns 0, or 1 with the
// reference's message in msg if it threw.
int ref_strixw_write(const char *path, const char *plan, const uint8_t *data, uint64_t data_bytes, char *msg,
                     int64_t cap) {
    try {
        std::map<std::string, std::string> meta;
        std::vector<strix::StrixwTensor> tensors;
        std::istringstream in(plan);
        for (std::string line; std::getline(in, line);) {
            if (line.empty()) continue;
            const std::vector<std::string> f = split_tabs(line);
            if (f[0] == "M") {
                meta[f.at(1)] = f.at(2);
                continue;
            }
            strix::StrixwTensor t;
            size_t i = 1;
            t.name = f.at(i++);
            t.encoding = (strix::StrixwEncoding)std::stoi(f.at(i++));
            t.group_size = std::stoll(f.at(i++));
            t.experts = std::stoll(f.at(i++));
            const int ndim = std::stoi(f.at(i++));
            for (int d = 0; d < ndim; ++d) t.shape.push_back(std::stoll(f.at(i++)));
            const int nparts = std::stoi(f.at(i++));
            for (int p = 0; p < nparts; ++p) {
                strix::StrixwPart part;
                part.source = f.at(i++);
                part.row_offset = std::stoll(f.at(i++));
                part.rows = std::stoll(f.at(i++));
                t.parts.push_back(part);
            }
            tensors.push_back(std::move(t));
        }
        strix::StrixwWriter w(path, meta, tensors);
        uint64_t at = 0;
        for (size_t ti = 0; ti < w.tensors().size(); ++ti)
            for (const strix::StrixwComponent &c : w.tensors()[ti].components) {
                if (at + c.bytes > data_bytes) throw std::runtime_error("ref_strixw_write: data too short");
                w.write(ti, c.role, data + at, (size_t)c.bytes);
                at += c.bytes;
            }
        w.finish();
        return 0;
    } catch (const std::exception &e) {
        put_msg(e.what(), msg, cap);
        return 1;
    }
}

// StrixwFile on path (and verify_hashes when threads > 0). Returns 0 with a listing of what was read in `dump`, or 1
// with the reference's message in msg. The listing: "H <version> <file bytes> <data offset>", "M <key> <value>", and
// per tensor "T <name> <enc> <group> <experts> <ndim> <dims> <nparts> <parts> <ncomp> (<role> <offset> <bytes>
// <hash>)..." (tab-separated, one line each).
int ref_strixw_read(const char *path, int threads, char *dump, int64_t dump_cap, char *msg, int64_t cap) {
    try {
        strix::StrixwFile f(path);
        if (threads > 0) f.verify_hashes(threads);
        std::ostringstream o;
        uint32_t version = 0;
        std::memcpy(&version, static_cast<const uint8_t *>(f.data(f.tensors()[0], f.tensors()[0].components[0].role)) -
                                  f.tensors()[0].components[0].offset + 8, 4);
        o << "H\t" << version << "\t" << f.file_bytes() << "\t" << f.data_offset() << "\n";
        for (const auto &[k, v] : f.meta()) o << "M\t" << k << "\t" << v << "\n";
        for (const strix::StrixwTensor &t : f.tensors()) {
            o << "T\t" << t.name << "\t" << (int)t.encoding << "\t" << t.group_size << "\t" << t.experts << "\t"
              << t.shape.size();
            for (int64_t d : t.shape) o << "\t" << d;
            o << "\t" << t.parts.size();
            for (const strix::StrixwPart &p : t.parts) o << "\t" << p.source << "\t" << p.row_offset << "\t" << p.rows;
            o << "\t" << t.components.size();
            for (const strix::StrixwComponent &c : t.components)
                o << "\t" << (int)c.role << "\t" << c.offset << "\t" << c.bytes << "\t" << c.hash;
            o << "\n";
        }
        put_msg(o.str(), dump, dump_cap);
        return 0;
    } catch (const std::exception &e) {
        put_msg(e.what(), msg, cap);
        return 1;
    }
}

}  // extern "C"
