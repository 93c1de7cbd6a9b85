// strixw weight files on MI355X: a validating reader over a read-only mapping (StrixwFile, formats/strixw.hpp:86-112)
// and the upload of a file's data region into device memory the caller owns (StrixwDevice,
// runtime/strixw_loader.hpp:22-52).
//
// The file: a 128-byte header, an index (metadata, then one record per tensor with its components' absolute offsets,
// sizes and hashes) and a data region starting on a 4096-byte boundary; every tensor starts on a 4096-byte boundary
// and every component on a 256-byte one (formats/strixw.cpp:276-290). Tensors keep their file offsets on the device, so
// a component's device address is base + (offset - data_offset) and the alignment carries over.
//
// Upload: the data region streams through a ring of pinned staging slots. A persistent pool of reader threads fills
// the slots with pread() pieces, several chunks ahead of the copies; each full chunk is handed to the copy engine with
// hipMemcpyAsync on the caller's stream, and a slot is refilled only after the event recorded behind its last copy
// has completed. The host never touches the device memory itself, and nothing here allocates device memory.
#include "common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <chrono>
#include <climits>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <thread>
#include <vector>

namespace {

constexpr uint64_t kHeaderBytes = 128, kTensorAlign = 4096, kComponentAlign = 256;
constexpr uint32_t kNewestVersion = 4, kOldestVersion = 1;  // v1-v3 files are subsets of v4's encodings

struct Part {
    std::string source;
    int64_t row_offset = 0, rows = 0;
};
struct Component {
    uint8_t role = 0;
    uint64_t offset = 0, bytes = 0, hash = 0;
};
struct Tensor {
    std::string name;
    uint8_t encoding = 0;
    std::vector<int64_t> shape;
    int64_t group = 0, experts = 0;
    std::vector<Part> parts;
    std::vector<Component> comps;
};

// A format violation: the text names what is wrong; the C boundary prefixes the file unless `whole` (the message of a
// record's shape / encoding check, which names the tensor alone, as the reference's does).
struct Reject {
    std::string msg;
    bool whole = false;
};

template <typename... Args>
[[noreturn]] void reject(Args &&...args) {
    throw Reject{sx::cat(std::forward<Args>(args)...)};
}

template <typename... Args>
[[noreturn]] void reject_record(Args &&...args) {
    throw Reject{sx::cat("strixw tensor ", std::forward<Args>(args)...), true};
}

std::string shape_text(const std::vector<int64_t> &s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

const char *encoding_name(uint8_t e) {
    static const char *names[] = {"?", "q4", "q4-chunk-major", "bf16", "f32", "i64", "q8", "q8-chunk-major", "q6", "q5"};
    return e >= 1 && e <= 9 ? names[e] : "unknown";
}

const char *role_name(uint8_t r) {
    static const char *names[] = {"data", "q", "scale", "min"};
    return r <= 3 ? names[r] : "unknown";
}

uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// strix_hash64 (formats/strixw.cpp:253-274): the file's own 64-bit checksum, so it is computed exactly as the
// writer computes it. Four multiply-xorshift lanes take the 32-byte blocks; the 8-byte words after the last block go
// to lanes 0, 1, 2 in turn; the last 1..7 bytes, zero-padded and tagged with their count in the top byte, go to lane 0;
// the lanes are then folded in order and finished with a xorshift-multiply-xorshift.
constexpr uint64_t kMulA = 0x9e3779b97f4a7c15ull, kMulB = 0xd6e8feb86659fd93ull;

inline uint64_t absorb(uint64_t lane, uint64_t word) {
    lane ^= word * kMulA;
    return (lane ^ (lane >> 31)) * kMulB;
}

uint64_t hash64(const uint8_t *p, uint64_t n) {
    uint64_t lane[4] = {n ^ kMulA, n ^ kMulB, ~n ^ kMulA, ~n ^ kMulB};
    const uint64_t blocks = n / 32;
    for (uint64_t b = 0; b < blocks; ++b) {
        uint64_t w[4];
        std::memcpy(w, p + 32 * b, 32);
        for (int l = 0; l < 4; ++l) lane[l] = absorb(lane[l], w[l]);
    }
    uint64_t at = 32 * blocks;
    for (int l = 0; n - at >= 8; at += 8, ++l) {
        uint64_t w;
        std::memcpy(&w, p + at, 8);
        lane[l] = absorb(lane[l], w);
    }
    if (at < n) {
        uint64_t w = 0;
        std::memcpy(&w, p + at, n - at);
        lane[0] = absorb(lane[0], w ^ ((n - at) << 56));
    }
    uint64_t r = absorb(absorb(absorb(lane[0], lane[1]), lane[2]), lane[3]);
    r = (r ^ (r >> 33)) * kMulA;
    return r ^ (r >> 29);
}

// The components an encoding has and their sizes for a record's shape and group (formats/strixw.cpp:177-251):
// q4 / q8 / q6 / q5 (row- or chunk-major) [N, K] with G in {32, 64, 128} dividing K: codes (N*K/2, N*K, N*3K/4 with
// K % 64 == 0, N*5K/8 with K % 128 == 0), then BF16 scale and min [N, K/G]; bf16 / f32 / i64 (group 0): one data
// component of numel * 2 / 4 / 8 bytes.
std::vector<Component> expected_components(const Tensor &t) {
    int64_t numel = 1;
    for (int64_t d : t.shape) {
        if (d < 1 || numel > INT64_MAX / d) reject_record("'", t.name, "': bad shape ", shape_text(t.shape));
        numel *= d;
    }
    auto make = [](uint8_t role, int64_t bytes) { return Component{role, 0, (uint64_t)bytes, 0}; };
    const uint8_t e = t.encoding;
    if (e == 1 || e == 2 || e == 6 || e == 7 || e == 8 || e == 9) {
        if (t.shape.size() != 2)
            reject_record("'", t.name, "': ", encoding_name(e), " needs shape [N, K], got ", shape_text(t.shape));
        const int64_t N = t.shape[0], K = t.shape[1], G = t.group;
        const int64_t kmul = e == 8 ? 64 : e == 9 ? 128 : 1;
        if (!(G == 32 || G == 64 || G == 128) || K % G != 0 || K % kmul != 0)
            reject_record("'", t.name, "': ", encoding_name(e), " with K = ", K, ", group size ", G,
                   " (must be 32/64/128 and divide K", kmul > 1 ? "; K a multiple of " + std::to_string(kmul) : "",
                   ")");
        const int64_t code_bytes = e == 1 || e == 2 ? N * K / 2 : e == 6 || e == 7 ? N * K
                                   : e == 8 ? N * (K / 2 + K / 4) : N * (K / 2 + K / 8);
        const int64_t side = N * (K / G) * 2;
        return {make(1, code_bytes), make(2, side), make(3, side)};
    }
    if (e == 3 || e == 4 || e == 5) {
        if (t.group != 0) reject_record("'", t.name, "': ", encoding_name(e), " has group size ", t.group, ", expected 0");
        const int64_t es = e == 3 ? 2 : e == 4 ? 4 : 8;
        if (numel > INT64_MAX / es) reject_record("'", t.name, "': ", numel, " elements overflow");
        return {make(0, numel * es)};
    }
    reject_record("'", t.name, "': unknown encoding ", (int)e);
}

// What every record must satisfy apart from its components (formats/strixw.cpp:80-100).
void check_record(const Tensor &t) {
    if (t.name.empty()) reject("tensor with an empty name");
    if (t.shape.empty() || t.shape.size() > 8)
        reject("tensor '", t.name, "' has ", t.shape.size(), " dims, expected 1..8");
    for (int64_t d : t.shape)
        if (d < 1) reject("tensor '", t.name, "' has shape ", shape_text(t.shape));
    if (t.experts < 0 || (t.experts > 0 && t.shape[0] % t.experts != 0))
        reject("tensor '", t.name, "': ", t.shape[0], " rows don't split into ", t.experts, " experts");
    int64_t row = 0;
    for (const Part &p : t.parts) {
        if (p.source.empty() || p.rows < 1 || p.row_offset != row)
            reject("tensor '", t.name, "' part '", p.source, "' at row ", p.row_offset, " (", p.rows,
                   " rows), expected to start at row ", row);
        row += p.rows;
    }
    if (!t.parts.empty() && row != t.shape[0])
        reject("tensor '", t.name, "' parts cover ", row, " rows of ", t.shape[0]);
}

// Little-endian reads off the index, each bounds-checked against the index's end.
struct IndexReader {
    const uint8_t *p;
    uint64_t n, at = 0;
    template <typename T>
    T get(const char *what) {
        if (n - at < sizeof(T)) reject("index ends inside ", what, " (at index byte ", at, " of ", n, ")");
        T v;
        std::memcpy(&v, p + at, sizeof(T));
        at += sizeof(T);
        return v;
    }
    std::string text(uint64_t len, const char *what) {
        if (n - at < len) reject("index ends inside ", what, " (", len, " bytes at index byte ", at, " of ", n, ")");
        std::string s(reinterpret_cast<const char *>(p + at), len);
        at += len;
        return s;
    }
};

}  // namespace

struct sx_strixw {
    std::string path;
    const uint8_t *map = nullptr;
    uint64_t size = 0, data_offset = 0;
    uint32_t version = 0;
    std::vector<std::pair<std::string, std::string>> meta;  // in file (key) order
    std::map<std::string, size_t> meta_at;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> tensor_at;

    ~sx_strixw() {
        if (map) ::munmap(const_cast<uint8_t *>(map), size);
    }

    void parse() {
        const uint8_t *b = map;
        auto u32 = [&](uint64_t off) { uint32_t v; std::memcpy(&v, b + off, 4); return v; };
        auto u64 = [&](uint64_t off) { uint64_t v; std::memcpy(&v, b + off, 8); return v; };
        if (std::memcmp(b, "STRIXWT", 8) != 0) reject("not a strixw file (bad magic)");
        version = u32(8);
        if (version < kOldestVersion || version > kNewestVersion)
            reject("format version ", version, ", this build reads ", kOldestVersion, "..", kNewestVersion,
                   " (re-run the converter)");
        if (u32(12) != kHeaderBytes) reject("header size ", u32(12), ", expected ", kHeaderBytes);
        if (u64(120) != hash64(b, 120)) reject("header hash mismatch (corrupt header)");
        const uint64_t index_off = u64(16), index_bytes = u64(24), file_bytes = u64(40);
        data_offset = u64(32);
        if (file_bytes != size) reject("header says ", file_bytes, " bytes, the file has ", size, " (truncated or appended to)");
        if (index_off != kHeaderBytes || index_bytes > size - index_off)
            reject("index at ", index_off, " (", index_bytes, " bytes) doesn't fit the ", size, "-byte file");
        if (data_offset % kTensorAlign != 0 || data_offset < index_off + index_bytes || data_offset > size)
            reject("data offset ", data_offset, " (index ends at ", index_off + index_bytes, ", alignment ", kTensorAlign,
                   ")");
        if (u64(48) != hash64(b + index_off, index_bytes)) reject("index hash mismatch (corrupt index)");

        IndexReader r{b + index_off, index_bytes};
        const uint32_t nmeta = r.get<uint32_t>("metadata count");
        for (uint32_t i = 0; i < nmeta; ++i) {
            std::string key = r.text(r.get<uint16_t>("metadata key length"), "metadata key");
            std::string val = r.text(r.get<uint32_t>("metadata value length"), "metadata value");
            if (!meta_at.emplace(key, meta.size()).second) reject("metadata key '", key, "' twice");
            meta.emplace_back(std::move(key), std::move(val));
        }
        const uint32_t ntensors = r.get<uint32_t>("tensor count");
        if (ntensors < 1) reject("no tensors");
        std::vector<std::pair<uint64_t, uint64_t>> spans;
        for (uint32_t i = 0; i < ntensors; ++i) {
            Tensor t;
            t.name = r.text(r.get<uint16_t>("tensor name length"), "tensor name");
            t.encoding = r.get<uint8_t>("encoding");
            const uint8_t ndim = r.get<uint8_t>("ndim");
            for (uint8_t d = 0; d < ndim; ++d) t.shape.push_back(r.get<int64_t>("shape"));
            t.group = r.get<int64_t>("group size");
            t.experts = r.get<int64_t>("experts");
            const uint16_t nparts = r.get<uint16_t>("part count");
            for (uint16_t p = 0; p < nparts; ++p) {
                Part part;
                part.source = r.text(r.get<uint16_t>("part name length"), "part name");
                part.row_offset = r.get<int64_t>("part row offset");
                part.rows = r.get<int64_t>("part rows");
                t.parts.push_back(std::move(part));
            }
            const uint8_t ncomp = r.get<uint8_t>("component count");
            for (uint8_t c = 0; c < ncomp; ++c) {
                Component comp;
                comp.role = r.get<uint8_t>("component role");
                comp.offset = r.get<uint64_t>("component offset");
                comp.bytes = r.get<uint64_t>("component bytes");
                comp.hash = r.get<uint64_t>("component hash");
                t.comps.push_back(comp);
            }
            check_record(t);
            const std::vector<Component> want = expected_components(t);
            if (want.size() != t.comps.size())
                reject("tensor '", t.name, "' (", encoding_name(t.encoding), ") has ", t.comps.size(),
                       " components, expected ", want.size());
            for (size_t c = 0; c < want.size(); ++c) {
                const Component &g = t.comps[c];
                if (g.role != want[c].role || g.bytes != want[c].bytes)
                    reject("tensor '", t.name, "' component ", c, " is ", role_name(g.role), " of ", g.bytes,
                           " bytes, expected ", role_name(want[c].role), " of ", want[c].bytes, " for ",
                           encoding_name(t.encoding), " ", shape_text(t.shape));
                if (g.offset < data_offset || g.offset % kComponentAlign != 0 || g.bytes > size - g.offset)
                    reject("tensor '", t.name, "' ", role_name(g.role), " at ", g.offset, " (", g.bytes,
                           " bytes) is outside the data region [", data_offset, ", ", size, ") or not ",
                           kComponentAlign, "-aligned");
                spans.emplace_back(g.offset, g.offset + g.bytes);
            }
            if (!tensor_at.emplace(t.name, tensors.size()).second) reject("tensor '", t.name, "' twice");
            tensors.push_back(std::move(t));
        }
        if (r.at != r.n) reject(r.n - r.at, " unread bytes after the last index record");
        std::sort(spans.begin(), spans.end());
        for (size_t i = 1; i < spans.size(); ++i)
            if (spans[i].first < spans[i - 1].second) reject("components overlap at byte ", spans[i].first);
    }
};

namespace {

// Runs `fn` and turns a Reject (or any other exception) into the C ABI's error channel.
template <typename Fn>
int guarded(const char *fn_name, const std::string &where, Fn &&fn) {
    try {
        return fn();
    } catch (const Reject &r) {
        sx::set_error(r.whole ? sx::cat(fn_name, ": ", r.msg) : sx::cat(fn_name, ": ", where, ": ", r.msg));
        return SX_EINVAL;
    } catch (const std::exception &e) {
        sx::set_error(sx::cat(fn_name, ": ", where, ": ", e.what()));
        return SX_EINVAL;
    }
}

std::string where_of(const sx_strixw *f) { return "strixw '" + f->path + "'"; }

const Tensor *lookup(const sx_strixw *f, const char *name) {
    auto it = f->tensor_at.find(name);
    return it == f->tensor_at.end() ? nullptr : &f->tensors[it->second];
}

// A pool of reader threads taking pread() pieces off one queue; each piece belongs to a chunk whose counter the
// last piece to finish brings to zero.
class ReadPool {
public:
    struct Chunk {
        std::atomic<int> left{0};
    };

    ReadPool(int fd, int threads) : fd_(fd) {
        for (int i = 0; i < threads; ++i) workers_.emplace_back([this] { run(); });
    }
    ~ReadPool() {
        {
            std::lock_guard<std::mutex> lock(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (std::thread &t : workers_) t.join();
    }

    // Queues bytes [off, off + n) of the file into dst, split into pieces of at most `piece` bytes.
    void read(Chunk &c, uint8_t *dst, uint64_t off, uint64_t n, uint64_t piece) {
        const int pieces = (int)((n + piece - 1) / piece);
        c.left.store(pieces);
        {
            std::lock_guard<std::mutex> lock(mu_);
            for (int i = 0; i < pieces; ++i) {
                const uint64_t a = (uint64_t)i * piece, len = std::min(piece, n - a);
                queue_.push_back(Job{&c, dst + a, off + a, len});
            }
        }
        cv_.notify_all();
    }

    // Blocks until every piece of c has been read (or failed); returns the first error text, empty if none.
    std::string wait(Chunk &c) {
        std::unique_lock<std::mutex> lock(mu_);
        done_cv_.wait(lock, [&] { return c.left.load() == 0; });
        return error_;
    }

private:
    struct Job {
        Chunk *chunk;
        uint8_t *dst;
        uint64_t off, n;
    };

    void run() {
        for (;;) {
            Job job;
            {
                std::unique_lock<std::mutex> lock(mu_);
                cv_.wait(lock, [&] { return stop_ || !queue_.empty(); });
                if (queue_.empty()) return;
                job = queue_.front();
                queue_.pop_front();
            }
            std::string err;
            uint64_t done = 0;
            while (done < job.n && err.empty()) {
                const ssize_t got = ::pread(fd_, job.dst + done, job.n - done, (off_t)(job.off + done));
                if (got < 0 && errno == EINTR) continue;
                if (got <= 0)
                    err = sx::cat("reading ", job.n, " bytes at ", job.off, " failed: ",
                                  got < 0 ? std::strerror(errno) : "unexpected end of file");
                else
                    done += (uint64_t)got;
            }
            std::lock_guard<std::mutex> lock(mu_);
            if (!err.empty() && error_.empty()) error_ = err;
            if (job.chunk->left.fetch_sub(1) == 1) done_cv_.notify_all();
        }
    }

    int fd_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    std::deque<Job> queue_;
    std::vector<std::thread> workers_;
    std::string error_;
    bool stop_ = false;
};

constexpr int kSlots = 4;
constexpr uint64_t kSlotBytes = 64ull << 20, kPieceBytes = 4ull << 20;

}  // namespace

extern "C" {

uint64_t sx_strix_hash64(const void *data, uint64_t n) { return hash64(static_cast<const uint8_t *>(data), n); }

int sx_strixw_open(const char *path, sx_strixw **out) {
    SX_CHECK(path != nullptr && out != nullptr, "null argument");
    *out = nullptr;
    auto f = std::make_unique<sx_strixw>();
    f->path = path;
    return guarded(__func__, where_of(f.get()), [&] {
        const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) reject("open failed: ", std::strerror(errno));
        struct stat st {};
        if (::fstat(fd, &st) != 0) {
            const int e = errno;
            ::close(fd);
            reject("fstat failed: ", std::strerror(e));
        }
        f->size = (uint64_t)st.st_size;
        if (f->size < kHeaderBytes) {
            ::close(fd);
            reject(f->size, " bytes, smaller than the ", kHeaderBytes, "-byte header");
        }
        void *m = ::mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, fd, 0);
        const int e = errno;
        ::close(fd);
        if (m == MAP_FAILED) reject("mmap of ", f->size, " bytes failed: ", std::strerror(e));
        f->map = static_cast<const uint8_t *>(m);
        f->parse();
        *out = f.release();
        return SX_OK;
    });
}

void sx_strixw_close(sx_strixw *f) { delete f; }

int sx_strixw_summary(const sx_strixw *f, uint32_t *version, uint64_t *file_bytes, uint64_t *data_offset,
                      int64_t *tensors, int64_t *meta) {
    SX_CHECK(f != nullptr, "null file");
    if (version) *version = f->version;
    if (file_bytes) *file_bytes = f->size;
    if (data_offset) *data_offset = f->data_offset;
    if (tensors) *tensors = (int64_t)f->tensors.size();
    if (meta) *meta = (int64_t)f->meta.size();
    return SX_OK;
}

int sx_strixw_meta_at(const sx_strixw *f, int64_t i, const char **key, const char **value) {
    SX_CHECK(f != nullptr && key != nullptr && value != nullptr, "null argument");
    SX_CHECK(i >= 0 && i < (int64_t)f->meta.size(), "metadata index ", i, " of ", f->meta.size());
    *key = f->meta[(size_t)i].first.c_str();
    *value = f->meta[(size_t)i].second.c_str();
    return SX_OK;
}

int sx_strixw_meta(const sx_strixw *f, const char *key, const char **value) {
    SX_CHECK(f != nullptr && key != nullptr && value != nullptr, "null argument");
    auto it = f->meta_at.find(key);
    SX_CHECK(it != f->meta_at.end(), where_of(f), " has no metadata '", key, "'");
    *value = f->meta[it->second].second.c_str();
    return SX_OK;
}

int sx_strixw_find(const sx_strixw *f, const char *name, int64_t *index) {
    SX_CHECK(f != nullptr && name != nullptr && index != nullptr, "null argument");
    auto it = f->tensor_at.find(name);
    *index = it == f->tensor_at.end() ? -1 : (int64_t)it->second;
    return SX_OK;
}

int sx_strixw_tensor_at(const sx_strixw *f, int64_t i, sx_strixw_tensor *out) {
    SX_CHECK(f != nullptr && out != nullptr, "null argument");
    SX_CHECK(i >= 0 && i < (int64_t)f->tensors.size(), "tensor index ", i, " of ", f->tensors.size());
    const Tensor &t = f->tensors[(size_t)i];
    std::memset(out, 0, sizeof(*out));
    out->name = t.name.c_str();
    out->encoding = t.encoding;
    out->ndim = (int32_t)t.shape.size();
    for (size_t d = 0; d < t.shape.size(); ++d) out->shape[d] = t.shape[d];
    out->group_size = t.group;
    out->experts = t.experts;
    out->nparts = (int32_t)t.parts.size();
    out->ncomp = (int32_t)t.comps.size();
    for (size_t c = 0; c < t.comps.size(); ++c)
        out->comp[c] = sx_strixw_component{t.comps[c].role, t.comps[c].offset, t.comps[c].bytes, t.comps[c].hash};
    return SX_OK;
}

int sx_strixw_part_at(const sx_strixw *f, int64_t tensor, int64_t part, const char **source, int64_t *row_offset,
                      int64_t *rows) {
    SX_CHECK(f != nullptr && source != nullptr && row_offset != nullptr && rows != nullptr, "null argument");
    SX_CHECK(tensor >= 0 && tensor < (int64_t)f->tensors.size(), "tensor index ", tensor, " of ", f->tensors.size());
    const Tensor &t = f->tensors[(size_t)tensor];
    SX_CHECK(part >= 0 && part < (int64_t)t.parts.size(), "part index ", part, " of ", t.parts.size());
    *source = t.parts[(size_t)part].source.c_str();
    *row_offset = t.parts[(size_t)part].row_offset;
    *rows = t.parts[(size_t)part].rows;
    return SX_OK;
}

int sx_strixw_verify_hashes(const sx_strixw *f, int threads) {
    SX_CHECK(f != nullptr, "null file");
    SX_CHECK(threads >= 1 && threads <= 1024, "threads = ", threads);
    std::vector<std::pair<size_t, size_t>> work;
    for (size_t t = 0; t < f->tensors.size(); ++t)
        for (size_t c = 0; c < f->tensors[t].comps.size(); ++c) work.emplace_back(t, c);
    std::vector<char> bad(work.size(), 0);
    std::atomic<size_t> next{0};
    auto worker = [&] {
        for (size_t i; (i = next.fetch_add(1)) < work.size();) {
            const Component &c = f->tensors[work[i].first].comps[work[i].second];
            bad[i] = hash64(f->map + c.offset, c.bytes) != c.hash;
        }
    };
    std::vector<std::thread> pool;
    for (int i = 0; i < std::min<int>(threads, (int)work.size()); ++i) pool.emplace_back(worker);
    for (std::thread &th : pool) th.join();
    for (size_t i = 0; i < work.size(); ++i)  // the first corrupt component in file order
        if (bad[i]) {
            const Tensor &t = f->tensors[work[i].first];
            const Component &c = t.comps[work[i].second];
            sx::set_error(sx::cat(__func__, ": ", where_of(f), ": hash mismatch in tensor '", t.name, "' ",
                                  role_name(c.role), " (", c.bytes, " bytes at ", c.offset, ") - the file is corrupt"));
            return SX_EINVAL;
        }
    return SX_OK;
}

int sx_strixw_load(const sx_strixw *f, void *dst, uint64_t dst_bytes, int read_threads, double *seconds,
                   sx_stream stream) {
    SX_CHECK(f != nullptr && dst != nullptr, "null argument");
    SX_CHECK(read_threads >= 1 && read_threads <= 64, "read_threads = ", read_threads);
    const uint64_t n = f->size - f->data_offset;
    SX_CHECK(n > 0, where_of(f), " has an empty data region");
    SX_CHECK(dst_bytes >= n, "destination holds ", dst_bytes, " bytes, the data region is ", n);
    SX_CHECK(sx::aligned(dst, kComponentAlign), "destination ", dst, " must be ", kComponentAlign, "-byte aligned");
    const auto t0 = std::chrono::steady_clock::now();
    const hipStream_t s = sx::stream_of(stream);
    const int fd = ::open(f->path.c_str(), O_RDONLY | O_CLOEXEC);
    SX_CHECK(fd >= 0, "open '", f->path, "' failed: ", std::strerror(errno));
    const uint64_t slot_bytes = std::min(kSlotBytes, round_up(n, kTensorAlign));
    const uint64_t nchunks = (n + slot_bytes - 1) / slot_bytes;
    const int slots = (int)std::min<uint64_t>(kSlots, nchunks);
    void *stage[kSlots] = {};
    hipEvent_t copied[kSlots] = {};
    bool pending[kSlots] = {};
    ReadPool::Chunk chunk_state[kSlots];
    std::string err;
    int rc = SX_OK;
    auto fail = [&](int code, std::string msg) {
        if (rc == SX_OK) rc = code, err = std::move(msg);
    };
    for (int i = 0; i < slots && rc == SX_OK; ++i) {
        hipError_t e = hipHostMalloc(&stage[i], slot_bytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&copied[i], hipEventDisableTiming);
        if (e != hipSuccess) fail(SX_EHIP, sx::cat("staging slot ", i, ": ", hipGetErrorName(e)));
    }
    if (rc == SX_OK) {
        ReadPool pool(fd, read_threads);
        uint64_t issued = 0;  // chunks whose reads are queued
        for (uint64_t c = 0; c < nchunks && rc == SX_OK; ++c) {
            // keep the readers up to (slots - 1) chunks ahead of the copy engine
            while (issued < nchunks && issued < c + (uint64_t)slots && rc == SX_OK) {
                const int k = (int)(issued % (uint64_t)slots);
                if (pending[k]) {
                    const hipError_t e = hipEventSynchronize(copied[k]);
                    if (e != hipSuccess) {
                        fail(SX_EHIP, sx::cat("waiting for the copy out of slot ", k, ": ", hipGetErrorName(e)));
                        break;
                    }
                    pending[k] = false;
                }
                const uint64_t at = issued * slot_bytes, len = std::min(slot_bytes, n - at);
                pool.read(chunk_state[k], static_cast<uint8_t *>(stage[k]), f->data_offset + at, len, kPieceBytes);
                ++issued;
            }
            if (rc != SX_OK) break;
            const int k = (int)(c % (uint64_t)slots);
            std::string read_err = pool.wait(chunk_state[k]);
            if (!read_err.empty()) {
                fail(SX_EINVAL, sx::cat("'", f->path, "': ", read_err));
                break;
            }
            const uint64_t at = c * slot_bytes, len = std::min(slot_bytes, n - at);
            hipError_t e = hipMemcpyAsync(static_cast<uint8_t *>(dst) + at, stage[k], len, hipMemcpyHostToDevice, s);
            if (e == hipSuccess) e = hipEventRecord(copied[k], s);
            if (e != hipSuccess) {
                fail(SX_EHIP, sx::cat("copy of ", len, " bytes at ", at, ": ", hipGetErrorName(e)));
                break;
            }
            pending[k] = true;
        }
        // drain: every queued read finishes before the pool and the staging go away
        for (int k = 0; k < slots; ++k) (void)pool.wait(chunk_state[k]);
    }
    const hipError_t es = hipStreamSynchronize(s);
    if (es != hipSuccess) fail(SX_EHIP, sx::cat("final synchronisation: ", hipGetErrorName(es)));
    for (int i = 0; i < slots; ++i) {
        if (copied[i]) (void)hipEventDestroy(copied[i]);
        if (stage[i]) (void)hipHostFree(stage[i]);
    }
    ::close(fd);
    if (rc != SX_OK) {
        sx::set_error(sx::cat(__func__, ": ", err));
        return rc;
    }
    if (seconds) *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return SX_OK;
}

int sx_strixw_qview(const sx_strixw *f, const void *base, const char *name, int bits, int64_t N, int64_t K,
                    sx_qview *out) {
    SX_CHECK(f != nullptr && name != nullptr && out != nullptr, "null argument");
    SX_CHECK(bits == 0 || bits == 4 || bits == 8, "bits = ", bits, ", expected 4, 8 or 0 (either)");
    const Tensor *t = lookup(f, name);
    SX_CHECK(t != nullptr, where_of(f), " has no tensor '", name, "'");
    const bool enc_ok = bits == 4 ? t->encoding == 1 : bits == 8 ? t->encoding == 6 : (t->encoding == 1 || t->encoding == 6);
    const std::vector<int64_t> want{N, K};
    SX_CHECK(enc_ok && t->shape == want, "'", name, "' in '", f->path, "' is ", encoding_name(t->encoding), " ",
             shape_text(t->shape), ", expected ", bits == 4 ? "q4" : bits == 8 ? "q8" : "q4 or q8 row-major", " ",
             shape_text(want));
    const uint8_t *b = base ? static_cast<const uint8_t *>(base) - f->data_offset : f->map;
    out->q = b + t->comps[0].offset;
    out->scale = reinterpret_cast<const uint16_t *>(b + t->comps[1].offset);
    out->minv = reinterpret_cast<const uint16_t *>(b + t->comps[2].offset);
    out->N = N, out->K = K, out->G = t->group;
    return SX_OK;
}

int sx_strixw_data(const sx_strixw *f, const void *base, const char *name, int encoding, const int64_t *shape,
                   int ndim, const void **out) {
    SX_CHECK(f != nullptr && name != nullptr && out != nullptr && (shape != nullptr || ndim == 0), "null argument");
    SX_CHECK(encoding == SX_STRIXW_BF16 || encoding == SX_STRIXW_F32 || encoding == SX_STRIXW_I64,
             "encoding ", encoding, ", expected bf16 (3), f32 (4) or i64 (5)");
    const Tensor *t = lookup(f, name);
    SX_CHECK(t != nullptr, where_of(f), " has no tensor '", name, "'");
    const std::vector<int64_t> want(shape, shape + ndim);
    SX_CHECK(t->encoding == encoding && t->shape == want, "'", name, "' in '", f->path, "' is ",
             encoding_name(t->encoding), " ", shape_text(t->shape), ", expected ", encoding_name((uint8_t)encoding), " ",
             shape_text(want));
    const uint8_t *b = base ? static_cast<const uint8_t *>(base) - f->data_offset : f->map;
    *out = b + t->comps[0].offset;
    return SX_OK;
}

}  // extern "C"
