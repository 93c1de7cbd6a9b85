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

// A file this reader refuses; the C boundary puts the function and the file's path in front of the text.
struct Reject {
    std::string msg;
};

template <typename... Args>
[[noreturn]] void reject(Args &&...args) {
    throw Reject{sx::cat(std::forward<Args>(args)...)};
}

std::string shape_text(const std::vector<int64_t> &s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

// The encodings the format defines (formats/strixw.hpp), by their code in the index. A grouped encoding stores
// `bits` code bits a weight (rows of K codes, K a multiple of `k_multiple`), then BF16 scale and min [N, K/G]; a plain
// one stores `elem_bytes` a value in one data component.
struct Encoding {
    const char *name;
    int bits;           // grouped: code bits a weight; 0 for a plain encoding
    int k_multiple;     // grouped: K must be a multiple of this (the packing of 6- and 5-bit codes)
    int elem_bytes;     // plain: bytes a value
};
constexpr Encoding kEncodings[] = {
    {nullptr, 0, 0, 0},       {"q4", 4, 1, 0},   {"q4-chunk-major", 4, 1, 0}, {"bf16", 0, 0, 2},
    {"f32", 0, 0, 4},         {"i64", 0, 0, 8},  {"q8", 8, 1, 0},             {"q8-chunk-major", 8, 1, 0},
    {"q6", 6, 64, 0},         {"q5", 5, 128, 0},
};
constexpr int kEncodingCount = (int)(sizeof(kEncodings) / sizeof(kEncodings[0]));

const Encoding *encoding_of(uint8_t code) {
    return code >= 1 && code < kEncodingCount ? &kEncodings[code] : nullptr;
}
const char *encoding_name(uint8_t code) {
    const Encoding *e = encoding_of(code);
    return e ? e->name : "unknown";
}
const char *role_name(uint8_t r) {
    static const char *names[] = {"data", "q", "scale", "min"};
    return r <= 3 ? names[r] : "unknown";
}

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

// ---- the header: decoded whole, then judged by a list of rules taken in order ----

struct Header {
    char magic[8];
    uint32_t version, header_bytes;
    uint64_t index_offset, index_bytes, data_offset, file_bytes, index_hash, header_hash;
};

Header decode_header(const uint8_t *b) {
    Header h;
    std::memcpy(h.magic, b, 8);
    std::memcpy(&h.version, b + 8, 4);
    std::memcpy(&h.header_bytes, b + 12, 4);
    std::memcpy(&h.index_offset, b + 16, 8);
    std::memcpy(&h.index_bytes, b + 24, 8);
    std::memcpy(&h.data_offset, b + 32, 8);
    std::memcpy(&h.file_bytes, b + 40, 8);
    std::memcpy(&h.index_hash, b + 48, 8);
    std::memcpy(&h.header_hash, b + 120, 8);
    return h;
}

// Each rule sees the header, the mapping and its size, and returns an empty string when the file passes it. The
// order matters only for which complaint a doubly broken file gets: the checksums come after the fields that say
// where the bytes they cover are.
using HeaderRule = std::string (*)(const Header &, const uint8_t *, uint64_t);

const HeaderRule kHeaderRules[] = {
    [](const Header &h, const uint8_t *, uint64_t) -> std::string {
        return std::memcmp(h.magic, "STRIXWT", 8) == 0 ? "" : "no STRIXWT signature at byte 0";
    },
    [](const Header &h, const uint8_t *, uint64_t) -> std::string {
        if (h.version >= kOldestVersion && h.version <= kNewestVersion) return "";
        return sx::cat("written as version ", h.version, "; versions ", kOldestVersion, " to ", kNewestVersion,
                       " are readable (convert the weights again)");
    },
    [](const Header &h, const uint8_t *, uint64_t) -> std::string {
        return h.header_bytes == kHeaderBytes ? "" : sx::cat("declares a ", h.header_bytes, "-byte header, not ", kHeaderBytes);
    },
    [](const Header &h, const uint8_t *b, uint64_t) -> std::string {
        return h.header_hash == hash64(b, 120) ? "" : "checksum of header bytes 0..119 does not match";
    },
    [](const Header &h, const uint8_t *, uint64_t size) -> std::string {
        return h.file_bytes == size ? "" : sx::cat("length on disk ", size, " differs from the recorded ", h.file_bytes);
    },
    [](const Header &h, const uint8_t *, uint64_t size) -> std::string {
        if (h.index_offset == kHeaderBytes && h.index_bytes <= size - h.index_offset) return "";
        return sx::cat("index [", h.index_offset, ", +", h.index_bytes, ") is not right after the header inside ", size,
                       " bytes");
    },
    [](const Header &h, const uint8_t *, uint64_t size) -> std::string {
        const uint64_t index_end = h.index_offset + h.index_bytes;
        if (h.data_offset % kTensorAlign == 0 && h.data_offset >= index_end && h.data_offset <= size) return "";
        return sx::cat("data region start ", h.data_offset, " must be a multiple of ", kTensorAlign, " in [", index_end,
                       ", ", size, "]");
    },
    [](const Header &h, const uint8_t *b, uint64_t) -> std::string {
        return h.index_hash == hash64(b + h.index_offset, h.index_bytes) ? "" : "checksum of the index does not match";
    },
};

// ---- the index: a stream with a sticky failure, decoded in one pass ----

// Reads little-endian fields off the index. A read past the end leaves the target zeroed and marks the stream
// broken; the decoder checks once a record, and the first field that did not fit names the place.
class IndexStream {
public:
    IndexStream(const uint8_t *p, uint64_t n) : p_(p), n_(n) {}

    template <typename T>
    T next(const char *field) {
        T v{};
        if (take(sizeof(T), field)) std::memcpy(&v, p_ + pos_ - sizeof(T), sizeof(T));
        return v;
    }
    template <typename LenT>
    std::string next_text(const char *field) {
        const uint64_t len = next<LenT>(field);
        if (!take(len, field)) return {};
        return std::string(reinterpret_cast<const char *>(p_ + pos_ - len), len);
    }
    void require_intact(const char *record) const {
        if (short_field_)
            reject("the index (", n_, " bytes) stops short of the ", short_field_, " of ", record);
    }
    uint64_t left() const { return n_ - pos_; }

private:
    bool take(uint64_t len, const char *field) {
        if (short_field_) return false;
        if (n_ - pos_ < len) {
            short_field_ = field;
            return false;
        }
        pos_ += len;
        return true;
    }
    const uint8_t *p_;
    uint64_t n_, pos_ = 0;
    const char *short_field_ = nullptr;
};

Tensor decode_record(IndexStream &in) {
    Tensor t;
    t.name = in.next_text<uint16_t>("name");
    t.encoding = in.next<uint8_t>("encoding");
    const uint8_t ndim = in.next<uint8_t>("rank");
    for (uint8_t d = 0; d < ndim; ++d) t.shape.push_back(in.next<int64_t>("dimension"));
    t.group = in.next<int64_t>("group size");
    t.experts = in.next<int64_t>("expert count");
    const uint16_t nparts = in.next<uint16_t>("part count");
    for (uint16_t i = 0; i < nparts; ++i) {
        Part part;
        part.source = in.next_text<uint16_t>("part source");
        part.row_offset = in.next<int64_t>("part first row");
        part.rows = in.next<int64_t>("part row count");
        t.parts.push_back(std::move(part));
    }
    const uint8_t ncomp = in.next<uint8_t>("component count");
    for (uint8_t i = 0; i < ncomp; ++i) {
        Component c;
        c.role = in.next<uint8_t>("component role");
        c.offset = in.next<uint64_t>("component offset");
        c.bytes = in.next<uint64_t>("component size");
        c.hash = in.next<uint64_t>("component checksum");
        t.comps.push_back(c);
    }
    return t;
}

// ---- a record's rules: geometry, row partition, then the components the encoding implies and where they lie ----

// The (role, bytes) list an encoding implies for the record's shape and group size, or a reason it cannot hold it.
bool implied_components(const Tensor &t, std::vector<std::pair<uint8_t, uint64_t>> &out, std::string &why) {
    const Encoding *e = encoding_of(t.encoding);
    if (!e) {
        why = sx::cat("encoding code ", (int)t.encoding, " is not one this format defines");
        return false;
    }
    uint64_t numel = 1;
    for (int64_t d : t.shape) {
        if ((uint64_t)d > (uint64_t)INT64_MAX / numel) {
            why = sx::cat("shape ", shape_text(t.shape), " holds more than 2^63 values");
            return false;
        }
        numel *= (uint64_t)d;
    }
    if (e->bits == 0) {
        if (t.group != 0) {
            why = sx::cat(e->name, " values take no group size (found ", t.group, ")");
            return false;
        }
        if (numel > (uint64_t)INT64_MAX / (uint64_t)e->elem_bytes) {
            why = sx::cat(numel, " ", e->name, " values exceed the addressable size");
            return false;
        }
        out = {{0, numel * (uint64_t)e->elem_bytes}};
        return true;
    }
    if (t.shape.size() != 2) {
        why = sx::cat(e->name, " is a matrix encoding; shape ", shape_text(t.shape), " is not [rows, K]");
        return false;
    }
    const uint64_t N = (uint64_t)t.shape[0], K = (uint64_t)t.shape[1];
    const bool group_ok = t.group == 32 || t.group == 64 || t.group == 128;
    if (!group_ok || K % (uint64_t)t.group != 0 || K % (uint64_t)e->k_multiple != 0) {
        why = sx::cat(e->name, " needs a group size of 32, 64 or 128 dividing K",
                      e->k_multiple > 1 ? sx::cat(" and K divisible by ", e->k_multiple) : std::string(), "; K = ", K,
                      ", group size ", t.group);
        return false;
    }
    const uint64_t side = N * (K / (uint64_t)t.group) * 2;
    out = {{1, N * K * (uint64_t)e->bits / 8}, {2, side}, {3, side}};
    return true;
}

// Every rule a single record must meet on its own; `data_offset` and `size` bound where its components may lie.
void validate_record(const Tensor &t, uint64_t data_offset, uint64_t size) {
    const std::string who = t.name.empty() ? std::string("an unnamed tensor") : sx::cat("tensor '", t.name, "'");
    if (t.name.empty()) reject("the index holds ", who);
    if (t.shape.empty() || t.shape.size() > 8) reject(who, ": rank ", t.shape.size(), " is outside 1..8");
    if (std::any_of(t.shape.begin(), t.shape.end(), [](int64_t d) { return d < 1; }))
        reject(who, ": every dimension must be positive, shape is ", shape_text(t.shape));
    if (t.experts < 0) reject(who, ": negative expert count ", t.experts);
    if (t.experts > 0 && t.shape[0] % t.experts != 0)
        reject(who, ": ", t.experts, " experts cannot share ", t.shape[0], " rows evenly");

    // The parts tile the rows in order, with no gap and no overlap.
    int64_t next_row = 0;
    for (size_t i = 0; i < t.parts.size(); ++i) {
        const Part &p = t.parts[i];
        if (p.source.empty()) reject(who, ": part ", i, " has no source name");
        if (p.rows < 1 || p.row_offset != next_row)
            reject(who, ": part ", i, " ('", p.source, "') covers rows from ", p.row_offset, " (", p.rows,
                   " of them) where row ", next_row, " comes next");
        next_row += p.rows;
    }
    if (!t.parts.empty() && next_row != t.shape[0])
        reject(who, ": its parts end at row ", next_row, " of ", t.shape[0]);

    std::vector<std::pair<uint8_t, uint64_t>> implied;
    std::string why;
    if (!implied_components(t, implied, why)) reject(who, ": ", why);
    if (implied.size() != t.comps.size())
        reject(who, ": ", encoding_name(t.encoding), " stores ", implied.size(), " components, the index lists ",
               t.comps.size());
    for (size_t i = 0; i < implied.size(); ++i) {
        const Component &c = t.comps[i];
        if (c.role != implied[i].first || c.bytes != implied[i].second)
            reject(who, ": listed component ", i, " (", role_name(c.role), ", ", c.bytes, " bytes) should be ",
                   role_name(implied[i].first), ", ", implied[i].second, " bytes for ", encoding_name(t.encoding), " ",
                   shape_text(t.shape));
        if (c.offset % kComponentAlign != 0)
            reject(who, ": ", role_name(c.role), " starts at ", c.offset, ", not on a ", kComponentAlign,
                   "-byte boundary");
        // (offset > size first: size - offset would wrap for a component placed past the end of the file)
        if (c.offset < data_offset || c.offset > size || c.bytes > size - c.offset)
            reject(who, ": ", role_name(c.role), " bytes [", c.offset, ", +", c.bytes, ") fall outside the data region [",
                   data_offset, ", ", size, ")");
    }
}

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

    // The header's rules, then the index in one pass (metadata, then each record decoded and validated), then the
    // file-wide rules: unique names, nothing left over, no two components sharing a byte.
    void parse() {
        const Header h = decode_header(map);
        for (HeaderRule rule : kHeaderRules) {
            const std::string problem = rule(h, map, size);
            if (!problem.empty()) reject(problem);
        }
        version = h.version;
        data_offset = h.data_offset;

        IndexStream in(map + h.index_offset, h.index_bytes);
        const uint32_t nmeta = in.next<uint32_t>("entry count");
        in.require_intact("the metadata");
        for (uint32_t i = 0; i < nmeta; ++i) {
            std::string key = in.next_text<uint16_t>("key");
            std::string value = in.next_text<uint32_t>("value");
            in.require_intact(sx::cat("metadata entry ", i).c_str());
            if (meta_at.count(key)) reject("metadata key '", key, "' appears more than once");
            meta_at[key] = meta.size();
            meta.emplace_back(std::move(key), std::move(value));
        }
        const uint32_t ntensors = in.next<uint32_t>("tensor count");
        in.require_intact("the tensor list");
        if (ntensors == 0) reject("the index lists no tensors");

        struct Extent {
            uint64_t begin, end;
            bool operator<(const Extent &o) const { return begin < o.begin; }
        };
        std::vector<Extent> extents;
        for (uint32_t i = 0; i < ntensors; ++i) {
            Tensor t = decode_record(in);
            in.require_intact(sx::cat("tensor record ", i).c_str());
            validate_record(t, data_offset, size);
            if (tensor_at.count(t.name)) reject("tensor '", t.name, "' is listed more than once");
            for (const Component &c : t.comps) extents.push_back({c.offset, c.offset + c.bytes});
            tensor_at[t.name] = tensors.size();
            tensors.push_back(std::move(t));
        }
        if (in.left() != 0) reject("the index has ", in.left(), " bytes past its last tensor record");
        std::sort(extents.begin(), extents.end());
        for (size_t i = 1; i < extents.size(); ++i)
            if (extents[i].begin < extents[i - 1].end)
                reject("two components share bytes from ", extents[i].begin);
    }
};

namespace {

// Runs `fn` and turns a Reject (or any other exception) into the C ABI's error channel.
template <typename Fn>
int guarded(const char *fn_name, const std::string &where, Fn &&fn) {
    try {
        return fn();
    } catch (const Reject &r) {
        sx::set_error(sx::cat(fn_name, ": ", where, ": ", r.msg));
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
            reject("only ", f->size, " bytes: too short for the ", kHeaderBytes, "-byte header");
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
    const uint64_t slot_bytes = std::min(kSlotBytes, (n + kTensorAlign - 1) / kTensorAlign * kTensorAlign);
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
