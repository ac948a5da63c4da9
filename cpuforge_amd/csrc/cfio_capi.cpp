// C ABI of the on-disk formats (include/cfio.h).
//
// The safetensors header is parsed, validated and written on the host with
// the rules and messages of the `safetensors` crate 0.8.0 that the reference
// builds against (Cargo.lock:1177-1178; the reference prefixes the crate's
// message with the path, crates/io/src/st.rs:26-32).  Tensor bytes move
// between the file and HBM through two pinned host chunks: while one chunk's
// PCIe copy and kernel run on the stream, the host reads or writes the file
// range of the other.  One launch per chunk moves all of its runs
// (io_kernels.hip), so a state file of thousands of small tensors costs one
// copy and one launch per chunk, not per tensor.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <condition_variable>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

#include "cfattn_ctx.hpp"
#include "cfio.h"
#include "cfio_kernels.hpp"

using namespace cfcapi;
using cfio::IoPiece;

struct cfio_file {
    struct Tensor {
        std::string name;
        int dtype = 0;
        std::vector<size_t> shape;
        size_t numel = 0;
        uint64_t begin = 0, end = 0;  // data_offsets, relative to the data section
    };
    std::string path;
    int fd = -1;
    uint64_t data_start = 0;  // 8 + header length
    std::vector<Tensor> tensors;
    std::vector<std::pair<std::string, std::string>> meta;
};

namespace {

struct DtypeInfo {
    const char* name;
    unsigned bits;
};
// The crate's Dtype variants in declaration order, with their sizes in bits.
constexpr DtypeInfo kDtypes[CFIO_NUM_DTYPES] = {
    {"BOOL", 8},     {"F4", 4},       {"F6_E2M3", 6}, {"F6_E3M2", 6}, {"U8", 8},   {"I8", 8},   {"F8_E5M2", 8},
    {"F8_E4M3", 8},  {"F8_E8M0", 8},  {"I16", 16},    {"U16", 16},    {"F16", 16}, {"BF16", 16}, {"I32", 32},
    {"U32", 32},     {"F32", 32},     {"C64", 64},    {"F64", 64},    {"I64", 64}, {"U64", 64}};

constexpr uint64_t kMaxHeader = 100000000;  // the crate's MAX_HEADER_SIZE

hipStream_t to_stream(void* st) { return static_cast<hipStream_t>(st); }

// std::io::Error's Display for an OS error.
std::string os_error(int e) {
    char tail[32];
    snprintf(tail, sizeof tail, " (os error %d)", e);
    return std::string(strerror(e)) + tail;
}

void put_err(char* err, size_t cap, const std::string& m) {
    if (!err || cap == 0) return;
    const size_t n = std::min(cap - 1, m.size());
    memcpy(err, m.data(), n);
    err[n] = '\0';
}

// UTF-8 validation with the text of Rust's Utf8Error.
bool utf8_valid(const unsigned char* s, size_t n, std::string* why) {
    size_t i = 0;
    auto bad = [&](size_t len) {
        if (why) *why = "invalid utf-8 sequence of " + std::to_string(len) + " bytes from index " + std::to_string(i);
        return false;
    };
    auto incomplete = [&]() {
        if (why) *why = "incomplete utf-8 byte sequence from index " + std::to_string(i);
        return false;
    };
    while (i < n) {
        const unsigned b = s[i];
        if (b < 0x80) {
            i++;
            continue;
        }
        const int w = (b >= 0xC2 && b <= 0xDF) ? 2 : (b >= 0xE0 && b <= 0xEF) ? 3 : (b >= 0xF0 && b <= 0xF4) ? 4 : 0;
        if (!w) return bad(1);
        if (i + 1 >= n) return incomplete();
        const unsigned b1 = s[i + 1];
        unsigned lo = 0x80, hi = 0xBF;
        if (b == 0xE0) lo = 0xA0;
        else if (b == 0xED) hi = 0x9F;
        else if (b == 0xF0) lo = 0x90;
        else if (b == 0xF4) hi = 0x8F;
        if (b1 < lo || b1 > hi) return bad(1);
        for (int k = 2; k < w; k++) {
            if (i + k >= n) return incomplete();
            const unsigned bk = s[i + k];
            if (bk < 0x80 || bk > 0xBF) return bad((size_t)k);
        }
        i += (size_t)w;
    }
    return true;
}

void utf8_append(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
        out.push_back((char)cp);
    } else if (cp < 0x800) {
        out.push_back((char)(0xC0 | (cp >> 6)));
        out.push_back((char)(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
        out.push_back((char)(0xE0 | (cp >> 12)));
        out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
        out.push_back((char)(0x80 | (cp & 0x3F)));
    } else {
        out.push_back((char)(0xF0 | (cp >> 18)));
        out.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
        out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
        out.push_back((char)(0x80 | (cp & 0x3F)));
    }
}

// serde_json's string escaping: quote, backslash and the C0 controls
// (\b \f \n \r \t by name, the rest as \u00xx); every other byte as is.
void json_string(std::string& out, const std::string& s) {
    static const char hex[] = "0123456789abcdef";
    out.push_back('"');
    for (unsigned char ch : s) {
        switch (ch) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (ch < 0x20) {
                    out += "\\u00";
                    out.push_back(hex[ch >> 4]);
                    out.push_back(hex[ch & 15]);
                } else {
                    out.push_back((char)ch);
                }
        }
    }
    out.push_back('"');
}

// A reader of the header's JSON: an object whose "__metadata__" entry is a
// string map (or null) and whose other entries are tensor records
// {"dtype", "shape", "data_offsets"} (unknown record fields are skipped, as
// serde does).  Later duplicates of a name replace earlier ones, as a
// HashMap insert does.
class HeaderParser {
   public:
    HeaderParser(const char* p, size_t n) : p_(p), e_(p + n) {}
    std::string err;

    bool parse(cfio_file* f) {
        std::unordered_map<std::string, size_t> where;
        bool seen_meta = false;
        ws();
        if (p_ >= e_) return fail("EOF while parsing a value");
        if (*p_ != '{') return fail(std::string("invalid type: ") + kind_of(*p_) + ", expected struct HashMetadata");
        ++p_;
        ws();
        if (p_ < e_ && *p_ == '}') {
            ++p_;
        } else {
            while (true) {
                std::string key;
                if (!string(key) || !colon()) return false;
                if (key == "__metadata__") {
                    if (seen_meta) return fail("duplicate field `__metadata__`");
                    seen_meta = true;
                    if (!metadata(f)) return false;
                } else {
                    cfio_file::Tensor t;
                    t.name = key;
                    if (!record(t)) return false;
                    auto it = where.find(key);
                    if (it == where.end()) {
                        where.emplace(key, f->tensors.size());
                        f->tensors.push_back(std::move(t));
                    } else {
                        f->tensors[it->second] = std::move(t);
                    }
                }
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == '}') {
                    ++p_;
                    break;
                }
                return fail(p_ >= e_ ? "EOF while parsing an object" : "expected `,` or `}`");
            }
        }
        ws();
        if (p_ != e_) return fail("trailing characters");
        return true;
    }

   private:
    const char* p_;
    const char* e_;
    int depth_ = 0;

    bool fail(const std::string& m) {
        if (err.empty()) err = m;
        return false;
    }
    static const char* kind_of(char c) {
        switch (c) {
            case '[': return "sequence";
            case '"': return "string";
            case 't':
            case 'f': return "boolean";
            case 'n': return "null";
            default: return (c == '-' || (c >= '0' && c <= '9')) ? "number" : "value";
        }
    }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool colon() {
        ws();
        if (p_ < e_ && *p_ == ':') {
            ++p_;
            return true;
        }
        return fail(p_ >= e_ ? "EOF while parsing an object" : "expected `:`");
    }
    bool hex4(uint32_t& v) {
        if (e_ - p_ < 4) return fail("EOF while parsing a string");
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return fail("invalid escape");
        }
        return true;
    }
    bool string(std::string& out) {
        ws();
        if (p_ >= e_) return fail("EOF while parsing a value");
        if (*p_ != '"') return fail(std::string("invalid type: ") + kind_of(*p_) + ", expected a string");
        ++p_;
        while (true) {
            if (p_ >= e_) return fail("EOF while parsing a string");
            const unsigned char c = (unsigned char)*p_++;
            if (c == '"') return true;
            if (c < 0x20) return fail("control character (\\u0000-\\u001F) found while parsing a string");
            if (c != '\\') {
                out.push_back((char)c);
                continue;
            }
            if (p_ >= e_) return fail("EOF while parsing a string");
            const char x = *p_++;
            switch (x) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {
                        if (e_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u')
                            return fail("lone leading surrogate in hex escape");
                        p_ += 2;
                        uint32_t lo;
                        if (!hex4(lo)) return false;
                        if (lo < 0xDC00 || lo > 0xDFFF) return fail("lone leading surrogate in hex escape");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return fail("lone trailing surrogate in hex escape");
                    }
                    utf8_append(out, cp);
                    break;
                }
                default: return fail("invalid escape");
            }
        }
    }
    // A usize: digits only (a sign, fraction or exponent is a type error).
    bool usize(size_t& v) {
        ws();
        if (p_ >= e_) return fail("EOF while parsing a value");
        if (*p_ == '-') return fail("invalid value: integer, expected usize");
        if (*p_ < '0' || *p_ > '9') return fail(std::string("invalid type: ") + kind_of(*p_) + ", expected usize");
        if (*p_ == '0' && p_ + 1 < e_ && p_[1] >= '0' && p_[1] <= '9') return fail("invalid number");
        uint64_t x = 0;
        bool big = false;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_++ - '0');
            if (x > (UINT64_MAX - d) / 10) big = true;
            else x = x * 10 + d;
        }
        if (big || (p_ < e_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')))
            return fail("invalid type: floating point, expected usize");
        v = (size_t)x;
        return true;
    }
    bool literal(const char* lit) {
        const size_t n = strlen(lit);
        if ((size_t)(e_ - p_) < n || memcmp(p_, lit, n) != 0) return fail("expected value");
        p_ += n;
        return true;
    }
    bool skip() {
        ws();
        if (p_ >= e_) return fail("EOF while parsing a value");
        const char c = *p_;
        if (c == '"') {
            std::string s;
            return string(s);
        }
        if (c == 't') return literal("true");
        if (c == 'f') return literal("false");
        if (c == 'n') return literal("null");
        if (c == '[' || c == '{') {
            if (++depth_ > 128) return fail("recursion limit exceeded");
            const char close = c == '[' ? ']' : '}';
            ++p_;
            ws();
            if (p_ < e_ && *p_ == close) {
                ++p_;
                --depth_;
                return true;
            }
            while (true) {
                if (c == '{') {
                    std::string k;
                    if (!string(k) || !colon()) return false;
                }
                if (!skip()) return false;
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == close) {
                    ++p_;
                    --depth_;
                    return true;
                }
                return fail("EOF while parsing a list or object");
            }
        }
        if (c == '-' || (c >= '0' && c <= '9')) {
            ++p_;
            while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                               *p_ == '-'))
                ++p_;
            return true;
        }
        return fail("expected value");
    }
    bool metadata(cfio_file* f) {
        ws();
        if (p_ < e_ && *p_ == 'n') return literal("null");
        if (p_ >= e_ || *p_ != '{')
            return fail(p_ >= e_ ? "EOF while parsing a value"
                                 : std::string("invalid type: ") + kind_of(*p_) + ", expected a map");
        ++p_;
        ws();
        if (p_ < e_ && *p_ == '}') {
            ++p_;
            return true;
        }
        while (true) {
            std::string k, v;
            if (!string(k) || !colon() || !string(v)) return false;
            bool replaced = false;
            for (auto& kv : f->meta)
                if (kv.first == k) {
                    kv.second = v;
                    replaced = true;
                }
            if (!replaced) f->meta.emplace_back(std::move(k), std::move(v));
            ws();
            if (p_ < e_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < e_ && *p_ == '}') {
                ++p_;
                return true;
            }
            return fail("EOF while parsing an object");
        }
    }
    bool usize_list(std::vector<size_t>& out) {
        ws();
        if (p_ >= e_) return fail("EOF while parsing a value");
        if (*p_ != '[') return fail(std::string("invalid type: ") + kind_of(*p_) + ", expected a sequence");
        ++p_;
        ws();
        if (p_ < e_ && *p_ == ']') {
            ++p_;
            return true;
        }
        while (true) {
            size_t v;
            if (!usize(v)) return false;
            out.push_back(v);
            ws();
            if (p_ < e_ && *p_ == ',') {
                ++p_;
                continue;
            }
            if (p_ < e_ && *p_ == ']') {
                ++p_;
                return true;
            }
            return fail("EOF while parsing a list");
        }
    }
    bool record(cfio_file::Tensor& t) {
        ws();
        if (p_ >= e_) return fail("EOF while parsing a value");
        if (*p_ != '{') return fail(std::string("invalid type: ") + kind_of(*p_) + ", expected struct TensorInfo");
        ++p_;
        bool has_dtype = false, has_shape = false, has_offsets = false;
        ws();
        if (p_ < e_ && *p_ == '}') {
            ++p_;
        } else {
            while (true) {
                std::string k;
                if (!string(k) || !colon()) return false;
                if (k == "dtype") {
                    if (has_dtype) return fail("duplicate field `dtype`");
                    std::string d;
                    if (!string(d)) return false;
                    int code = -1;
                    for (int i = 0; i < CFIO_NUM_DTYPES; i++)
                        if (d == kDtypes[i].name) code = i;
                    if (code < 0) return fail("unknown variant `" + d + "`");
                    t.dtype = code;
                    has_dtype = true;
                } else if (k == "shape") {
                    if (has_shape) return fail("duplicate field `shape`");
                    if (!usize_list(t.shape)) return false;
                    has_shape = true;
                } else if (k == "data_offsets") {
                    if (has_offsets) return fail("duplicate field `data_offsets`");
                    std::vector<size_t> o;
                    if (!usize_list(o)) return false;
                    if (o.size() != 2)
                        return fail("invalid length " + std::to_string(o.size()) + ", expected 2 elements in sequence");
                    t.begin = o[0];
                    t.end = o[1];
                    has_offsets = true;
                } else if (!skip()) {
                    return false;
                }
                ws();
                if (p_ < e_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < e_ && *p_ == '}') {
                    ++p_;
                    break;
                }
                return fail("EOF while parsing an object");
            }
        }
        if (!has_dtype) return fail("missing field `dtype`");
        if (!has_shape) return fail("missing field `shape`");
        if (!has_offsets) return fail("missing field `data_offsets`");
        return true;
    }
};

// The crate's Metadata::validate: records ordered by offsets must tile the
// data section from 0, each as long as its elements need.
bool validate(cfio_file* f, uint64_t data_len, std::string* why) {
    std::stable_sort(f->tensors.begin(), f->tensors.end(), [](const cfio_file::Tensor& a, const cfio_file::Tensor& b) {
        return a.begin != b.begin ? a.begin < b.begin : a.end < b.end;
    });
    uint64_t start = 0;
    for (auto& t : f->tensors) {
        if (t.begin != start || t.end < t.begin) {
            *why = "invalid offset for tensor `" + t.name + "`";
            return false;
        }
        start = t.end;
        unsigned __int128 n = 1;
        for (size_t d : t.shape) {
            n *= d;
            if (n > (unsigned __int128)SIZE_MAX) {
                *why = "overflow computing buffer size from shape and/or element type";
                return false;
            }
        }
        const unsigned __int128 bits = n * kDtypes[t.dtype].bits;
        if (bits > (unsigned __int128)SIZE_MAX) {
            *why = "overflow computing buffer size from shape and/or element type";
            return false;
        }
        if (bits % 8) {
            *why =
                "The slice is slicing for subbytes dtypes, and the slice does not end up at a byte boundary, this is "
                "invalid.";
            return false;
        }
        if ((unsigned __int128)(t.end - t.begin) != bits / 8) {
            *why = "invalid shape, data type, or offset for tensor";
            return false;
        }
        t.numel = (size_t)n;
    }
    if (start != data_len) {
        *why = "incomplete metadata, file not fully covered";
        return false;
    }
    return true;
}

// pread / pwrite of a whole range on the calling thread.  Returns 0, an
// errno, or -1 at an early end of file.
int io_range(bool write, int fd, uint8_t* b, size_t n, uint64_t o) {
    while (n) {
        const ssize_t r = write ? pwrite(fd, b, n, (off_t)o) : pread(fd, b, n, (off_t)o);
        if (r < 0) {
            if (errno == EINTR) continue;
            return errno;
        }
        if (r == 0) return -1;
        b += r;
        n -= (size_t)r;
        o += (uint64_t)r;
    }
    return 0;
}

bool file_range(bool write, int fd, uint8_t* buf, size_t len, uint64_t off, std::string* why) {
    const int r = io_range(write, fd, buf, len, off);
    if (r == 0) return true;
    *why = r > 0 ? os_error(r) : (write ? "failed to write whole buffer" : "failed to fill whole buffer");
    return false;
}

// Worker threads that read a staging chunk's file ranges in parallel: one
// thread's page-cache copy runs well below the PCIe rate.  (Writes stay on
// the calling thread: parallel writes to one file measured no faster.)
class ReadPool {
   public:
    struct Task {
        uint8_t* buf;
        size_t len;
        uint64_t off;
    };
    explicit ReadPool(int n) {
        for (int i = 0; i < n; i++) th_.emplace_back([this] { loop(); });
    }
    ~ReadPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : th_) t.join();
    }
    // Reads every task from fd; returns 0, the first errno, or -1 at an early
    // end of file.  The caller's thread takes part.
    int run(int fd, const std::vector<Task>& tasks) {
        if (tasks.empty()) return 0;
        {
            std::lock_guard<std::mutex> lk(mu_);
            fd_ = fd;
            tasks_ = &tasks;
            next_ = 0;
            done_ = 0;
            err_ = 0;
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return done_ == tasks.size(); });
        tasks_ = nullptr;
        return err_;
    }

   private:
    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    const std::vector<Task>* tasks_ = nullptr;
    int fd_ = -1;
    size_t next_ = 0, done_ = 0;
    int err_ = 0;
    unsigned long gen_ = 0;
    bool stop_ = false;

    void work() {
        while (true) {
            Task t;
            int fd;
            {
                std::lock_guard<std::mutex> lk(mu_);
                if (!tasks_ || next_ >= tasks_->size()) return;
                t = (*tasks_)[next_++];
                fd = fd_;
            }
            const int r = io_range(false, fd, t.buf, t.len, t.off);
            std::lock_guard<std::mutex> lk(mu_);
            if (r && !err_) err_ = r;
            if (++done_ == tasks_->size()) done_cv_.notify_all();
        }
    }
    void loop() {
        unsigned long seen = 0;
        while (true) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            work();
        }
    }
};

// Path::with_extension("tmp"): the file name's last extension (a dot not at
// its start) replaced, or ".tmp" appended.
std::string tmp_path(const std::string& path) {
    const size_t slash = path.rfind('/');
    const size_t n0 = slash == std::string::npos ? 0 : slash + 1;
    const std::string name = path.substr(n0);
    const size_t dot = name.rfind('.');
    const std::string stem = (dot == std::string::npos || dot == 0) ? name : name.substr(0, dot);
    return path.substr(0, n0) + stem + ".tmp";
}

// ---- pinned staging --------------------------------------------------------

constexpr int kReadThreads = 8;        // pool workers besides the calling thread
constexpr size_t kReadTask = (size_t)1 << 20;  // bytes per parallel read

struct IoState {
    size_t chunk = 0;
    uint8_t* host[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool busy[2] = {false, false};
    ReadPool pool{kReadThreads};
};

// One staging chunk: the data, then (256-byte aligned) its run table.
size_t stage_bytes(size_t chunk) { return chunk + 256 + (size_t)cfio::kMaxPieces * sizeof(IoPiece); }

void io_release(void* p) {
    IoState* s = static_cast<IoState*>(p);
    for (int k = 0; k < 2; k++) {
        if (s->ev[k]) {
            (void)hipEventSynchronize(s->ev[k]);
            (void)hipEventDestroy(s->ev[k]);
        }
        if (s->host[k]) (void)hipHostFree(s->host[k]);
    }
    delete s;
}

IoState* get_io(cfattn_ctx* c, int* rc) {
    if (c->io) {
        IoState* s = static_cast<IoState*>(c->io);
        if (s->chunk == c->io_chunk) return s;
        io_release(s);
        c->io = nullptr;
    }
    IoState* s = new IoState;
    s->chunk = c->io_chunk;
    for (int k = 0; k < 2; k++) {
        void* h = nullptr;
        hipError_t e = hipHostMalloc(&h, stage_bytes(s->chunk), hipHostMallocDefault);
        if (e == hipSuccess) {
            s->host[k] = static_cast<uint8_t*>(h);
            e = hipEventCreateWithFlags(&s->ev[k], hipEventDisableTiming);
        }
        if (e != hipSuccess) {
            io_release(s);
            *rc = fail(c, CFATTN_ERR_NOMEM, "pinned staging of %zu bytes: %s", stage_bytes(c->io_chunk),
                       hipGetErrorString(e));
            return nullptr;
        }
    }
    c->io = s;
    c->io_release = io_release;
    return s;
}

int wait_chunk(cfattn_ctx* c, IoState* s, int k) {
    if (!s->busy[k]) return CFATTN_OK;
    CF_HIP(c, hipEventSynchronize(s->ev[k]), "staging chunk wait");
    s->busy[k] = false;
    return CFATTN_OK;
}

#define CF_LOCK(c)                                   \
    if (!(c)) return CFATTN_ERR_ARG;                 \
    std::lock_guard<std::mutex> lk((c)->mu);         \
    (c)->err.clear();                                \
    DeviceGuard dev_guard_((c)->device);             \
    if (!dev_guard_.ok) return fail((c), CFATTN_ERR_HIP, "hipSetDevice(%d) failed", (c)->device);

}  // namespace

extern "C" {

const char* cfio_dtype_name(int dtype) {
    return (dtype >= 0 && dtype < CFIO_NUM_DTYPES) ? kDtypes[dtype].name : "?";
}

int cfio_bf16_to_f32(cfattn_ctx* c, const uint16_t* src, float* dst, size_t n, void* stream) {
    CF_LOCK(c);
    if (n && (!src || !dst)) return fail(c, CFATTN_ERR_ARG, "null buffer");
    CF_HIP(c, cfio::launch_widen(false, src, dst, n, to_stream(stream)), "bf16 widen launch");
    return CFATTN_OK;
}

int cfio_f16_to_f32(cfattn_ctx* c, const uint16_t* src, float* dst, size_t n, void* stream) {
    CF_LOCK(c);
    if (n && (!src || !dst)) return fail(c, CFATTN_ERR_ARG, "null buffer");
    CF_HIP(c, cfio::launch_widen(true, src, dst, n, to_stream(stream)), "f16 widen launch");
    return CFATTN_OK;
}

int cfio_st_open(const char* path, cfio_file** out, char* err, size_t err_cap) {
    if (!out) return CFATTN_ERR_ARG;
    *out = nullptr;
    if (!path) {
        put_err(err, err_cap, "null path");
        return CFATTN_ERR_ARG;
    }
    const std::string p(path);
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        put_err(err, err_cap, "cannot open " + p + ": " + os_error(errno));
        return CFATTN_ERR_IO;
    }
    auto bail = [&](const std::string& m) {
        close(fd);
        put_err(err, err_cap, m);
        return CFATTN_ERR_IO;
    };
    struct stat sb;
    if (fstat(fd, &sb) != 0) return bail("cannot mmap " + p + ": " + os_error(errno));
    if (!S_ISREG(sb.st_mode)) return bail("cannot mmap " + p + ": " + os_error(ENODEV));
    const uint64_t size = (uint64_t)sb.st_size;
    if (size < 8) return bail(p + ": header too small");
    uint8_t len8[8];
    std::string why;
    if (!file_range(false, fd, len8, 8, 0, &why)) return bail(p + ": " + why);
    uint64_t n = 0;
    for (int i = 7; i >= 0; i--) n = (n << 8) | len8[i];
    if (n > kMaxHeader) return bail(p + ": header too large");
    if (n + 8 > size) return bail(p + ": invalid header length");
    std::string hdr(n, '\0');
    if (n && !file_range(false, fd, reinterpret_cast<uint8_t*>(&hdr[0]), n, 8, &why)) return bail(p + ": " + why);
    if (!utf8_valid(reinterpret_cast<const unsigned char*>(hdr.data()), n, &why))
        return bail(p + ": invalid UTF-8 in header: " + why);
    cfio_file* f = new cfio_file;
    HeaderParser hp(hdr.data(), hdr.size());
    if (!hp.parse(f)) {
        delete f;
        return bail(p + ": invalid JSON in header: " + hp.err);
    }
    if (!validate(f, size - 8 - n, &why)) {
        delete f;
        return bail(p + ": " + why);
    }
    f->path = p;
    f->fd = fd;
    f->data_start = 8 + n;
    *out = f;
    return CFATTN_OK;
}

int cfio_st_close(cfio_file* f) {
    if (!f) return CFATTN_ERR_ARG;
    if (f->fd >= 0) close(f->fd);
    delete f;
    return CFATTN_OK;
}

size_t cfio_st_count(const cfio_file* f) { return f ? f->tensors.size() : 0; }

int cfio_st_tensor(const cfio_file* f, size_t i, const char** name, int* dtype, size_t* ndim, const size_t** shape,
                   size_t* numel) {
    if (!f || i >= f->tensors.size()) return CFATTN_ERR_ARG;
    const auto& t = f->tensors[i];
    if (name) *name = t.name.c_str();
    if (dtype) *dtype = t.dtype;
    if (ndim) *ndim = t.shape.size();
    if (shape) *shape = t.shape.data();
    if (numel) *numel = t.numel;
    return CFATTN_OK;
}

long long cfio_st_find(const cfio_file* f, const char* name) {
    if (!f || !name) return -1;
    for (size_t i = 0; i < f->tensors.size(); i++)
        if (f->tensors[i].name == name) return (long long)i;
    return -1;
}

size_t cfio_st_meta_count(const cfio_file* f) { return f ? f->meta.size() : 0; }

int cfio_st_meta(const cfio_file* f, size_t i, const char** key, const char** value) {
    if (!f || i >= f->meta.size()) return CFATTN_ERR_ARG;
    if (key) *key = f->meta[i].first.c_str();
    if (value) *value = f->meta[i].second.c_str();
    return CFATTN_OK;
}

int cfio_set_chunk_bytes(cfattn_ctx* c, size_t bytes) {
    CF_LOCK(c);
    if (bytes < ((size_t)1 << 20) || bytes > ((size_t)1 << 30))
        return fail(c, CFATTN_ERR_ARG, "chunk size %zu outside [1 MiB, 1 GiB]", bytes);
    c->io_chunk = (bytes + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
    return CFATTN_OK;
}

int cfio_st_read_f32(cfattn_ctx* c, const cfio_file* f, size_t count, const size_t* idx, float* const* dst,
                     void* stream) {
    CF_LOCK(c);
    if (!f) return fail(c, CFATTN_ERR_ARG, "null file");
    if (count && (!idx || !dst)) return fail(c, CFATTN_ERR_ARG, "null index or destination list");
    struct Job {
        const cfio_file::Tensor* t;
        uint8_t* dst;
        uint32_t kind;
        uint64_t esz;
    };
    std::vector<Job> jobs;
    for (size_t j = 0; j < count; j++) {
        if (idx[j] >= f->tensors.size())
            return fail(c, CFATTN_ERR_ARG, "tensor index %zu out of range (%zu tensors)", idx[j], f->tensors.size());
        const auto& t = f->tensors[idx[j]];
        Job jb{&t, reinterpret_cast<uint8_t*>(dst[j]), 0, 4};
        if (t.dtype == CFIO_F32) jb.kind = cfio::kCopyF32;
        else if (t.dtype == CFIO_BF16) jb = Job{&t, jb.dst, cfio::kWidenBF16, 2};
        else if (t.dtype == CFIO_F16) jb = Job{&t, jb.dst, cfio::kWidenF16, 2};
        else return fail(c, CFATTN_ERR_ARG, "tensor '%s' has unsupported dtype %s", t.name.c_str(), kDtypes[t.dtype].name);
        if (t.numel == 0) continue;
        if (!jb.dst) return fail(c, CFATTN_ERR_ARG, "null destination for tensor '%s'", t.name.c_str());
        if ((uintptr_t)jb.dst % 4) return fail(c, CFATTN_ERR_ARG, "destination of '%s' is not 4-byte aligned", t.name.c_str());
        jobs.push_back(jb);
    }
    if (jobs.empty()) return CFATTN_OK;
    std::stable_sort(jobs.begin(), jobs.end(), [](const Job& a, const Job& b) { return a.t->begin < b.t->begin; });
    int rc = CFATTN_OK;
    IoState* io = get_io(c, &rc);
    if (!io) return rc;
    const size_t sb = stage_bytes(io->chunk);
    uint8_t* dev = static_cast<uint8_t*>(slot(c, cfattn_ctx::IO_STAGE, 2 * sb, &rc));
    if (!dev) return rc;
    const hipStream_t st = to_stream(stream);
    std::vector<IoPiece> pcs;
    std::vector<ReadPool::Task> reads;
    size_t jj = 0;
    uint64_t done = 0;  // bytes of jobs[jj] already staged
    int k = 0;
    while (jj < jobs.size()) {
        CF_TRY(wait_chunk(c, io, k));
        uint8_t* h = io->host[k];
        uint8_t* d = dev + (size_t)k * sb;
        pcs.clear();
        reads.clear();
        size_t pos = 0;
        uint32_t blocks = 0;
        while (jj < jobs.size() && pcs.size() < (size_t)cfio::kMaxPieces) {
            const Job& J = jobs[jj];
            const uint64_t total = J.t->end - J.t->begin;
            const size_t room = (io->chunk - pos) & ~(size_t)15;
            if (room == 0) break;
            const uint64_t take = std::min<uint64_t>(total - done, room);
            for (uint64_t b = 0; b < take; b += kReadTask)
                reads.push_back({h + pos + b, (size_t)std::min<uint64_t>(kReadTask, take - b),
                                 f->data_start + J.t->begin + done + b});
            IoPiece p{};
            p.dev = reinterpret_cast<uint64_t>(J.dst + done / J.esz * 4);
            p.off = (uint32_t)pos;
            p.bytes = (uint32_t)take;
            p.kind = J.kind;
            p.blk0 = blocks;
            blocks += cfio::piece_blocks((uint32_t)take);
            pcs.push_back(p);
            pos = (pos + take + 15) & ~(size_t)15;
            done += take;
            if (done == total) {
                jj++;
                done = 0;
            }
        }
        const int r = io->pool.run(f->fd, reads);
        if (r) {
            const std::string m = r > 0 ? os_error(r) : "failed to fill whole buffer";
            return fail(c, CFATTN_ERR_IO, "%s: %s", f->path.c_str(), m.c_str());
        }
        const size_t toff = (pos + 255) & ~(size_t)255;
        memcpy(h + toff, pcs.data(), pcs.size() * sizeof(IoPiece));
        CF_HIP(c, hipMemcpyAsync(d, h, toff + pcs.size() * sizeof(IoPiece), hipMemcpyHostToDevice, st),
               "staging copy to the device");
        CF_HIP(c, cfio::launch_scatter(d, reinterpret_cast<const IoPiece*>(d + toff), (int)pcs.size(), blocks, st),
               "scatter launch");
        CF_HIP(c, hipEventRecord(io->ev[k], st), "staging event");
        io->busy[k] = true;
        k ^= 1;
    }
    return CFATTN_OK;
}

int cfio_st_write(cfattn_ctx* c, const char* path, size_t count, const char* const* names, const size_t* ndims,
                  const size_t* const* shapes, const float* const* data, size_t n_meta, const char* const* keys,
                  const char* const* values, void* stream) {
    CF_LOCK(c);
    if (!path) return fail(c, CFATTN_ERR_ARG, "null path");
    if (count && (!names || !ndims || !shapes || !data)) return fail(c, CFATTN_ERR_ARG, "null tensor list");
    if (n_meta && (!keys || !values)) return fail(c, CFATTN_ERR_ARG, "null metadata list");
    struct W {
        std::string name;
        std::vector<size_t> shape;
        size_t numel;
        const uint8_t* src;
        uint64_t begin, end;
    };
    std::vector<W> ts(count);
    for (size_t j = 0; j < count; j++) {
        if (!names[j]) return fail(c, CFATTN_ERR_ARG, "null tensor name");
        W& w = ts[j];
        w.name = names[j];
        if (!utf8_valid(reinterpret_cast<const unsigned char*>(w.name.data()), w.name.size(), nullptr))
            return fail(c, CFATTN_ERR_ARG, "tensor name is not valid UTF-8");
        if (ndims[j] && !shapes[j]) return fail(c, CFATTN_ERR_ARG, "null shape of tensor '%s'", w.name.c_str());
        unsigned __int128 n = 1;
        for (size_t d = 0; d < ndims[j]; d++) {
            w.shape.push_back(shapes[j][d]);
            n *= shapes[j][d];
            if (n * 4 > (unsigned __int128)SIZE_MAX) return fail(c, CFATTN_ERR_ARG, "tensor '%s' is too large", w.name.c_str());
        }
        w.numel = (size_t)n;
        w.src = reinterpret_cast<const uint8_t*>(data[j]);
        if (w.numel && !w.src) return fail(c, CFATTN_ERR_ARG, "null data of tensor '%s'", w.name.c_str());
        if ((uintptr_t)w.src % 4) return fail(c, CFATTN_ERR_ARG, "data of '%s' is not 4-byte aligned", w.name.c_str());
    }
    // serialize_to_file's order: dtype (all F32 here), then name byte-wise.
    std::stable_sort(ts.begin(), ts.end(), [](const W& a, const W& b) { return a.name < b.name; });
    for (size_t j = 1; j < ts.size(); j++)
        if (ts[j].name == ts[j - 1].name) return fail(c, CFATTN_ERR_ARG, "duplicate tensor name '%s'", ts[j].name.c_str());
    uint64_t off = 0;
    for (W& w : ts) {
        w.begin = off;
        off += (uint64_t)w.numel * 4;
        w.end = off;
    }
    std::map<std::string, std::string> meta;  // a later duplicate key replaces an earlier one
    for (size_t j = 0; j < n_meta; j++) {
        if (!keys[j] || !values[j]) return fail(c, CFATTN_ERR_ARG, "null metadata entry");
        std::string k = keys[j], v = values[j];
        if (!utf8_valid(reinterpret_cast<const unsigned char*>(k.data()), k.size(), nullptr) ||
            !utf8_valid(reinterpret_cast<const unsigned char*>(v.data()), v.size(), nullptr))
            return fail(c, CFATTN_ERR_ARG, "metadata is not valid UTF-8");
        meta[k] = v;
    }
    std::string hdr = "{";
    bool first = true;
    if (!meta.empty()) {
        hdr += "\"__metadata__\":{";
        bool f1 = true;
        for (const auto& kv : meta) {
            if (!f1) hdr += ",";
            f1 = false;
            json_string(hdr, kv.first);
            hdr += ":";
            json_string(hdr, kv.second);
        }
        hdr += "}";
        first = false;
    }
    for (const W& w : ts) {
        if (!first) hdr += ",";
        first = false;
        json_string(hdr, w.name);
        hdr += ":{\"dtype\":\"F32\",\"shape\":[";
        for (size_t d = 0; d < w.shape.size(); d++) {
            if (d) hdr += ",";
            hdr += std::to_string(w.shape[d]);
        }
        hdr += "],\"data_offsets\":[" + std::to_string(w.begin) + "," + std::to_string(w.end) + "]}";
    }
    hdr += "}";
    hdr.append((8 - hdr.size() % 8) % 8, ' ');

    const std::string final_path(path), tmp = tmp_path(final_path);
    const int fd = open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0666);
    if (fd < 0) return fail(c, CFATTN_ERR_IO, "cannot write %s: %s", path, os_error(errno).c_str());
    auto bail = [&](int code, const std::string& m) {
        close(fd);
        unlink(tmp.c_str());
        return fail(c, code, "%s", m.c_str());
    };
    std::string why;
    {
        std::string head(8, '\0');
        uint64_t n = hdr.size();
        for (int i = 0; i < 8; i++) head[i] = (char)((n >> (8 * i)) & 0xff);
        head += hdr;
        if (!file_range(true, fd, reinterpret_cast<uint8_t*>(&head[0]), head.size(), 0, &why))
            return bail(CFATTN_ERR_IO, "cannot write " + final_path + ": " + why);
    }
    const uint64_t base = 8 + hdr.size();
    if (off) {
        int rc = CFATTN_OK;
        IoState* io = get_io(c, &rc);
        if (!io) return bail(rc, c->err);
        const size_t sb = stage_bytes(io->chunk);
        uint8_t* dev = static_cast<uint8_t*>(slot(c, cfattn_ctx::IO_STAGE, 2 * sb, &rc));
        if (!dev) return bail(rc, c->err);
        const hipStream_t st = to_stream(stream);
        struct Pending {
            bool on = false;
            uint64_t file_off = 0;
            size_t len = 0;
        } pend[2];
        auto flush = [&](int k) -> int {
            if (!pend[k].on) return CFATTN_OK;
            int r = wait_chunk(c, io, k);
            if (r != CFATTN_OK) return r;
            pend[k].on = false;
            if (!file_range(true, fd, io->host[k], pend[k].len, base + pend[k].file_off, &why))
                return fail(c, CFATTN_ERR_IO, "cannot write %s: %s", path, why.c_str());
            return CFATTN_OK;
        };
        std::vector<IoPiece> pcs;
        size_t jj = 0;
        uint64_t done = 0, file_off = 0;
        int k = 0;
        while (jj < ts.size()) {
            int r = flush(k);
            if (r == CFATTN_OK) r = wait_chunk(c, io, k);
            if (r != CFATTN_OK) return bail(r, c->err);
            uint8_t* h = io->host[k];
            uint8_t* d = dev + (size_t)k * sb;
            pcs.clear();
            size_t pos = 0;
            uint32_t blocks = 0;
            while (jj < ts.size() && pcs.size() < (size_t)cfio::kMaxPieces) {
                const W& w = ts[jj];
                const uint64_t total = w.end - w.begin;
                if (total == 0) {
                    jj++;
                    continue;
                }
                const size_t room = (io->chunk - pos) & ~(size_t)3;
                if (room == 0) break;
                const uint64_t take = std::min<uint64_t>(total - done, room);
                IoPiece p{};
                p.dev = reinterpret_cast<uint64_t>(w.src + done);
                p.off = (uint32_t)pos;
                p.bytes = (uint32_t)take;
                p.kind = cfio::kCopyF32;
                p.blk0 = blocks;
                blocks += cfio::piece_blocks((uint32_t)take);
                pcs.push_back(p);
                pos += take;
                done += take;
                if (done == total) {
                    jj++;
                    done = 0;
                }
            }
            if (pcs.empty()) continue;
            const size_t toff = (pos + 255) & ~(size_t)255;
            memcpy(h + toff, pcs.data(), pcs.size() * sizeof(IoPiece));
            hipError_t e = hipMemcpyAsync(d + toff, h + toff, pcs.size() * sizeof(IoPiece), hipMemcpyHostToDevice, st);
            if (e == hipSuccess) e = cfio::launch_gather(d, reinterpret_cast<const IoPiece*>(d + toff), (int)pcs.size(), blocks, st);
            if (e == hipSuccess) e = hipMemcpyAsync(h, d, pos, hipMemcpyDeviceToHost, st);
            if (e == hipSuccess) e = hipEventRecord(io->ev[k], st);
            if (e != hipSuccess) return bail(hip_fail(c, e, "staging copy from the device"), c->err);
            io->busy[k] = true;
            pend[k] = Pending{true, file_off, pos};
            file_off += pos;
            k ^= 1;
        }
        for (int i = 0; i < 2; i++) {
            const int r = flush(i);
            if (r != CFATTN_OK) return bail(r, c->err);
        }
    }
    if (close(fd) != 0) {
        const int e = errno;
        unlink(tmp.c_str());
        return fail(c, CFATTN_ERR_IO, "cannot write %s: %s", path, os_error(e).c_str());
    }
    if (rename(tmp.c_str(), path) != 0)
        return fail(c, CFATTN_ERR_IO, "cannot move %s into place: %s", tmp.c_str(), os_error(errno).c_str());
    return CFATTN_OK;
}

}  // extern "C"
