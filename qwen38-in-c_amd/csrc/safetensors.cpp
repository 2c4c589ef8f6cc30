// safetensors.cpp -- header parsing and indexing of safetensors shards.
// Only the structure the format uses is parsed: a JSON object of objects
// with string, integer-array and nested-object values.
#include "safetensors.h"

#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>

namespace q35mm {
namespace st {

size_t dtype_size(int d) {
    switch (d) {
    case kF8E4M3: return 1;
    case kBF16: return 2;
    case kF16: return 2;
    case kF32: return 4;
    case kI64: return 8;
    default: return 0;
    }
}

const char *dtype_name(int d) {
    switch (d) {
    case kF8E4M3: return "F8_E4M3";
    case kBF16: return "BF16";
    case kF16: return "F16";
    case kF32: return "F32";
    case kI64: return "I64";
    default: return "UNKNOWN";
    }
}

static int dtype_of(const std::string &s) {
    static const char *names[] = {"F8_E4M3", "BF16", "F32", "F16", "I64"};
    static const int codes[] = {kF8E4M3, kBF16, kF32, kF16, kI64};
    for (int i = 0; i < 5; i++)
        if (s == names[i]) return codes[i];
    return kUnknown;
}

bool is_shard_name(const char *name) {
    return strstr(name, ".safetensors") != nullptr && strstr(name, "json") == nullptr;
}

const char *status_str(int s) {
    switch (s) {
    case kOk: return "ok";
    case kOpen: return "cannot open";
    case kHeader: return "bad safetensors header";
    case kDtype: return "unsupported dtype";
    case kRange: return "tensor range out of file";
    case kIo: return "io error";
    default: return "unknown";
    }
}

namespace {

// ---- a small JSON reader ------------------------------------------------
struct JValue {
    enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
    bool integral = false;     // a number without fraction or exponent
    uint64_t u = 0;            // its value, when integral and non-negative
    double num = 0;
    std::string str;
    std::vector<JValue> items;                                  // array
    std::vector<std::pair<std::string, JValue>> members;        // object, in order

    const JValue *get(const char *key) const {
        for (const auto &m : members)
            if (m.first == key) return &m.second;
        return nullptr;
    }
};

class JParser {
  public:
    JParser(const char *p, size_t n) : p_(p), end_(p + n) {}

    bool parse(JValue &out) {
        if (!value(out, 0)) return false;
        ws();
        return p_ == end_;
    }

  private:
    const char *p_, *end_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(const char *s) {
        const size_t n = strlen(s);
        if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(std::string &o, uint32_t c) {
        if (c < 0x80) {
            o += (char)c;
        } else if (c < 0x800) {
            o += (char)(0xC0 | (c >> 6));
            o += (char)(0x80 | (c & 63));
        } else if (c < 0x10000) {
            o += (char)(0xE0 | (c >> 12));
            o += (char)(0x80 | ((c >> 6) & 63));
            o += (char)(0x80 | (c & 63));
        } else {
            o += (char)(0xF0 | (c >> 18));
            o += (char)(0x80 | ((c >> 12) & 63));
            o += (char)(0x80 | ((c >> 6) & 63));
            o += (char)(0x80 | (c & 63));
        }
    }
    bool hex4(uint32_t &v) {
        if (end_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string &o) {
        if (p_ >= end_ || *p_ != '"') return false;
        p_++;
        while (p_ < end_ && *p_ != '"') {
            const char c = *p_++;
            if ((unsigned char)c < 0x20) return false;
            if (c != '\\') {
                o += c;
                continue;
            }
            if (p_ >= end_) return false;
            const char e = *p_++;
            switch (e) {
            case '"': o += '"'; break;
            case '\\': o += '\\'; break;
            case '/': o += '/'; break;
            case 'b': o += '\b'; break;
            case 'f': o += '\f'; break;
            case 'n': o += '\n'; break;
            case 'r': o += '\r'; break;
            case 't': o += '\t'; break;
            case 'u': {
                uint32_t c1;
                if (!hex4(c1)) return false;
                if (c1 >= 0xD800 && c1 < 0xDC00) {   // surrogate pair
                    uint32_t c2;
                    if (!lit("\\u") || !hex4(c2) || c2 < 0xDC00 || c2 >= 0xE000) return false;
                    c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
                }
                utf8(o, c1);
                break;
            }
            default: return false;
            }
        }
        if (p_ >= end_) return false;
        p_++;
        return true;
    }
    bool number(JValue &v) {
        const char *s = p_;
        bool neg = false;
        if (p_ < end_ && *p_ == '-') {
            neg = true;
            p_++;
        }
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
        uint64_t u = 0;
        bool overflow = false;
        while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
            const uint64_t d = (uint64_t)(*p_++ - '0');
            if (u > (UINT64_MAX - d) / 10) overflow = true;
            u = u * 10 + d;
        }
        bool frac = false;
        if (p_ < end_ && *p_ == '.') {
            frac = true;
            p_++;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            frac = true;
            p_++;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) p_++;
            if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
        }
        v.kind = JValue::kNumber;
        v.num = strtod(std::string(s, (size_t)(p_ - s)).c_str(), nullptr);
        v.integral = !frac && !neg && !overflow;
        v.u = v.integral ? u : 0;
        return true;
    }
    bool value(JValue &v, int depth) {
        if (depth > 32) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            p_++;
            v.kind = JValue::kObject;
            ws();
            if (p_ < end_ && *p_ == '}') {
                p_++;
                return true;
            }
            for (;;) {
                ws();
                std::pair<std::string, JValue> m;
                if (!string(m.first)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                p_++;
                if (!value(m.second, depth + 1)) return false;
                v.members.push_back(std::move(m));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    p_++;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            p_++;
            v.kind = JValue::kArray;
            ws();
            if (p_ < end_ && *p_ == ']') {
                p_++;
                return true;
            }
            for (;;) {
                JValue item;
                if (!value(item, depth + 1)) return false;
                v.items.push_back(std::move(item));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    p_++;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v.kind = JValue::kString;
            return string(v.str);
        }
        if (lit("true")) {
            v.kind = JValue::kBool;
            v.u = 1;
            return true;
        }
        if (lit("false")) {
            v.kind = JValue::kBool;
            return true;
        }
        if (lit("null")) {
            v.kind = JValue::kNull;
            return true;
        }
        return number(v);
    }
};

bool read_full(int fd, uint64_t off, uint64_t len, void *dst) {
    uint8_t *d = static_cast<uint8_t *>(dst);
    while (len) {
        const ssize_t got = pread(fd, d, len > (1u << 30) ? (1u << 30) : (size_t)len, (off_t)off);
        if (got <= 0) return false;
        d += got;
        off += (uint64_t)got;
        len -= (uint64_t)got;
    }
    return true;
}

// Persistent reader threads: run(n, fn) calls fn(0..n-1) on the workers
// and the caller and returns when all calls are done.  Never destroyed (its
// idle threads end with the process).
class ReadPool {
  public:
    static ReadPool &get() {
        static ReadPool *p = new ReadPool();
        return *p;
    }

    void run(int n, const std::function<void(int)> &fn) {
        std::lock_guard<std::mutex> one(run_mu_);
        {
            std::lock_guard<std::mutex> lk(mu_);
            fn_ = &fn;
            n_ = n;
            next_ = 0;
            done_ = 0;
            gen_++;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return done_ == n_; });
        fn_ = nullptr;
    }

  private:
    static constexpr int kWorkers = 3;

    ReadPool() {
        for (int i = 0; i < kWorkers; i++)
            std::thread([this] {
                uint64_t seen = 0;
                for (;;) {
                    {
                        std::unique_lock<std::mutex> lk(mu_);
                        cv_.wait(lk, [&] { return gen_ != seen; });
                        seen = gen_;
                    }
                    work();
                }
            }).detach();
    }

    void work() {
        std::unique_lock<std::mutex> lk(mu_);
        while (fn_ && next_ < n_) {
            const int k = next_++;
            const std::function<void(int)> *fn = fn_;
            lk.unlock();
            (*fn)(k);
            lk.lock();
            if (++done_ == n_) done_cv_.notify_all();
        }
    }

    std::mutex run_mu_, mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(int)> *fn_ = nullptr;
    int n_ = 0, next_ = 0, done_ = 0;
    uint64_t gen_ = 0;
};

}  // namespace

bool Archive::read_parallel(const Tensor &t, uint64_t off, uint64_t len, void *dst) const {
    constexpr uint64_t kPart = 2u << 20;   // bytes per reader call
    if (len <= kPart) return read(t, off, len, dst);
    const int n = (int)((len + kPart - 1) / kPart);
    std::vector<char> ok((size_t)n, 0);
    ReadPool::get().run(n, [&](int k) {
        const uint64_t o = (uint64_t)k * kPart, e = std::min(len, o + kPart);
        ok[(size_t)k] = read(t, off + o, e - o, static_cast<uint8_t *>(dst) + o) ? 1 : 0;
    });
    for (char c : ok)
        if (!c) return false;
    return true;
}

Archive::~Archive() {
    for (int fd : fds)
        if (fd >= 0) ::close(fd);
}

int Archive::index_file(const std::string &path, uint32_t file, std::string &msg) {
    msg = path;
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return kOpen;
    fds.push_back(fd);
    paths.push_back(path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) return kIo;
    const uint64_t fsize = (uint64_t)sb.st_size;
    uint8_t h8[8];
    if (fsize < 8 || !read_full(fd, 0, 8, h8)) return kHeader;
    uint64_t hlen = 0;
    for (int i = 0; i < 8; i++) hlen |= (uint64_t)h8[i] << (8 * i);
    if (hlen == 0 || hlen > (1u << 24) || 8 + hlen > fsize) return kHeader;
    std::string text(hlen, '\0');
    if (!read_full(fd, 8, hlen, &text[0])) return kHeader;
    JValue root;
    if (!JParser(text.data(), text.size()).parse(root) || root.kind != JValue::kObject) return kHeader;
    const uint64_t base = 8 + hlen;
    for (const auto &m : root.members) {
        const JValue &tv = m.second;
        if (m.first == "__metadata__" || tv.kind != JValue::kObject) continue;
        msg = path + ": " + m.first;
        const JValue *dt = tv.get("dtype");
        const JValue *shape = tv.get("shape");
        const JValue *offs = tv.get("data_offsets");
        const int d = (dt && dt->kind == JValue::kString) ? dtype_of(dt->str) : kUnknown;
        if (d == kUnknown) return kDtype;
        if (!shape || shape->kind != JValue::kArray || shape->items.size() > 8 || !offs ||
            offs->kind != JValue::kArray || offs->items.size() != 2)
            return kHeader;
        for (const JValue &x : offs->items)
            if (x.kind != JValue::kNumber || !x.integral) return kHeader;
        const uint64_t o0 = offs->items[0].u, o1 = offs->items[1].u;
        if (o1 < o0 || o1 > fsize || base + o1 > fsize) return kRange;
        Tensor t;
        t.name = m.first;
        t.dtype = d;
        t.ndim = (uint32_t)shape->items.size();
        uint64_t elems = 1;
        for (uint32_t k = 0; k < t.ndim; k++) {
            const JValue &x = shape->items[k];
            if (x.kind != JValue::kNumber || !x.integral || x.u > UINT32_MAX) return kHeader;
            t.shape[k] = (uint32_t)x.u;
            if (x.u && elems > UINT64_MAX / x.u) return kRange;
            elems *= x.u;
        }
        if (elems > UINT64_MAX / dtype_size(d) || elems * dtype_size(d) != o1 - o0) return kRange;
        t.file = file;
        t.offset = base + o0;
        t.bytes = o1 - o0;
        if (index.emplace(t.name, (uint32_t)tensors.size()).second)   // a repeated name keeps its first entry
            tensors.push_back(std::move(t));
    }
    msg.clear();
    return kOk;
}

int Archive::open(const char *path, std::string &msg) {
    struct stat sb;
    if (!path || stat(path, &sb) != 0) {
        msg = path ? path : "(null)";
        return kOpen;
    }
    if (!S_ISDIR(sb.st_mode)) return index_file(path, 0, msg);
    std::unique_ptr<DIR, int (*)(DIR *)> dir(opendir(path), closedir);
    if (!dir) {
        msg = path;
        return kOpen;
    }
    std::vector<std::string> names;
    while (const dirent *e = readdir(dir.get()))
        if (is_shard_name(e->d_name)) names.push_back(e->d_name);
    std::sort(names.begin(), names.end());
    if (names.empty()) {
        msg = std::string(path) + ": no safetensors shards";
        return kOpen;
    }
    std::string base(path);
    if (base.back() != '/') base += '/';
    for (const std::string &n : names) {
        const int s = index_file(base + n, (uint32_t)paths.size(), msg);
        if (s != kOk) return s;
    }
    return kOk;
}

const Tensor *Archive::find(const char *name) const {
    auto it = index.find(name);
    return it == index.end() ? nullptr : &tensors[it->second];
}

bool Archive::read(const Tensor &t, uint64_t off, uint64_t len, void *dst) const {
    if (t.file >= fds.size() || off > t.bytes || len > t.bytes - off) return false;
    return read_full(fds[t.file], t.offset + off, len, dst);
}

}  // namespace st
}  // namespace q35mm
