// pk_container.cpp — picchio's converted checkpoint (config.json + safetensors
// shards) into the HBM store.
//
// Replaces the reference's loading path: cfg_load (picchio.c:349-420), the
// shard discovery of main (picchio.c:2848-2915), load_dense_weights
// (picchio.c:2534-2650) with load_f32_tensor / load_qt_i4
// (picchio.c:2387-2531), and expert_load / load_expert_bias
// (picchio.c:634-888) for every (layer, expert) — the whole model becomes
// resident instead of streamed through the LRU cache. The container format is
// the converter's (convert.py:216-334, :440-470): F32 norms, biases, router,
// sinks and attention; INT8-per-row (or F32) embedding and lm_head with a
// ".qs" tensor of row scales; INT4 experts as uint8 [O][I/2] with ".qs" group
// scales; expert biases F32, aggregated [E][n] or per expert. Embedding,
// lm_head and attention also take load_qt_i4's other forms (BF16 / F16
// quantized to INT4 rows, INT4 rows or groups, INT8 rows).
//
// Host code only: it reads the shards with pread and hands each tensor to the
// engine's store entry points (pk_store_expert / _layer / _globals).
#include "pk_engine.h"

#include <dirent.h>
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <memory>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

// ───────────────────────── a small JSON reader ─────────────────────────
// Enough of RFC 8259 for safetensors headers and config.json: objects,
// arrays, strings (escapes incl. \uXXXX to UTF-8), numbers, true/false/null.
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } k = NUL;
    bool b = false;
    double num = 0.0;
    std::string s;
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;
    const JVal *get(const char *key) const {
        if (k != OBJ) return nullptr;
        for (const auto &kv : o)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JParser {
public:
    JParser(const char *p, size_t n) : p_(p), end_(p + n) {}
    bool parse(JVal &v) {
        if (!value(v, 0)) return false;
        ws();
        return p_ == end_;
    }

private:
    const char *p_, *end_;
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char *w) {
        const size_t n = strlen(w);
        if ((size_t)(end_ - p_) < n || memcmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(std::string &out, uint32_t c) {
        if (c < 0x80) {
            out += (char)c;
        } else if (c < 0x800) {
            out += (char)(0xC0 | (c >> 6));
            out += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            out += (char)(0xE0 | (c >> 12));
            out += (char)(0x80 | ((c >> 6) & 0x3F));
            out += (char)(0x80 | (c & 0x3F));
        } else {
            out += (char)(0xF0 | (c >> 18));
            out += (char)(0x80 | ((c >> 12) & 0x3F));
            out += (char)(0x80 | ((c >> 6) & 0x3F));
            out += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t &c) {
        if (end_ - p_ < 4) return false;
        c = 0;
        for (int i = 0; i < 4; ++i) {
            const char h = *p_++;
            c <<= 4;
            if (h >= '0' && h <= '9') c |= (uint32_t)(h - '0');
            else if (h >= 'a' && h <= 'f') c |= (uint32_t)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') c |= (uint32_t)(h - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool str(std::string &out) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            if (*p_ == '\\') {
                if (++p_ >= end_) return false;
                const char e = *p_++;
                switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t c;
                    if (!hex4(c)) return false;
                    if (c >= 0xD800 && c < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                        p_ += 2;
                        uint32_t lo;
                        if (!hex4(lo)) return false;
                        c = 0x10000 + ((c - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(out, c);
                    break;
                }
                default: return false;
                }
            } else {
                out += *p_++;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool value(JVal &v, int depth) {
        if (depth > 64) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            v.k = JVal::OBJ;
            ++p_;
            ws();
            if (p_ < end_ && *p_ == '}') { ++p_; return true; }
            for (;;) {
                ws();
                std::string key;
                if (!str(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                v.o.emplace_back(std::move(key), JVal());
                if (!value(v.o.back().second, depth + 1)) return false;
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') { ++p_; return true; }
                return false;
            }
        }
        if (c == '[') {
            v.k = JVal::ARR;
            ++p_;
            ws();
            if (p_ < end_ && *p_ == ']') { ++p_; return true; }
            for (;;) {
                v.a.emplace_back();
                if (!value(v.a.back(), depth + 1)) return false;
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') { ++p_; return true; }
                return false;
            }
        }
        if (c == '"') {
            v.k = JVal::STR;
            return str(v.s);
        }
        if (lit("true")) { v.k = JVal::BOOL; v.b = true; return true; }
        if (lit("false")) { v.k = JVal::BOOL; v.b = false; return true; }
        if (lit("null")) { v.k = JVal::NUL; return true; }
        // number
        const char *q = p_;
        if (q < end_ && (*q == '-' || *q == '+')) ++q;
        while (q < end_ && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' || *q == '-' ||
                            *q == '+'))
            ++q;
        if (q == p_) return false;
        const std::string t(p_, q);
        char *ep = nullptr;
        v.num = strtod(t.c_str(), &ep);
        if (!ep || *ep) return false;
        v.k = JVal::NUM;
        p_ = q;
        return true;
    }
};

bool read_text(const std::string &path, std::string &out) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    fclose(f);
    return true;
}

// ───────────────────────── safetensors shards ─────────────────────────
enum StType { ST_F32, ST_F16, ST_BF16, ST_I32, ST_I16, ST_I8, ST_U8, ST_F64, ST_BOOL, ST_BAD };

StType st_type(const std::string &s) {
    static const char *names[] = {"F32", "F16", "BF16", "I32", "I16", "I8", "U8", "F64", "BOOL"};
    for (int i = 0; i < 9; ++i)
        if (s == names[i]) return (StType)i;
    return ST_BAD;
}
int st_size(StType t) {
    switch (t) {
    case ST_F32: case ST_I32: return 4;
    case ST_F16: case ST_BF16: case ST_I16: return 2;
    case ST_I8: case ST_U8: case ST_BOOL: return 1;
    case ST_F64: return 8;
    default: return 0;
    }
}

struct StTensor {
    int file = -1;
    StType dtype = ST_BAD;
    std::vector<int64_t> shape;
    int64_t begin = 0, end = 0;       // absolute byte range in the file
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        return n;
    }
};

// Every tensor of the container's shards by name (the first shard that holds
// a name wins, as st_find over the opened files does).
class StDb {
public:
    ~StDb() {
        for (int fd : fds_) close(fd);
    }
    int open_file(const std::string &path) {
        const int fd = open(path.c_str(), O_RDONLY);
        PK_CHECK(fd >= 0, PK_ERR_MISSING, "container: cannot open %s", path.c_str());
        fds_.push_back(fd);
        const int fi = (int)fds_.size() - 1;
        struct stat stt;
        PK_CHECK(fstat(fd, &stt) == 0, PK_ERR_ARG, "container: stat %s", path.c_str());
        const int64_t fsize = stt.st_size;
        uint8_t lb[8];
        PK_CHECK(pread(fd, lb, 8, 0) == 8, PK_ERR_ARG, "container: %s: no header", path.c_str());
        uint64_t hlen = 0;
        for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | lb[i];
        PK_CHECK(hlen > 1 && (int64_t)hlen <= fsize - 8 && hlen < ((uint64_t)1 << 30), PK_ERR_ARG,
                 "container: %s: header length %llu", path.c_str(), (unsigned long long)hlen);
        std::string h(hlen, '\0');
        PK_CHECK(pread(fd, &h[0], hlen, 8) == (ssize_t)hlen, PK_ERR_ARG, "container: %s: short header",
                 path.c_str());
        JVal root;
        PK_CHECK(JParser(h.data(), h.size()).parse(root) && root.k == JVal::OBJ, PK_ERR_ARG,
                 "container: %s: header is not a JSON object", path.c_str());
        const int64_t base = 8 + (int64_t)hlen;
        for (const auto &kv : root.o) {
            if (kv.first == "__metadata__") continue;
            const JVal &d = kv.second;
            const JVal *dt = d.get("dtype"), *sh = d.get("shape"), *of = d.get("data_offsets");
            PK_CHECK(dt && dt->k == JVal::STR && sh && sh->k == JVal::ARR && of && of->k == JVal::ARR &&
                         of->a.size() == 2,
                     PK_ERR_ARG, "container: %s: bad entry %s", path.c_str(), kv.first.c_str());
            StTensor t;
            t.file = fi;
            t.dtype = st_type(dt->s);
            for (const JVal &x : sh->a) {
                PK_CHECK(x.k == JVal::NUM && x.num >= 0, PK_ERR_ARG, "container: %s: bad shape",
                         kv.first.c_str());
                t.shape.push_back((int64_t)x.num);
            }
            t.begin = base + (int64_t)of->a[0].num;
            t.end = base + (int64_t)of->a[1].num;
            PK_CHECK(t.begin <= t.end && t.end <= fsize, PK_ERR_ARG, "container: %s: %s outside the file",
                     path.c_str(), kv.first.c_str());
            PK_CHECK(t.dtype == ST_BAD || t.numel() * st_size(t.dtype) == t.end - t.begin, PK_ERR_ARG,
                     "container: %s: %s has %lld bytes for its shape", path.c_str(), kv.first.c_str(),
                     (long long)(t.end - t.begin));
            tensors_.emplace(kv.first, std::move(t));    // first shard wins
        }
        return PK_OK;
    }
    const StTensor *find(const std::string &name) const {
        auto it = tensors_.find(name);
        return it == tensors_.end() ? nullptr : &it->second;
    }
    // n bytes from byte `off` of the tensor's data
    int read(const StTensor &t, void *dst, int64_t off, int64_t n) const {
        PK_CHECK(off >= 0 && n >= 0 && t.begin + off + n <= t.end, PK_ERR_ARG, "container: read past a tensor");
        char *p = (char *)dst;
        int64_t pos = t.begin + off;
        while (n > 0) {
            const ssize_t r = pread(fds_[t.file], p, (size_t)std::min<int64_t>(n, (int64_t)1 << 30), pos);
            PK_CHECK(r > 0, PK_ERR_ARG, "container: read failed");
            p += r;
            pos += r;
            n -= r;
        }
        return PK_OK;
    }
    size_t n_files() const { return fds_.size(); }

private:
    std::vector<int> fds_;
    std::unordered_map<std::string, StTensor> tensors_;
};

// Shards in the reference's order (picchio.c:2848-2915): dense.safetensors,
// model.safetensors, model-NNNNN-of-NNNNN.safetensors (HF), then the
// converter's model-NNNNN.safetensors and experts-NN.safetensors.
int open_container(const std::string &dir, StDb &db) {
    std::vector<std::string> names;
    if (DIR *d = opendir(dir.c_str())) {
        while (dirent *ent = readdir(d)) names.emplace_back(ent->d_name);
        closedir(d);
    }
    PK_CHECK(!names.empty(), PK_ERR_MISSING, "container: cannot list %s", dir.c_str());
    std::sort(names.begin(), names.end());
    auto is_digits = [](const std::string &s, size_t a, size_t n) {
        if (s.size() < a + n) return false;
        for (size_t i = a; i < a + n; ++i)
            if (s[i] < '0' || s[i] > '9') return false;
        return true;
    };
    std::vector<std::string> order;
    for (const char *fixed : {"dense.safetensors", "model.safetensors"})
        if (std::find(names.begin(), names.end(), fixed) != names.end()) order.push_back(fixed);
    for (const auto &n : names)       // model-00001-of-00003.safetensors
        if (n.size() == 32 && n.compare(0, 6, "model-") == 0 && is_digits(n, 6, 5) && n.compare(11, 4, "-of-") == 0 &&
            is_digits(n, 15, 5) && n.compare(20, 12, ".safetensors") == 0)
            order.push_back(n);
    for (const auto &n : names)       // model-00000.safetensors
        if (n.size() == 23 && n.compare(0, 6, "model-") == 0 && is_digits(n, 6, 5) &&
            n.compare(11, 12, ".safetensors") == 0)
            order.push_back(n);
    for (const auto &n : names)       // experts-00.safetensors
        if (n.size() == 22 && n.compare(0, 8, "experts-") == 0 && is_digits(n, 8, 2) &&
            n.compare(10, 12, ".safetensors") == 0)
            order.push_back(n);
    PK_CHECK(!order.empty(), PK_ERR_MISSING, "container: no safetensors shard in %s", dir.c_str());
    for (const auto &n : order) PK_TRY(db.open_file(dir + "/" + n));
    return PK_OK;
}

// ───────────────────────── tensor conversions ─────────────────────────
float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
// load_f32_tensor's F16 rule (picchio.c:2412-2429): subnormals to signed zero
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16, ex = (h >> 10) & 0x1F, man = h & 0x3FF;
    uint32_t f;
    if (ex == 0) f = sign;
    else if (ex == 31) f = sign | 0x7F800000u | (man << 13);
    else f = sign | ((ex + 112) << 23) | (man << 13);
    float r;
    memcpy(&r, &f, 4);
    return r;
}

// An F32 / BF16 / F16 tensor of n values as fp32 (load_f32_tensor,
// picchio.c:2387-2436). Missing: PK_ERR_MISSING (the callers decide).
int read_f32(const StDb &db, const std::string &name, int64_t n, std::vector<float> &out) {
    const StTensor *t = db.find(name);
    if (!t) {
        pk_set_error("container: tensor %s not found", name.c_str());
        return PK_ERR_MISSING;
    }
    PK_CHECK(t->numel() == n, PK_ERR_ARG, "container: %s has %lld values, expected %lld", name.c_str(),
             (long long)t->numel(), (long long)n);
    out.resize(n);
    if (t->dtype == ST_F32) return db.read(*t, out.data(), 0, n * 4);
    PK_CHECK(t->dtype == ST_BF16 || t->dtype == ST_F16, PK_ERR_UNSUPPORTED, "container: %s: dtype %d",
             name.c_str(), (int)t->dtype);
    std::vector<uint16_t> h(n);
    PK_TRY(db.read(*t, h.data(), 0, n * 2));
    for (int64_t i = 0; i < n; ++i) out[i] = t->dtype == ST_BF16 ? bf16_to_f32(h[i]) : f16_to_f32(h[i]);
    return PK_OK;
}

// Optional tensors: the reference's default when absent (norms 1.0,
// picchio.c:2563-2569, :2580-2585; biases and router bias absent = 0, which
// adds nothing).
int read_f32_or(const StDb &db, const std::string &name, int64_t n, float dflt, std::vector<float> &out) {
    if (!db.find(name)) {
        out.assign(n, dflt);
        return PK_OK;
    }
    return read_f32(db, name, n, out);
}

std::string fmtname(const char *fmt, int a, int b = 0) {
    char buf[320];
    snprintf(buf, sizeof buf, fmt, a, b);
    return buf;
}

// An INT4 group-scaled expert matrix [O][I] (expert_load's U8 branch,
// picchio.c:760-790 / :832-859): packed nibbles + ".qs" scales; the group
// size is O*I / n_scales (picchio.c:781-784), which must be gs.
struct I4Host {
    std::vector<uint8_t> q;
    std::vector<float> s;
};
int read_i4(const StDb &db, const std::vector<std::string> &names, const std::vector<std::string> &qs_names,
            int O, int I, int gs, I4Host &out, std::string &found) {
    const StTensor *t = nullptr;
    for (const auto &n : names)
        if ((t = db.find(n))) { found = n; break; }
    if (!t) {
        pk_set_error("container: expert tensor %s not found", names[0].c_str());
        return PK_ERR_MISSING;
    }
    PK_CHECK(t->dtype == ST_U8, PK_ERR_UNSUPPORTED,
             "container: %s is dtype %d; the expert store holds INT4 (uint8 + .qs) experts from convert.py",
             found.c_str(), (int)t->dtype);
    const int64_t rb = (int64_t)O * ((I + 1) / 2);
    PK_CHECK(t->numel() == rb, PK_ERR_ARG, "container: %s: %lld bytes, expected %lld", found.c_str(),
             (long long)t->numel(), (long long)rb);
    const StTensor *ts = nullptr;
    for (const auto &n : qs_names)
        if ((ts = db.find(n))) break;
    PK_CHECK(ts && ts->dtype == ST_F32, PK_ERR_UNSUPPORTED, "container: %s: no F32 .qs scales", found.c_str());
    const int64_t ns = ts->numel();
    PK_CHECK(ns > O && (int64_t)O * I / ns == gs && ns == (int64_t)O * ((I + gs - 1) / gs), PK_ERR_UNSUPPORTED,
             "container: %s: %lld scales for [%d,%d] (group size %d expected)", found.c_str(), (long long)ns, O,
             I, gs);
    out.q.resize(rb);
    out.s.resize(ns);
    PK_TRY(db.read(*t, out.q.data(), 0, rb));
    return db.read(*ts, out.s.data(), 0, ns * 4);
}

// load_expert_bias (picchio.c:634-696): per-expert or aggregated [E][n]
// tensor, F32, or the legacy INT4 bias (uint8 or F32-stored bytes + .qs, gs
// 64) of an aggregated tensor, dequantized q * scale as the reference does.
int read_expert_bias(const StDb &db, int layer, int eid, const char *suffix, int n_experts, int n,
                     std::vector<float> &out) {
    std::string name = fmtname("model.layers.%d.mlp.experts.%d.", layer, eid) + suffix;
    const StTensor *t = db.find(name);
    bool aggregated = false;
    if (!t) {
        name = fmtname("model.layers.%d.mlp.experts.", layer) + suffix;
        t = db.find(name);
        aggregated = t != nullptr;
    }
    if (!t) {
        pk_set_error("container: expert bias %s (layer %d expert %d) not found", suffix, layer, eid);
        return PK_ERR_MISSING;
    }
    out.assign(n, 0.0f);
    const StTensor *ts = db.find(name + ".qs");
    const bool full_f32 = t->dtype == ST_F32 && t->numel() == (int64_t)n_experts * n;
    if (aggregated && ts && !full_f32) {
        const int packed_n = (n + 1) / 2, groups = (n + 63) / 64;
        std::vector<uint8_t> packed(packed_n);
        std::vector<float> sc(groups);
        if (t->dtype == ST_F32) {
            std::vector<float> stored(packed_n);
            PK_TRY(db.read(*t, stored.data(), (int64_t)eid * packed_n * 4, (int64_t)packed_n * 4));
            for (int i = 0; i < packed_n; ++i) packed[i] = (uint8_t)lrintf(stored[i]);
        } else {
            PK_CHECK(t->dtype == ST_U8, PK_ERR_UNSUPPORTED, "container: %s: dtype %d", name.c_str(),
                     (int)t->dtype);
            PK_TRY(db.read(*t, packed.data(), (int64_t)eid * packed_n, packed_n));
        }
        PK_TRY(db.read(*ts, sc.data(), (int64_t)eid * groups * 4, (int64_t)groups * 4));
        for (int i = 0; i < n; ++i) {
            const uint8_t byte = packed[i >> 1];
            const int q = (i & 1) ? (int)(byte >> 4) - 8 : (int)(byte & 0x0F) - 8;
            out[i] = (float)q * sc[i / 64];
        }
        return PK_OK;
    }
    PK_CHECK(t->dtype == ST_F32, PK_ERR_UNSUPPORTED, "container: %s: dtype %d", name.c_str(), (int)t->dtype);
    const int64_t off = aggregated ? (int64_t)eid * n * 4 : 0;
    PK_CHECK(t->end - t->begin >= off + (int64_t)n * 4, PK_ERR_ARG, "container: %s is too short", name.c_str());
    return db.read(*t, out.data(), off, (int64_t)n * 4);
}

// quantize_rows_i4 (quant.h:366-392): per row s = amax / 7 (at least
// 1e-8), v = lrintf(w / s) clipped to [-8, 7]. Values are kept signed
// (nibble - 8), one per byte.
void quantize_rows_i4(const float *w, int64_t r0, int64_t r1, int I, int8_t *q, float *s) {
    for (int64_t o = r0; o < r1; ++o) {
        const float *wr = w + o * I;
        float amax = 0.0f;
        for (int i = 0; i < I; ++i) amax = std::max(amax, fabsf(wr[i]));
        float sc = amax / 7.0f;
        if (sc < 1e-8f) sc = 1e-8f;
        s[o] = sc;
        for (int i = 0; i < I; ++i) {
            int v = (int)lrintf(wr[i] / sc);
            q[o * I + i] = (int8_t)std::min(7, std::max(-8, v));
        }
    }
}

// A dense matrix [O][I] in the form load_qt_i4 (picchio.c:2443-2531) leaves
// it: F32 kept F32; I8 rows with ".qs" row scales; U8 nibbles with ".qs"
// row scales, group scales (more scales than rows: group size O*I/n), or
// none (every row scale 1.0); BF16 / F16 quantized to INT4 rows. ROWS and
// GROUPS hold the signed values (nibble - 8 for INT4) one per byte.
struct QtHost {
    enum Kind { F32, ROWS, GROUPS };
    Kind kind = F32;
    int O = 0, I = 0, gs = 0;
    std::vector<float> f;
    std::vector<int8_t> q;
    std::vector<float> s;
    // (float)q * scale per value: embed_token's product (picchio.c:1482-1502)
    void dequant(std::vector<float> &out) const {
        if (kind == F32) {
            out = f;
            return;
        }
        out.resize((int64_t)O * I);
        const int ng = kind == GROUPS ? (I + gs - 1) / gs : 1;
        for (int64_t o = 0; o < O; ++o)
            for (int i = 0; i < I; ++i)
                out[o * I + i] = (float)q[o * I + i] * s[o * ng + (kind == GROUPS ? i / gs : 0)];
    }
};

// What load_qt_i4 makes of a tensor, from its dtype and the ".qs" beside it,
// with the sizes checked (the reference reads what the shapes say; a short
// tensor or scale vector is an error here).
int qt_layout(const StDb &db, const std::string &name, int O, int I, QtHost::Kind &kind, int &gs) {
    const StTensor *t = db.find(name);
    if (!t) {
        pk_set_error("container: tensor %s not found", name.c_str());
        return PK_ERR_MISSING;
    }
    gs = 0;
    const int64_t n = (int64_t)O * I;
    const StTensor *ts = db.find(name + ".qs");
    if (t->dtype == ST_F32 || t->dtype == ST_BF16 || t->dtype == ST_F16) {
        PK_CHECK(t->numel() == n, PK_ERR_ARG, "container: %s has %lld values, expected %lld", name.c_str(),
                 (long long)t->numel(), (long long)n);
        kind = t->dtype == ST_F32 ? QtHost::F32 : QtHost::ROWS;
        return PK_OK;
    }
    if (t->dtype == ST_I8) {
        PK_CHECK(t->numel() == n && ts && ts->dtype == ST_F32 && ts->numel() == O, PK_ERR_ARG,
                 "container: INT8 %s needs [%d,%d] values and %d F32 row scales", name.c_str(), O, I, O);
        kind = QtHost::ROWS;
        return PK_OK;
    }
    PK_CHECK(t->dtype == ST_U8, PK_ERR_UNSUPPORTED, "container: %s dtype %d", name.c_str(), (int)t->dtype);
    PK_CHECK(t->numel() == (int64_t)O * ((I + 1) / 2), PK_ERR_ARG, "container: INT4 %s: %lld bytes for [%d,%d]",
             name.c_str(), (long long)t->numel(), O, I);
    kind = QtHost::ROWS;
    if (!ts) return PK_OK;
    PK_CHECK(ts->dtype == ST_F32, PK_ERR_ARG, "container: %s.qs is not F32", name.c_str());
    const int64_t ns = ts->numel();
    if (ns > O) {
        gs = (int)(n / ns);
        if (gs <= 0) gs = 64;
        PK_CHECK(ns == (int64_t)O * ((I + gs - 1) / gs), PK_ERR_ARG,
                 "container: %s: %lld scales for [%d,%d] and group size %d", name.c_str(), (long long)ns, O, I, gs);
        kind = QtHost::GROUPS;
        return PK_OK;
    }
    PK_CHECK(ns == O, PK_ERR_ARG, "container: %s: %lld scales for %d rows", name.c_str(), (long long)ns, O);
    return PK_OK;
}

int read_qt(const StDb &db, const std::string &name, int O, int I, int n_threads, QtHost &out) {
    PK_TRY(qt_layout(db, name, O, I, out.kind, out.gs));
    out.O = O;
    out.I = I;
    const StTensor *t = db.find(name);
    const StTensor *ts = db.find(name + ".qs");
    const int64_t n = (int64_t)O * I;
    if (t->dtype == ST_F32) return read_f32(db, name, n, out.f);
    if (t->dtype == ST_BF16 || t->dtype == ST_F16) {
        std::vector<float> w;
        PK_TRY(read_f32(db, name, n, w));
        out.q.resize(n);
        out.s.resize(O);
        const int nt = std::max(1, std::min(n_threads, 64));
        std::vector<std::thread> pool;
        for (int k = 0; k < nt; ++k)
            pool.emplace_back(quantize_rows_i4, w.data(), (int64_t)O * k / nt, (int64_t)O * (k + 1) / nt, I,
                              out.q.data(), out.s.data());
        for (auto &th : pool) th.join();
        return PK_OK;
    }
    out.q.resize(n);
    if (t->dtype == ST_I8) {
        out.s.resize(O);
        PK_TRY(db.read(*t, out.q.data(), 0, n));
        return db.read(*ts, out.s.data(), 0, (int64_t)O * 4);
    }
    const int64_t rb = (I + 1) / 2;
    std::vector<uint8_t> packed((int64_t)O * rb);
    PK_TRY(db.read(*t, packed.data(), 0, (int64_t)packed.size()));
    for (int64_t o = 0; o < O; ++o)
        for (int i = 0; i < I; ++i) {
            const uint8_t byte = packed[o * rb + (i >> 1)];
            out.q[o * I + i] = (int8_t)(((i & 1) ? byte >> 4 : byte & 0x0F) - 8);
        }
    if (!ts) {
        out.s.assign(O, 1.0f);
        return PK_OK;
    }
    out.s.resize(ts->numel());
    return db.read(*ts, out.s.data(), 0, (int64_t)out.s.size() * 4);
}

// The engine's lm_head formats for load_qt_i4's results: INT4 or INT8 rows
// as INT8 rows (matmul_i4 and matmul_q8 are the same sum of x * q times the
// row scale, quant.h:152-257); F32 and group-scaled INT4 as F32.
int lm_head_fmt_of(QtHost::Kind k) { return k == QtHost::ROWS ? PK_FMT_INT8 : PK_FMT_F32; }

// cfg_load's reads (picchio.c:349-420). The reference looks a key up
// anywhere in the text, so the rope_scaling entries (factor, beta_fast, ...)
// are found inside their object; here: top level first, then rope_scaling.
const JVal *cfg_key(const JVal &root, const char *k) {
    if (const JVal *v = root.get(k)) return v;
    if (const JVal *rs = root.get("rope_scaling"))
        if (const JVal *v = rs->get(k)) return v;
    return nullptr;
}
double cfg_num(const JVal &root, const char *k, double dflt) {
    const JVal *v = cfg_key(root, k);
    return v && v->k == JVal::NUM ? v->num : dflt;
}
bool cfg_bool(const JVal &root, const char *k, bool dflt) {
    const JVal *v = cfg_key(root, k);
    if (v && v->k == JVal::BOOL) return v->b;
    if (v && v->k == JVal::NUM) return v->num != 0;
    return dflt;
}

}  // namespace

extern "C" int pk_cfg_from_container(const char *dir, int ctx_len, pk_cfg *out) {
    PK_CHECK(dir && out, PK_ERR_ARG, "null argument");
    std::string text;
    PK_CHECK(read_text(std::string(dir) + "/config.json", text), PK_ERR_MISSING, "container: %s/config.json",
             dir);
    JVal root;
    PK_CHECK(JParser(text.data(), text.size()).parse(root) && root.k == JVal::OBJ, PK_ERR_ARG,
             "container: config.json is not a JSON object");
    pk_cfg c;
    memset(&c, 0, sizeof c);
    c.hidden = (int)cfg_num(root, "hidden_size", 2880);
    c.n_layers = (int)cfg_num(root, "num_hidden_layers", 36);
    c.n_heads = (int)cfg_num(root, "num_attention_heads", 64);
    c.n_kv_heads = (int)cfg_num(root, "num_key_value_heads", 8);
    c.head_dim = (int)cfg_num(root, "head_dim", 64);
    c.n_experts = (int)cfg_num(root, "num_local_experts", 128);
    c.topk = (int)cfg_num(root, "num_experts_per_tok", 4);
    c.moe_inter = (int)cfg_num(root, "intermediate_size", 2880) * 2;
    c.vocab = (int)cfg_num(root, "vocab_size", 201088);
    const int max_pos = (int)cfg_num(root, "max_position_embeddings", 131072);
    c.ctx_len = ctx_len > 0 ? ctx_len : max_pos;
    c.sliding_window = (int)cfg_num(root, "sliding_window", 128);
    c.eps = (float)cfg_num(root, "rms_norm_eps", 1e-5);
    c.theta = (float)cfg_num(root, "rope_theta", 150000.0);
    c.rope_factor = (float)cfg_num(root, "factor", 1.0);
    c.rope_beta_fast = (float)cfg_num(root, "beta_fast", 32.0);
    c.rope_beta_slow = (float)cfg_num(root, "beta_slow", 1.0);
    // the reference's default is its own ctx_len, i.e. max_position_embeddings
    c.rope_original_ctx = (int)cfg_num(root, "original_max_position_embeddings", max_pos);
    c.rope_truncate = cfg_bool(root, "truncate", true) ? 1 : 0;
    c.rope_attn_factor = c.rope_factor > 1.0f ? 0.1f * logf(c.rope_factor) + 1.0f : 1.0f;
    c.swiglu_limit = (float)cfg_num(root, "swiglu_limit", 7.0);
    c.swiglu_alpha = 1.702f;
    c.routed_scale = (float)cfg_num(root, "routed_scaling_factor", 1.0);
    PK_CHECK(c.n_layers > 0 && c.n_layers <= 128, PK_ERR_UNSUPPORTED, "container: %d layers", c.n_layers);
    const JVal *lt = root.get("layer_types");
    if (lt && lt->k == JVal::ARR && !lt->a.empty()) {
        const int nt = (int)lt->a.size();
        for (int i = 0; i < c.n_layers; ++i) {
            const JVal &s = lt->a[i % nt];
            c.layer_type[i] = s.k == JVal::STR && s.s.find("full") != std::string::npos ? 1 : 0;
        }
    } else {
        for (int i = 0; i < c.n_layers; ++i) c.layer_type[i] = (int8_t)(i % 2);
    }
    // read from the checkpoint: the expert group size (picchio.c:781-784)
    // and the lm_head format
    StDb db;
    PK_TRY(open_container(dir, db));
    c.group_size = 64;
    for (const char *fmt : {"model.layers.%d.mlp.experts.gate_up_proj.%d.qs",
                            "model.layers.%d.mlp.experts.%d.gate_up_proj.qs"}) {
        if (const StTensor *ts = db.find(fmtname(fmt, 0, 0))) {
            const int64_t ns = ts->numel();
            if (ns > c.moe_inter) c.group_size = (int)((int64_t)c.moe_inter * c.hidden / ns);
            break;
        }
    }
    QtHost::Kind lm_kind;
    int lm_gs;
    PK_TRY(qt_layout(db, "lm_head.weight", c.vocab, c.hidden, lm_kind, lm_gs));
    c.lm_head_fmt = lm_head_fmt_of(lm_kind);
    *out = c;
    return PK_OK;
}

extern "C" int pk_load_container(pk_engine *e, const char *dir, int n_threads) {
    PK_CHECK(e && dir, PK_ERR_ARG, "null argument");
    const pk_cfg *c = &e->c;
    const int D = c->hidden, H = c->n_heads, KVH = c->n_kv_heads, hd = c->head_dim, E = c->n_experts;
    const int V = c->vocab, I = c->moe_inter, Id = c->moe_inter / 2;
    StDb db;
    PK_TRY(open_container(dir, db));

    // ── globals (load_dense_weights, picchio.c:2546-2575) ──
    {
        const int nt = std::max(1, std::min(n_threads > 0 ? n_threads : 8, 64));
        std::vector<float> emb, lmf, fn;
        {
            QtHost et;
            PK_TRY(read_qt(db, "model.embed_tokens.weight", V, D, nt, et));
            et.dequant(emb);
        }
        QtHost lt;
        PK_TRY(read_qt(db, "lm_head.weight", V, D, nt, lt));
        PK_CHECK(lm_head_fmt_of(lt.kind) == c->lm_head_fmt, PK_ERR_ARG,
                 "container: lm_head format %d, engine built for %d", lm_head_fmt_of(lt.kind), c->lm_head_fmt);
        pk_qt_host eh{PK_FMT_F32, emb.data(), nullptr, V, D, 0};
        pk_qt_host lh{};
        if (lt.kind == QtHost::ROWS) {
            lh = pk_qt_host{PK_FMT_INT8, lt.q.data(), lt.s.data(), V, D, 0};
        } else {
            lt.dequant(lmf);
            lh = pk_qt_host{PK_FMT_F32, lmf.data(), nullptr, V, D, 0};
        }
        PK_TRY(read_f32_or(db, "model.norm.weight", D, 1.0f, fn));
        PK_TRY(pk_store_globals(e, &eh, &lh, fn.data()));
    }

    // ── dense tensors of each layer (picchio.c:2577-2642) ──
    for (int l = 0; l < c->n_layers; ++l) {
        std::vector<float> in_ln, post_ln, wq, wk, wv, wo, bq, bk, bv, bo, sinks, router, rbias;
        auto p = [l](const char *rest) { return fmtname("model.layers.%d.", l) + rest; };
        PK_TRY(read_f32_or(db, p("input_layernorm.weight"), D, 1.0f, in_ln));
        PK_TRY(read_f32_or(db, p("post_attention_layernorm.weight"), D, 1.0f, post_ln));
        // attention is F32 in the converter's output (convert.py:305-309) and
        // stays F32; load_qt_i4's other forms (INT8 rows, INT4 rows or groups,
        // BF16/F16 quantized to INT4 rows) are held as their fp32 values
        // q * scale, so the projections compute sum(x * q * s) where
        // matmul_q8 / matmul_i4 compute sum(x * q) * s
        {
            QtHost t;
            const int nt = std::max(1, std::min(n_threads > 0 ? n_threads : 8, 64));
            PK_TRY(read_qt(db, p("self_attn.q_proj.weight"), H * hd, D, nt, t));
            t.dequant(wq);
            PK_TRY(read_qt(db, p("self_attn.k_proj.weight"), KVH * hd, D, nt, t));
            t.dequant(wk);
            PK_TRY(read_qt(db, p("self_attn.v_proj.weight"), KVH * hd, D, nt, t));
            t.dequant(wv);
            PK_TRY(read_qt(db, p("self_attn.o_proj.weight"), D, H * hd, nt, t));
            t.dequant(wo);
        }
        PK_TRY(read_f32_or(db, p("self_attn.q_proj.bias"), H * hd, 0.0f, bq));
        PK_TRY(read_f32_or(db, p("self_attn.k_proj.bias"), KVH * hd, 0.0f, bk));
        PK_TRY(read_f32_or(db, p("self_attn.v_proj.bias"), KVH * hd, 0.0f, bv));
        PK_TRY(read_f32_or(db, p("self_attn.o_proj.bias"), D, 0.0f, bo));
        PK_TRY(read_f32(db, p("self_attn.sinks"), H, sinks));
        int rc = read_f32(db, p("mlp.router.weight"), (int64_t)E * D, router);
        if (rc == PK_ERR_MISSING) rc = read_f32(db, p("block_sparse_moe.gate.weight"), (int64_t)E * D, router);
        PK_TRY(rc);
        PK_TRY(read_f32_or(db, p("mlp.router.bias"), E, 0.0f, rbias));
        pk_layer_host lh{};
        lh.in_ln = in_ln.data();
        lh.post_ln = post_ln.data();
        lh.wq = pk_qt_host{PK_FMT_F32, wq.data(), nullptr, H * hd, D, 0};
        lh.wk = pk_qt_host{PK_FMT_F32, wk.data(), nullptr, KVH * hd, D, 0};
        lh.wv = pk_qt_host{PK_FMT_F32, wv.data(), nullptr, KVH * hd, D, 0};
        lh.wo = pk_qt_host{PK_FMT_F32, wo.data(), nullptr, D, H * hd, 0};
        lh.bq = bq.data(); lh.bk = bk.data(); lh.bv = bv.data(); lh.bo = bo.data();
        lh.sinks = sinks.data();
        lh.router = router.data();
        lh.router_bias = rbias.data();
        PK_TRY(pk_store_layer(e, l, &lh));
    }

    // ── experts (expert_load for every (layer, expert)): read in parallel,
    //    stored in order by this thread ──
    struct Ex {
        I4Host gu, dn;
        std::vector<float> gb, db;
        int rc = PK_OK;
        std::string err;
    };
    const int nt = std::max(1, std::min(n_threads > 0 ? n_threads : 8, 64));
    for (int l = 0; l < c->n_layers; ++l) {
        std::vector<Ex> ex(E);
        auto work = [&](int first) {
            for (int x = first; x < E; x += nt) {
                Ex &r = ex[x];
                std::string found;
                auto both = [&](const char *proj) {
                    return std::vector<std::string>{
                        fmtname("model.layers.%d.mlp.experts.", l) + proj + "." + std::to_string(x),
                        fmtname("model.layers.%d.mlp.experts.%d.", l, x) + proj,
                        fmtname("model.layers.%d.mlp.experts.%d.", l, x) + proj + ".weight"};
                };
                auto qs = [&](const char *proj) {
                    return std::vector<std::string>{
                        fmtname("model.layers.%d.mlp.experts.", l) + proj + "." + std::to_string(x) + ".qs",
                        fmtname("model.layers.%d.mlp.experts.%d.", l, x) + proj + ".qs"};
                };
                r.rc = read_i4(db, both("gate_up_proj"), qs("gate_up_proj"), I, D, c->group_size, r.gu, found);
                if (r.rc == PK_OK)
                    r.rc = read_i4(db, both("down_proj"), qs("down_proj"), D, Id, c->group_size, r.dn, found);
                if (r.rc == PK_OK) r.rc = read_expert_bias(db, l, x, "gate_up_proj_bias", E, I, r.gb);
                if (r.rc == PK_OK) r.rc = read_expert_bias(db, l, x, "down_proj_bias", E, D, r.db);
                if (r.rc != PK_OK) r.err = pk_last_error();
            }
        };
        std::vector<std::thread> pool;
        for (int t = 0; t < nt; ++t) pool.emplace_back(work, t);
        for (auto &t : pool) t.join();
        for (int x = 0; x < E; ++x) {
            if (ex[x].rc != PK_OK) {
                pk_set_error("%s", ex[x].err.c_str());
                return ex[x].rc;
            }
            const pk_qt_host gu{PK_FMT_INT4, ex[x].gu.q.data(), ex[x].gu.s.data(), I, D, c->group_size};
            const pk_qt_host dn{PK_FMT_INT4, ex[x].dn.q.data(), ex[x].dn.s.data(), D, Id, c->group_size};
            PK_TRY(pk_store_expert(e, l, x, &gu, &dn, ex[x].gb.data(), ex[x].db.data()));
            ex[x] = Ex();
        }
    }
    return pk_engine_sync(e);
}
