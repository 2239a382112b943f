// The checkpoint file format (Checkpoint.cs:48-649): writer, and a reader that checks an untrusted file in the
// reference's order — header, manifest, fit against the target, tensor extents — before returning any data.
#include "checkpoint.hpp"

#include <sys/stat.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <limits>
#include <memory>

namespace omt {
namespace ckpt {
namespace {

constexpr uint64_t kHeader = 64;
constexpr uint64_t kMaxManifest = 256ull << 20;
constexpr int kMaxDepth = 32;

[[noreturn]] void fail(Kind k, const std::string &m) { throw Failure(k, m); }

uint64_t align64(uint64_t v) { return (v + 63) & ~uint64_t(63); }

void put_u32(unsigned char *p, uint32_t v) {
    for (int i = 0; i < 4; i++) p[i] = (unsigned char)(v >> (8 * i));
}
void put_u64(unsigned char *p, uint64_t v) {
    for (int i = 0; i < 8; i++) p[i] = (unsigned char)(v >> (8 * i));
}
uint32_t get_u32(const unsigned char *p) {
    uint32_t v = 0;
    for (int i = 3; i >= 0; i--) v = (v << 8) | p[i];
    return v;
}
uint64_t get_u64(const unsigned char *p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; i--) v = (v << 8) | p[i];
    return v;
}

// ------------------------------------------------------------------------------------------------ JSON reading
// A strict RFC 8259 reader over a UTF-8 manifest: no comments, no trailing commas, nesting at most kMaxDepth,
// strings with valid escapes and no lone surrogates. Numbers keep whether they are integers that fit in int64
// (no fraction or exponent), which is what the manifest's integer fields require.
struct JVal {
    enum Type { Null, Bool, Num, Str, Arr, Obj } type = Null;
    bool b = false;
    bool is_int = false;
    int64_t i = 0;
    std::string s;
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;

    const JVal *get(const char *key) const {
        if (type != Obj) return nullptr;
        for (auto it = o.rbegin(); it != o.rend(); ++it)  // a repeated name: the last one counts
            if (it->first == key) return &it->second;
        return nullptr;
    }
};

bool valid_utf8(const unsigned char *p, size_t n) {
    size_t i = 0;
    while (i < n) {
        unsigned c = p[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int len;
        uint32_t cp;
        if (c >= 0xC2 && c <= 0xDF) {
            len = 2;
            cp = c & 0x1F;
        } else if (c >= 0xE0 && c <= 0xEF) {
            len = 3;
            cp = c & 0x0F;
        } else if (c >= 0xF0 && c <= 0xF4) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + len > n) return false;
        for (int k = 1; k < len; k++) {
            if ((p[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (p[i + k] & 0x3F);
        }
        if ((len == 3 && cp < 0x800) || (len == 4 && (cp < 0x10000 || cp > 0x10FFFF)) ||
            (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += len;
    }
    return true;
}

class Reader {
   public:
    Reader(const char *p, size_t n) : p_(p), end_(p + n) {}
    JVal document() {
        JVal v = value(0);
        ws();
        if (p_ != end_) bad("trailing characters after the JSON value");
        return v;
    }

   private:
    const char *p_, *end_;
    [[noreturn]] void bad(const char *what) { fail(BadManifest, std::string("The manifest is not valid JSON: ") + what); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(const char *w) {
        size_t n = std::strlen(w);
        if ((size_t)(end_ - p_) >= n && std::memcmp(p_, w, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    JVal value(int depth) {
        ws();
        if (p_ == end_) bad("unexpected end");
        JVal v;
        const char c = *p_;
        if (c == '{' || c == '[') {
            if (depth + 1 > kMaxDepth) bad("nested too deeply");
            p_++;
            ws();
            const char close = c == '{' ? '}' : ']';
            v.type = c == '{' ? JVal::Obj : JVal::Arr;
            if (p_ < end_ && *p_ == close) {
                p_++;
                return v;
            }
            for (;;) {
                if (v.type == JVal::Obj) {
                    ws();
                    if (p_ == end_ || *p_ != '"') bad("expected a property name");
                    std::string key = string();
                    ws();
                    if (p_ == end_ || *p_ != ':') bad("expected ':'");
                    p_++;
                    v.o.emplace_back(std::move(key), value(depth + 1));
                } else {
                    v.a.push_back(value(depth + 1));
                }
                ws();
                if (p_ == end_) bad("unexpected end");
                if (*p_ == ',') {
                    p_++;
                    continue;
                }
                if (*p_ == close) {
                    p_++;
                    return v;
                }
                bad("expected ',' or a closing bracket");
            }
        }
        if (c == '"') {
            v.type = JVal::Str;
            v.s = string();
            return v;
        }
        if (lit("true")) {
            v.type = JVal::Bool;
            v.b = true;
            return v;
        }
        if (lit("false")) {
            v.type = JVal::Bool;
            return v;
        }
        if (lit("null")) return v;
        if (c == '-' || (c >= '0' && c <= '9')) return number();
        bad("unexpected character");
    }
    JVal number() {
        const char *s = p_;
        if (*p_ == '-') p_++;
        if (p_ == end_) bad("bad number");
        if (*p_ == '0') {
            p_++;
        } else if (*p_ >= '1' && *p_ <= '9') {
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
        } else {
            bad("bad number");
        }
        bool integer = true;
        if (p_ < end_ && *p_ == '.') {
            integer = false;
            p_++;
            if (p_ == end_ || !(*p_ >= '0' && *p_ <= '9')) bad("bad number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
        }
        if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
            integer = false;
            p_++;
            if (p_ < end_ && (*p_ == '+' || *p_ == '-')) p_++;
            if (p_ == end_ || !(*p_ >= '0' && *p_ <= '9')) bad("bad number");
            while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
        }
        JVal v;
        v.type = JVal::Num;
        if (integer) {
            // decimal digits into int64 with overflow detection
            const char *q = s;
            const bool neg = *q == '-';
            if (neg) q++;
            uint64_t mag = 0;
            bool fits = true;
            for (; q < p_; q++) {
                const uint64_t d = (uint64_t)(*q - '0');
                if (mag > (std::numeric_limits<uint64_t>::max() - d) / 10) {
                    fits = false;
                    break;
                }
                mag = mag * 10 + d;
            }
            const uint64_t lim = neg ? (uint64_t)std::numeric_limits<int64_t>::max() + 1
                                     : (uint64_t)std::numeric_limits<int64_t>::max();
            if (fits && mag <= lim) {
                v.is_int = true;
                v.i = neg ? (int64_t)(0 - mag) : (int64_t)mag;
            }
        }
        return v;
    }
    static int hex(char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        return -1;
    }
    uint32_t u4() {
        if (end_ - p_ < 4) bad("bad \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; k++) {
            const int h = hex(p_[k]);
            if (h < 0) bad("bad \\u escape");
            v = (v << 4) | (uint32_t)h;
        }
        p_ += 4;
        return v;
    }
    static void utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char)cp;
        } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18));
            out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
        }
    }
    std::string string() {
        p_++;  // opening quote
        std::string out;
        for (;;) {
            if (p_ == end_) bad("unterminated string");
            const unsigned char c = (unsigned char)*p_;
            if (c == '"') {
                p_++;
                return out;
            }
            if (c < 0x20) bad("control character in a string");
            if (c != '\\') {
                out += (char)c;
                p_++;
                continue;
            }
            p_++;
            if (p_ == end_) bad("unterminated escape");
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
                    uint32_t cp = u4();
                    if (cp >= 0xD800 && cp <= 0xDBFF) {
                        if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') bad("lone surrogate in a string");
                        p_ += 2;
                        const uint32_t lo = u4();
                        if (lo < 0xDC00 || lo > 0xDFFF) bad("lone surrogate in a string");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
                        bad("lone surrogate in a string");
                    }
                    utf8(out, cp);
                    break;
                }
                default: bad("bad escape");
            }
        }
    }
};

// The manifest accessors of Checkpoint.cs:449-480: a missing field or one of the wrong kind is a BadManifest.
const std::string &str(const JVal &o, const char *name) {
    const JVal *v = o.get(name);
    if (!v || v->type != JVal::Str) fail(BadManifest, std::string("Manifest field '") + name + "' is missing or not a string.");
    return v->s;
}
int64_t integer(const JVal &o, const char *name) {
    const JVal *v = o.get(name);
    if (!v || v->type != JVal::Num || !v->is_int)
        fail(BadManifest, std::string("Manifest field '") + name + "' is missing or not an integer.");
    return v->i;
}
const JVal &arr(const JVal &o, const char *name) {
    const JVal *v = o.get(name);
    if (!v || v->type != JVal::Arr) fail(BadManifest, std::string("Manifest field '") + name + "' is missing or not an array.");
    return *v;
}

struct Entry {
    std::string name;
    DType dtype;
    std::vector<int> dims;
    int64_t offset, length;
};

// Checkpoint.Entries (Checkpoint.cs:334-364).
std::vector<Entry> entries(const JVal &array) {
    std::vector<Entry> out;
    for (const JVal &e : array.a) {
        Entry x;
        x.name = str(e, "name");
        const std::string &dt = str(e, "dtype");
        if (dt == "f32") x.dtype = F32;
        else if (dt == "i32") x.dtype = I32;
        else if (dt == "i64") x.dtype = I64;
        else fail(BadManifest, "Tensor '" + x.name + "' has unsupported dtype '" + dt + "'.");
        for (const JVal &d : arr(e, "shape").a) {
            if (d.type != JVal::Num || !d.is_int || d.i < 0 || d.i > std::numeric_limits<int32_t>::max())
                fail(BadManifest, "Tensor '" + x.name + "' has a bad dimension.");
            x.dims.push_back((int)d.i);
        }
        x.offset = integer(e, "offset");
        x.length = integer(e, "length");
        out.push_back(std::move(x));
    }
    return out;
}

std::string dims_str(const std::vector<int> &d) {
    std::string s = "[";
    for (size_t i = 0; i < d.size(); i++) s += (i ? "," : "") + std::to_string(d[i]);
    return s + "]";
}

// Offset and length inside the data region, checked without overflow (Checkpoint.cs:386-391).
void check_extent(const char *what, const Entry &e, int64_t expected, int64_t data_len) {
    if (e.length != expected || e.offset < 0 || e.offset > data_len || e.length > data_len - e.offset)
        fail(BadTensor, std::string(what) + " tensor '" + e.name + "' has offset " + std::to_string(e.offset) +
                            ", length " + std::to_string(e.length) + " (expected " + std::to_string(expected) +
                            ") in a data region of " + std::to_string(data_len) + " bytes.");
}

// Checkpoint.CheckFit (Checkpoint.cs:367-392): count, then per entry names/types/shapes (Mismatch) before extents.
void check_fit(const std::vector<Entry> &es, const std::vector<Tensor> &dest, int64_t data_len) {
    if (es.size() != dest.size())
        fail(Mismatch, "The checkpoint has " + std::to_string(es.size()) + " model tensors, the target has " +
                           std::to_string(dest.size()) + ".");
    for (size_t i = 0; i < es.size(); i++) {
        const Entry &e = es[i];
        const Tensor &t = dest[i];
        if (e.name != t.name || e.dtype != t.dtype || e.dims != t.dims)
            fail(Mismatch, "model entry " + std::to_string(i) + " is '" + e.name + "' " + dims_str(e.dims) +
                               ", the target expects '" + t.name + "' " + dims_str(t.dims) + ".");
        check_extent("model", e, t.bytes(), data_len);
    }
}

// Checkpoint.CheckFitOptimizerState (Checkpoint.cs:394-419): a state entry may also be empty ([0]) or its
// parameter's shape (Optimizer.CanAdoptState, Optimizers.cs:135-144).
void check_fit_state(const std::vector<Entry> &es, const Optimizer &opt, int64_t data_len) {
    if (es.size() != opt.state.size())
        fail(Mismatch, "The checkpoint has " + std::to_string(es.size()) + " optimizer state tensors, the target has " +
                           std::to_string(opt.state.size()) + ".");
    for (size_t i = 0; i < es.size(); i++) {
        const Entry &e = es[i];
        const Tensor &t = opt.state[i];
        const bool param = i < opt.param_dims.size() && !opt.param_dims[i].empty();
        const bool adopt = param && t.dtype == F32 &&
                           (e.dims == opt.param_dims[i] || (e.dims.size() == 1 && e.dims[0] == 0));
        if (e.name != t.name || e.dtype != t.dtype || !(e.dims == t.dims || adopt))
            fail(Mismatch, "optimizer state entry " + std::to_string(i) + " is '" + e.name + "' " + dims_str(e.dims) +
                               ", the target expects '" + t.name + "' " + dims_str(t.dims) + ".");
        int64_t n = 1;
        for (int d : e.dims) n *= d;  // bounded: the shape equals the target's or its parameter's, or is [0]
        check_extent("optimizer state", e, n * elem_size(e.dtype), data_len);
    }
}

// ------------------------------------------------------------------------------------------------ JSON writing
// Utf8JsonWriter's compact output with its default escaping: quote, backslash and control characters, the
// HTML-sensitive & < > ' + `, and everything outside ASCII, as \uXXXX (short forms for \b \t \n \f \r).
void jstr(std::string &out, const std::string &s) {
    static const char *hexd = "0123456789ABCDEF";
    auto u = [&](uint32_t cp) {
        out += "\\u";
        for (int k = 3; k >= 0; k--) out += hexd[(cp >> (4 * k)) & 15];
    };
    out += '"';
    size_t i = 0;
    while (i < s.size()) {
        const unsigned char c = (unsigned char)s[i];
        if (c >= 0x80) {  // decode one UTF-8 sequence (names are validated UTF-8) and escape it as UTF-16
            int len = c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : 2;
            uint32_t cp = c & (len == 4 ? 0x07 : len == 3 ? 0x0F : 0x1F);
            for (int k = 1; k < len && i + k < s.size(); k++) cp = (cp << 6) | ((unsigned char)s[i + k] & 0x3F);
            if (cp >= 0x10000) {
                cp -= 0x10000;
                u(0xD800 + (cp >> 10));
                u(0xDC00 + (cp & 0x3FF));
            } else {
                u(cp);
            }
            i += len;
            continue;
        }
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\b': out += "\\b"; break;
            case '\t': out += "\\t"; break;
            case '\n': out += "\\n"; break;
            case '\f': out += "\\f"; break;
            case '\r': out += "\\r"; break;
            case '&': case '<': case '>': case '\'': case '+': case '`': u(c); break;
            default:
                if (c < 0x20) u(c);
                else out += (char)c;
        }
        i++;
    }
    out += '"';
}

const char *dtype_name(DType t) { return t == F32 ? "f32" : t == I32 ? "i32" : "i64"; }

void jentries(std::string &out, const std::vector<Tensor> &ts, const std::vector<uint64_t> &offsets, size_t base) {
    out += '[';
    for (size_t i = 0; i < ts.size(); i++) {
        if (i) out += ',';
        out += "{\"name\":";
        jstr(out, ts[i].name);
        out += ",\"dtype\":\"";
        out += dtype_name(ts[i].dtype);
        out += "\",\"shape\":[";
        for (size_t d = 0; d < ts[i].dims.size(); d++) out += (d ? "," : "") + std::to_string(ts[i].dims[d]);
        out += "],\"offset\":" + std::to_string(offsets[base + i]) + ",\"length\":" + std::to_string(ts[i].bytes()) + "}";
    }
    out += ']';
}

struct File {
    FILE *f = nullptr;
    ~File() {
        if (f) std::fclose(f);
    }
};

}  // namespace

void save(const std::string &path, const std::vector<Tensor> &model, const Optimizer *opt,
          const std::map<std::string, int64_t> &extra) {
    std::vector<const Tensor *> all;
    for (const Tensor &t : model) all.push_back(&t);
    if (opt)
        for (const Tensor &t : opt->state) all.push_back(&t);
    // data region: model tensors then optimizer state, each at a multiple of 64 (Checkpoint.cs:91-99)
    std::vector<uint64_t> offsets;
    uint64_t cursor = 0;
    for (const Tensor *t : all) {
        offsets.push_back(cursor);
        cursor = align64(cursor + (uint64_t)t->bytes());
    }
    std::string m = "{\"format\":\"onemodel-checkpoint\",\"version\":1,\"model\":";
    jentries(m, model, offsets, 0);
    if (opt) {
        m += ",\"optimizer\":{\"kind\":";
        jstr(m, opt->kind);
        m += ",\"step\":" + std::to_string(opt->step) + ",\"hyper\":[";
        for (size_t i = 0; i < opt->hyper.size(); i++) {
            uint32_t bits;
            std::memcpy(&bits, &opt->hyper[i].second, 4);
            m += i ? ",{\"name\":" : "{\"name\":";
            jstr(m, opt->hyper[i].first);
            m += ",\"bits\":" + std::to_string(bits) + "}";
        }
        m += "],\"state\":";
        jentries(m, opt->state, offsets, model.size());
        m += '}';
    }
    m += ",\"extra\":[";
    bool first = true;
    for (const auto &kv : extra) {  // std::map: ordinal key order
        m += first ? "{\"key\":" : ",{\"key\":";
        first = false;
        jstr(m, kv.first);
        m += ",\"value\":" + std::to_string(kv.second) + "}";
    }
    m += "]}";

    const uint64_t data_offset = align64(kHeader + m.size());
    unsigned char header[kHeader] = {0};
    std::memcpy(header, "ONEMCKPT", 8);
    put_u32(header + 8, 1);
    put_u64(header + 16, kHeader);
    put_u64(header + 24, m.size());
    put_u64(header + 32, data_offset);
    put_u64(header + 40, cursor);
    put_u64(header + 48, data_offset + cursor);

    const std::string tmp = path + ".tmp";
    {
        File f;
        f.f = std::fopen(tmp.c_str(), "wb");
        if (!f.f) throw std::runtime_error("cannot create " + tmp + ": " + std::strerror(errno));
        static const char zeros[64] = {0};
        bool ok = std::fwrite(header, 1, kHeader, f.f) == kHeader && std::fwrite(m.data(), 1, m.size(), f.f) == m.size() &&
                  std::fwrite(zeros, 1, data_offset - kHeader - m.size(), f.f) == data_offset - kHeader - m.size();
        uint64_t written = 0;
        for (size_t i = 0; ok && i < all.size(); i++) {
            const uint64_t pad = offsets[i] - written;
            ok = std::fwrite(zeros, 1, pad, f.f) == pad;
            const uint64_t n = (uint64_t)all[i]->bytes();
            if (ok && n) ok = std::fwrite(all[i]->data, 1, n, f.f) == n;
            written = offsets[i] + n;
        }
        if (ok && cursor > written) ok = std::fwrite(zeros, 1, cursor - written, f.f) == cursor - written;
        if (ok) ok = std::fflush(f.f) == 0;
        if (!ok) {
            std::fclose(f.f);
            f.f = nullptr;
            std::remove(tmp.c_str());
            throw std::runtime_error("cannot write " + tmp);
        }
    }
    if (std::rename(tmp.c_str(), path.c_str()) != 0) {
        std::remove(tmp.c_str());
        throw std::runtime_error("cannot rename " + tmp + " to " + path + ": " + std::strerror(errno));
    }
}

Loaded load(const std::string &path, const std::vector<Tensor> &model, const Optimizer *opt,
            std::string (*settings_ok)(const std::map<std::string, float> &, const Optimizer &)) {
    File f;
    f.f = std::fopen(path.c_str(), "rb");
    if (!f.f) throw std::runtime_error("cannot open " + path + ": " + std::strerror(errno));
    struct stat st;
    if (fstat(fileno(f.f), &st) != 0 || !S_ISREG(st.st_mode))
        fail(UnsupportedStream, "A checkpoint is read from a regular (seekable) file; spool other inputs to a file first.");
    const uint64_t length = (uint64_t)st.st_size;
    if (length < kHeader)
        fail(BadHeader, "The file has " + std::to_string(length) + " bytes, less than the 64-byte header.");
    unsigned char h[kHeader];
    if (std::fread(h, 1, kHeader, f.f) != kHeader) fail(BadHeader, "The header cannot be read.");
    if (std::memcmp(h, "ONEMCKPT", 8) != 0) fail(BadHeader, "The magic is not ONEMCKPT.");
    const uint32_t version = get_u32(h + 8), flags = get_u32(h + 12);
    const uint64_t moff = get_u64(h + 16), mlen = get_u64(h + 24), doff = get_u64(h + 32), dlen = get_u64(h + 40),
                   flen = get_u64(h + 48), reserved = get_u64(h + 56);
    if (version != 1 || flags != 0 || reserved != 0)
        fail(BadHeader, "Unsupported version " + std::to_string(version) + ", flags " + std::to_string(flags) +
                            " or reserved field.");
    if (flen != length)
        fail(BadHeader, "The header says " + std::to_string(flen) + " bytes, the file has " + std::to_string(length) +
                            " (truncated or extended).");
    if (moff != kHeader || mlen > kMaxManifest || mlen > flen - kHeader || doff % 64 != 0 || doff < kHeader + mlen ||
        doff > flen || dlen != flen - doff)
        fail(BadHeader, "Manifest or data region offsets are inconsistent with the file length.");

    std::vector<char> mbytes((size_t)mlen);
    if (mlen && std::fread(mbytes.data(), 1, (size_t)mlen, f.f) != mlen) fail(BadHeader, "The manifest cannot be read.");
    if (!valid_utf8(reinterpret_cast<const unsigned char *>(mbytes.data()), mbytes.size()))
        fail(BadManifest, "The manifest is not valid UTF-8.");
    const JVal root = Reader(mbytes.data(), mbytes.size()).document();
    if (root.type != JVal::Obj || str(root, "format") != "onemodel-checkpoint" || integer(root, "version") != 1)
        fail(BadManifest, "The manifest is not a version 1 onemodel-checkpoint.");

    const int64_t data_len = (int64_t)dlen;
    const std::vector<Entry> model_entries = entries(arr(root, "model"));
    check_fit(model_entries, model, data_len);

    Loaded out;
    const JVal *o = root.get("optimizer");
    out.had_optimizer = o && o->type == JVal::Obj;
    std::vector<Entry> state_entries;
    if (out.had_optimizer && opt) {
        const std::string &kind = str(*o, "kind");
        if (kind != opt->kind)
            fail(Mismatch, "The checkpoint holds a '" + kind + "' optimizer, not '" + opt->kind + "'.");
        out.step = integer(*o, "step");
        if (out.step < 0) fail(BadManifest, "The optimizer step count is negative.");
        for (const JVal &hp : arr(*o, "hyper").a) {
            const int64_t bits = integer(hp, "bits");
            if (bits < 0 || bits > (int64_t)std::numeric_limits<uint32_t>::max())
                fail(BadManifest, "A hyper-parameter bit pattern is out of range.");
            const uint32_t b32 = (uint32_t)bits;
            float v;
            std::memcpy(&v, &b32, 4);
            out.hyper[str(hp, "name")] = v;
        }
        for (const auto &hp : opt->hyper)
            if (!out.hyper.count(hp.first)) fail(Mismatch, "The checkpoint lacks hyper-parameter '" + hp.first + "'.");
        state_entries = entries(arr(*o, "state"));
        check_fit_state(state_entries, *opt, data_len);
    } else if (opt) {
        fail(Mismatch, "The checkpoint holds no optimizer state.");
    }
    const JVal *ex = root.get("extra");
    if (ex && ex->type == JVal::Arr)
        for (const JVal &e : ex->a) {
            const std::string key = str(e, "key");
            out.extra[key] = integer(e, "value");
        }
    if (opt && out.had_optimizer && settings_ok) {
        const std::string why = settings_ok(out.hyper, *opt);
        if (!why.empty()) fail(Mismatch, why);
    }

    // Every check has passed: read the tensors.
    auto read = [&](const Entry &e) {
        std::vector<char> b((size_t)e.length);
        if (e.length) {
            if (fseeko(f.f, (off_t)(doff + (uint64_t)e.offset), SEEK_SET) != 0 ||
                std::fread(b.data(), 1, (size_t)e.length, f.f) != (size_t)e.length)
                throw std::runtime_error("reading tensor '" + e.name + "' failed (file changed while loading?)");
        }
        return b;
    };
    for (const Entry &e : model_entries) out.model.push_back(read(e));
    for (const Entry &e : state_entries) out.state.push_back(read(e));
    return out;
}

}  // namespace ckpt
}  // namespace omt
