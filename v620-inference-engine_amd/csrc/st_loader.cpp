// Read-only access to safetensors files (the checkpoint container the
// reference reads with src/core/safetensors.cpp): the file is mapped, its JSON
// header indexed by tensor name. Format: u64 little-endian header length,
// the header (a JSON object: name -> {"dtype", "shape", "data_offsets"
// relative to the end of the header}, plus an optional "__metadata__"), then
// the tensor bytes.
#include "st_loader.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cstring>

namespace qwq4 {

namespace {

// A small JSON reader for the header: objects, arrays, strings, integers and
// the literals; what the header does not use is rejected.
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    int64_t inum = 0;
    bool is_int = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
};

struct Parser {
    const char *p, *end;
    std::string err;

    bool fail(const char *m) {
        if (err.empty()) err = m;
        return false;
    }
    void ws() {
        while (p < end && std::isspace(static_cast<unsigned char>(*p))) ++p;
    }
    bool string(std::string &out) {
        if (p >= end || *p != '"') return fail("expected a string");
        ++p;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) return fail("bad escape");
                const char e = *p++;
                switch (e) {
                    case '"': c = '"'; break;
                    case '\\': c = '\\'; break;
                    case '/': c = '/'; break;
                    case 'b': c = '\b'; break;
                    case 'f': c = '\f'; break;
                    case 'n': c = '\n'; break;
                    case 'r': c = '\r'; break;
                    case 't': c = '\t'; break;
                    case 'u': {
                        if (end - p < 4) return fail("bad \\u escape");
                        unsigned v = 0;
                        for (int i = 0; i < 4; ++i) {
                            const char h = *p++;
                            v = v * 16 + unsigned(std::isdigit(static_cast<unsigned char>(h)) ? h - '0'
                                                                                               : (std::tolower(h) - 'a' + 10));
                        }
                        // UTF-8 of a BMP code point (names are ASCII in practice)
                        if (v < 0x80) out += char(v);
                        else if (v < 0x800) {
                            out += char(0xc0 | (v >> 6));
                            out += char(0x80 | (v & 0x3f));
                        } else {
                            out += char(0xe0 | (v >> 12));
                            out += char(0x80 | ((v >> 6) & 0x3f));
                            out += char(0x80 | (v & 0x3f));
                        }
                        continue;
                    }
                    default: return fail("bad escape");
                }
            }
            out += c;
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    bool value(Json &v, int depth) {
        if (depth > 16) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        const char c = *p;
        if (c == '{') {
            v.kind = Json::OBJ;
            ++p;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return true;
            }
            while (true) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                ++p;
                Json e;
                if (!value(e, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(e));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = Json::ARR;
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            while (true) {
                Json e;
                if (!value(e, depth + 1)) return false;
                v.arr.push_back(std::move(e));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Json::STR;
            return string(v.str);
        }
        auto lit = [&](const char *w, Json::Kind k, bool b) {
            const size_t n = std::strlen(w);
            if (size_t(end - p) < n || std::memcmp(p, w, n) != 0) return fail("bad literal");
            p += n;
            v.kind = k;
            v.num = b;
            return true;
        };
        if (c == 't') return lit("true", Json::BOOL, true);
        if (c == 'f') return lit("false", Json::BOOL, false);
        if (c == 'n') return lit("null", Json::NUL, false);
        // number: integers exactly, anything else as a double
        const char *s = p;
        if (p < end && (*p == '-' || *p == '+')) ++p;
        bool frac = false;
        while (p < end && (std::isdigit(static_cast<unsigned char>(*p)) || *p == '.' || *p == 'e' || *p == 'E' ||
                           *p == '-' || *p == '+')) {
            frac |= (*p == '.' || *p == 'e' || *p == 'E');
            ++p;
        }
        if (p == s) return fail("unexpected character");
        const std::string t(s, p);
        v.kind = Json::NUM;
        v.is_int = !frac;
        if (v.is_int) {
            char *e = nullptr;
            v.inum = std::strtoll(t.c_str(), &e, 10);
            v.num = double(v.inum);
        } else {
            v.num = std::strtod(t.c_str(), nullptr);
        }
        return true;
    }
};

size_t dtype_bytes(const std::string &d) {
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "F32" || d == "I32" || d == "U32") return 4;
    if (d == "F16" || d == "BF16" || d == "I16" || d == "U16") return 2;
    if (d == "I8" || d == "U8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    return 0;
}

}  // namespace

bool StFile::open(const std::string &path, std::string &err) {
    path_ = path;
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        err = "cannot open " + path;
        return false;
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 8) {
        ::close(fd);
        err = path + ": not a safetensors file (too short)";
        return false;
    }
    size_ = size_t(sb.st_size);
    void *m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) {
        err = "cannot map " + path;
        return false;
    }
    data_ = static_cast<const uint8_t *>(m);
    uint64_t hl = 0;
    for (int i = 7; i >= 0; --i) hl = (hl << 8) | data_[i];
    if (hl > size_ - 8) {
        err = path + ": header length beyond the file";
        return false;
    }
    Parser ps{reinterpret_cast<const char *>(data_ + 8), reinterpret_cast<const char *>(data_ + 8 + hl), {}};
    Json root;
    if (!ps.value(root, 0) || root.kind != Json::OBJ) {
        err = path + ": bad header: " + (ps.err.empty() ? std::string("not an object") : ps.err);
        return false;
    }
    const size_t base = 8 + hl;
    for (auto &kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const Json &t = kv.second;
        if (t.kind != Json::OBJ) {
            err = path + ": entry " + kv.first + " is not an object";
            return false;
        }
        StTensor ti;
        ti.name = kv.first;
        bool have_d = false, have_s = false, have_o = false;
        size_t b = 0, e = 0;
        for (auto &f : t.obj) {
            if (f.first == "dtype" && f.second.kind == Json::STR) {
                ti.dtype = f.second.str;
                have_d = true;
            } else if (f.first == "shape" && f.second.kind == Json::ARR) {
                for (auto &d : f.second.arr) {
                    if (d.kind != Json::NUM || !d.is_int || d.inum < 0) {
                        err = path + ": " + kv.first + ": bad shape";
                        return false;
                    }
                    ti.shape.push_back(d.inum);
                }
                have_s = true;
            } else if (f.first == "data_offsets" && f.second.kind == Json::ARR && f.second.arr.size() == 2) {
                const Json &x = f.second.arr[0], &y = f.second.arr[1];
                if (x.kind != Json::NUM || y.kind != Json::NUM || !x.is_int || !y.is_int || x.inum < 0 ||
                    y.inum < x.inum) {
                    err = path + ": " + kv.first + ": bad data_offsets";
                    return false;
                }
                b = size_t(x.inum);
                e = size_t(y.inum);
                have_o = true;
            }
        }
        if (!have_d || !have_s || !have_o) {
            err = path + ": " + kv.first + ": missing dtype, shape or data_offsets";
            return false;
        }
        const size_t es = dtype_bytes(ti.dtype);
        int64_t n = 1;
        for (int64_t d : ti.shape) n *= d;
        if (es == 0 || size_t(n) * es != e - b || base + e > size_) {
            err = path + ": " + kv.first + ": size does not match dtype and shape, or lies beyond the file";
            return false;
        }
        ti.data = data_ + base + b;
        ti.nbytes = e - b;
        index_.emplace(ti.name, std::move(ti));
    }
    return true;
}

StFile::~StFile() {
    if (data_) munmap(const_cast<uint8_t *>(data_), size_);
}

const StTensor *StFile::find(const std::string &name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &it->second;
}

}  // namespace qwq4
