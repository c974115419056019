// Kokoro decoder weights from a safetensors file: the reference's
// DecoderBackbone / Generator / HarmonicSource load_from over
// brotensor::safetensors (kokoro_modules.cpp:99-122 `upload`, 1021-1063,
// 1147-1195, 1237-1347, 1556-1572) for the whole-decoder model, whose
// parameter names are the upstream state-dict keys ("decoder.module....").
//
// A safetensors file is an 8-byte little-endian header length, a JSON object
// {name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__":
// {...}} and the raw tensor bytes (offsets relative to the end of the
// header). As in the reference, tensors must be F32 and hold exactly the
// parameter's element count. A weight stored in weight-norm form (the
// upstream checkpoint's weight_g / weight_v pairs, which the reference's
// scripts/convert-kokoro.py:71-110 fuses offline) is fused on load:
// weight[r, :] = g[r] * v[r, :] / max(||v[r, :]||, 1e-12), the norm over
// every axis but the first.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "kdec.h"
#include "kdec_internal.hpp"
#include "kdec_model.h"

namespace kdec {
namespace {

// ─── a minimal JSON reader for safetensors headers ───────────────────────
struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const std::string& k) const {
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct Parser {
    const char* p;
    const char* e;
    std::string err;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool fail(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    bool string(std::string& out) {
        if (p >= e || *p != '"') return fail("expected a string");
        ++p;
        while (p < e && *p != '"') {
            if (*p == '\\') {
                if (++p >= e) return fail("bad escape");
                switch (*p) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (e - p < 5) return fail("bad \\u escape");
                        unsigned cp = 0;
                        for (int i = 1; i <= 4; ++i) {
                            const char c = p[i];
                            cp = cp * 16 + (c >= '0' && c <= '9' ? c - '0' : (c | 32) >= 'a' && (c | 32) <= 'f' ? (c | 32) - 'a' + 10 : 99);
                            if (cp > 0xffff) return fail("bad \\u escape");
                        }
                        p += 4;
                        if (cp < 0x80) {
                            out += static_cast<char>(cp);
                        } else if (cp < 0x800) {
                            out += static_cast<char>(0xc0 | (cp >> 6));
                            out += static_cast<char>(0x80 | (cp & 0x3f));
                        } else {
                            out += static_cast<char>(0xe0 | (cp >> 12));
                            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
                            out += static_cast<char>(0x80 | (cp & 0x3f));
                        }
                        break;
                    }
                    default: return fail("bad escape");
                }
                ++p;
            } else {
                out += *p++;
            }
        }
        if (p >= e) return fail("unterminated string");
        ++p;
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 16) return fail("nesting too deep");
        ws();
        if (p >= e) return fail("unexpected end");
        if (*p == '{') {
            v.kind = Json::OBJ;
            ++p;
            ws();
            if (p < e && *p == '}') return ++p, true;
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p >= e || *p != ':') return fail("expected ':'");
                ++p;
                v.obj.emplace_back(std::move(k), Json());
                if (!value(v.obj.back().second, depth + 1)) return false;
                ws();
                if (p < e && *p == ',') { ++p; continue; }
                if (p < e && *p == '}') return ++p, true;
                return fail("expected ',' or '}'");
            }
        }
        if (*p == '[') {
            v.kind = Json::ARR;
            ++p;
            ws();
            if (p < e && *p == ']') return ++p, true;
            for (;;) {
                v.arr.emplace_back();
                if (!value(v.arr.back(), depth + 1)) return false;
                ws();
                if (p < e && *p == ',') { ++p; continue; }
                if (p < e && *p == ']') return ++p, true;
                return fail("expected ',' or ']'");
            }
        }
        if (*p == '"') {
            v.kind = Json::STR;
            return string(v.str);
        }
        if (e - p >= 4 && !std::strncmp(p, "null", 4)) return p += 4, true;
        if (e - p >= 4 && !std::strncmp(p, "true", 4)) { v.kind = Json::BOOL; v.num = 1; return p += 4, true; }
        if (e - p >= 5 && !std::strncmp(p, "false", 5)) { v.kind = Json::BOOL; return p += 5, true; }
        const char* s = p;
        while (p < e && (std::strchr("+-0123456789.eE", *p) != nullptr)) ++p;
        if (p == s) return fail("unexpected character");
        v.kind = Json::NUM;
        v.num = std::strtod(std::string(s, p).c_str(), nullptr);
        return true;
    }
};

struct Entry {
    std::string dtype;
    std::vector<long> shape;
    std::uint64_t begin = 0, end = 0;
    long numel() const {
        long n = 1;
        for (long d : shape) n *= d;
        return n;
    }
};

struct StFile {
    std::FILE* f = nullptr;
    std::uint64_t data0 = 0, size = 0;
    std::map<std::string, Entry> t;
    ~StFile() {
        if (f) std::fclose(f);
    }
};

// Opens and indexes `path`; returns "" or the reason it is not a safetensors file.
std::string open_st(const char* path, StFile& s) {
    s.f = std::fopen(path, "rb");
    if (!s.f) return std::string("cannot open '") + path + "'";
    std::fseek(s.f, 0, SEEK_END);
    s.size = static_cast<std::uint64_t>(std::ftell(s.f));
    std::fseek(s.f, 0, SEEK_SET);
    unsigned char nb[8];
    if (s.size < 8 || std::fread(nb, 1, 8, s.f) != 8) return "truncated header length";
    std::uint64_t n = 0;
    for (int i = 7; i >= 0; --i) n = (n << 8) | nb[i];
    if (n > s.size - 8 || n > (100u << 20)) return "header length past the end of the file";
    std::string js(n, '\0');
    if (std::fread(&js[0], 1, n, s.f) != n) return "truncated header";
    s.data0 = 8 + n;
    Parser ps{js.data(), js.data() + js.size(), {}};
    Json root;
    if (!ps.value(root, 0)) return "bad header JSON: " + ps.err;
    if (root.kind != Json::OBJ) return "header is not a JSON object";
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& o = kv.second;
        const Json* dt = o.get("dtype");
        const Json* sh = o.get("shape");
        const Json* of = o.get("data_offsets");
        if (o.kind != Json::OBJ || !dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !of ||
            of->kind != Json::ARR || of->arr.size() != 2)
            return "bad entry for '" + kv.first + "'";
        Entry en;
        en.dtype = dt->str;
        for (const auto& d : sh->arr) {
            if (d.kind != Json::NUM || d.num < 0) return "bad shape for '" + kv.first + "'";
            en.shape.push_back(static_cast<long>(d.num));
        }
        if (of->arr[0].kind != Json::NUM || of->arr[1].kind != Json::NUM) return "bad offsets for '" + kv.first + "'";
        en.begin = static_cast<std::uint64_t>(of->arr[0].num);
        en.end = static_cast<std::uint64_t>(of->arr[1].num);
        if (en.end < en.begin || s.data0 + en.end > s.size) return "offsets of '" + kv.first + "' past the end";
        s.t[kv.first] = std::move(en);
    }
    return "";
}

bool read_f32(StFile& s, const Entry& en, std::vector<float>& out) {
    out.resize(static_cast<std::size_t>(en.numel()));
    if (en.end - en.begin != out.size() * sizeof(float)) return false;
    if (std::fseek(s.f, static_cast<long>(s.data0 + en.begin), SEEK_SET) != 0) return false;
    return std::fread(out.data(), sizeof(float), out.size(), s.f) == out.size();
}

}  // namespace
}  // namespace kdec

using namespace kdec;

extern "C" {

int kdec_safetensors_count(const char* path) {
    if (!path) return KDEC_EINVAL;
    StFile s;
    if (!open_st(path, s).empty()) return KDEC_EINVAL;
    return static_cast<int>(s.t.size());
}

int kdec_model_load_safetensors(kdec_model* m, const char* path) {
    if (!m || !path) return KDEC_EINVAL;
    kdec_ctx* ctx = kdec_model_context(m);
    const std::string where = "kdec_model_load_safetensors: ";
    StFile s;
    const std::string why = open_st(path, s);
    if (!why.empty()) return fail(ctx, KDEC_EINVAL, where + why);
    std::vector<float> h, g, v;
    const int n = kdec_model_param_count(m);
    for (int i = 0; i < n; ++i) {
        const std::string name = kdec_model_param_name(m, i);
        int rows = 0, cols = 0;
        kdec_model_param_shape(m, name.c_str(), &rows, &cols);
        const long want = static_cast<long>(rows) * cols;
        auto it = s.t.find(name);
        if (it == s.t.end()) {
            // weight-norm form: name_g (one per row), name_v (the direction)
            const std::string stem = name.size() > 7 && name.compare(name.size() - 7, 7, ".weight") == 0
                                         ? name.substr(0, name.size() - 7) : std::string();
            auto ig = stem.empty() ? s.t.end() : s.t.find(stem + ".weight_g");
            auto iv = stem.empty() ? s.t.end() : s.t.find(stem + ".weight_v");
            if (ig == s.t.end() || iv == s.t.end())
                return fail(ctx, KDEC_EINVAL, where + "missing safetensors key '" + name + "'");
            for (auto* e : {&ig->second, &iv->second})
                if (e->dtype != "F32")
                    return fail(ctx, KDEC_EINVAL, where + "tensor '" + stem + "' weight-norm parts are not F32 (got " +
                                                      e->dtype + ")");
            if (iv->second.numel() != want || ig->second.numel() != rows)
                return fail(ctx, KDEC_EINVAL, where + "tensor '" + stem + ".weight_v' has " +
                                                  std::to_string(iv->second.numel()) + " elements; expected " +
                                                  std::to_string(want));
            if (!read_f32(s, ig->second, g) || !read_f32(s, iv->second, v))
                return fail(ctx, KDEC_EINVAL, where + "cannot read '" + stem + "'");
            h.resize(static_cast<std::size_t>(want));
            for (int r = 0; r < rows; ++r) {
                double ss = 0.0;
                for (int c = 0; c < cols; ++c) ss += static_cast<double>(v[r * cols + c]) * v[r * cols + c];
                const double k = g[r] / std::max(std::sqrt(ss), 1e-12);
                for (int c = 0; c < cols; ++c) h[r * cols + c] = static_cast<float>(k * v[r * cols + c]);
            }
        } else {
            const Entry& en = it->second;
            if (en.dtype != "F32")
                return fail(ctx, KDEC_EINVAL, where + "tensor '" + name + "' is not F32 (got dtype " + en.dtype + ")");
            if (en.numel() != want)
                return fail(ctx, KDEC_EINVAL, where + "tensor '" + name + "' has " + std::to_string(en.numel()) +
                                                  " elements; expected " + std::to_string(want));
            if (!read_f32(s, en, h)) return fail(ctx, KDEC_EINVAL, where + "cannot read '" + name + "'");
        }
        if (int rc = kdec_model_set_param(m, name.c_str(), h.data(), want)) return rc;
    }
    return KDEC_OK;
}

}  // extern "C"
