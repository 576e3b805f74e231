// The model files of tenzo_load_model (load_model_from_files,
// src/runtime/TenzoEngine.cpp:1887-2078): model.mlir names the byte offset of
// every tensor in weights.bin and the scale of every ternary projection.
//
// Two statement pairs carry them, each a constant whose next non-blank line
// consumes it (only whitespace, with at least one line break, in between):
//   %c = arith.constant <digits> : index
//   %v = memref.view %buf[%c][] : memref<?xi8> to memref<...>     -> offset
//   %s = arith.constant <[0-9.e+-]+> : f32
//   %r = "tenzo.bitlinear_elut"(<a>, <b>, %s) ...                 -> scale
// in order of appearance (TenzoEngine.cpp:1943-1959). This is a scanner over
// the text, not a regular-expression engine: at each '%' it tries the
// constant, then the consumer, and after a match resumes past the consumer;
// a failed try resumes at the next '%'.
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "common.h"
#include "model_file.h"

namespace tz {
namespace {

bool is_word(char c) {
    return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') || c == '_';
}
bool is_space(char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\f' || c == '\v'; }

struct Cursor {
    const char* p;
    const char* end;
    bool done() const { return p >= end; }
    void skip_space() {
        while (p < end && is_space(*p)) ++p;
    }
    bool skip_space1() {  // one or more
        const char* q = p;
        skip_space();
        return p > q;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end - p) < n || std::memcmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    // '%' followed by one or more word characters (maximal)
    bool name(std::string* out) {
        if (p >= end || *p != '%') return false;
        const char* q = p + 1;
        while (q < end && is_word(*q)) ++q;
        if (q == p + 1) return false;
        if (out) out->assign(p, q);
        p = q;
        return true;
    }
    bool run(bool (*ok)(char), std::string* out) {  // one or more characters in a class
        const char* q = p;
        while (q < end && ok(*q)) ++q;
        if (q == p) return false;
        if (out) out->assign(p, q);
        p = q;
        return true;
    }
    // whitespace that holds at least one line break
    bool line_break() {
        const char* q = p;
        bool nl = false;
        while (q < end && is_space(*q)) nl |= *q++ == '\n';
        if (!nl) return false;
        p = q;
        return true;
    }
};

bool is_digit(char c) { return c >= '0' && c <= '9'; }
bool is_num(char c) { return is_digit(c) || c == '.' || c == 'e' || c == '+' || c == '-'; }

// "%c = arith.constant <value> : <type>" with value in the class; the name
// and the value text are returned.
bool constant(Cursor& c, bool (*cls)(char), const char* type, std::string* nm, std::string* val) {
    if (!c.name(nm)) return false;
    c.skip_space();
    if (!c.lit("=")) return false;
    c.skip_space();
    if (!c.lit("arith.constant") || !c.skip_space1()) return false;
    if (!c.run(cls, val)) return false;
    c.skip_space();
    if (!c.lit(":")) return false;
    c.skip_space();
    return c.lit(type);
}

// "%v = memref.view %buf[%c][] : memref<?xi8> to memref<...>"
bool view_of(Cursor& c, const std::string& nm) {
    if (!c.name(nullptr)) return false;
    c.skip_space();
    if (!c.lit("=")) return false;
    c.skip_space();
    if (!c.lit("memref.view") || !c.skip_space1()) return false;
    if (!c.name(nullptr) || !c.lit("[") || !c.lit(nm.c_str()) || !c.lit("][]")) return false;
    c.skip_space();
    if (!c.lit(":")) return false;
    c.skip_space();
    if (!c.lit("memref<?xi8>") || !c.skip_space1() || !c.lit("to") || !c.skip_space1()) return false;
    if (!c.lit("memref<")) return false;
    const char* q = c.p;
    while (c.p < c.end && *c.p != '>') ++c.p;
    if (c.p == q || c.p >= c.end) return false;
    ++c.p;
    return true;
}

// '%r = "tenzo.bitlinear_elut"(<a>, <b>, %s)' with a, b free of commas
bool elut_with(Cursor& c, const std::string& nm) {
    if (!c.name(nullptr)) return false;
    c.skip_space();
    if (!c.lit("=")) return false;
    c.skip_space();
    if (!c.lit("\"tenzo.bitlinear_elut\"(")) return false;
    for (int arg = 0; arg < 2; ++arg) {
        const char* q = c.p;
        while (c.p < c.end && *c.p != ',') ++c.p;
        if (c.p == q || c.p >= c.end) return false;
        ++c.p;  // the comma
        c.skip_space();
    }
    return c.lit(nm.c_str()) && c.lit(")");
}

template <typename Pair>
void scan(const char* text, size_t len, Pair try_at) {
    Cursor c{text, text + len};
    while (!c.done()) {
        const char* pct = static_cast<const char*>(std::memchr(c.p, '%', c.end - c.p));
        if (!pct) break;
        Cursor t{pct, c.end};
        if (try_at(t))
            c.p = t.p;
        else
            c.p = pct + 1;
    }
}

}  // namespace

void parse_model_mlir(const char* text, size_t len, ModelFileIndex* out) {
    out->views.clear();
    out->scales.clear();
    scan(text, len, [&](Cursor& t) {
        std::string nm, val;
        if (!constant(t, is_digit, "index", &nm, &val) || !t.line_break() || !view_of(t, nm))
            return false;
        out->views.push_back(std::strtoull(val.c_str(), nullptr, 10));
        return true;
    });
    scan(text, len, [&](Cursor& t) {
        std::string nm, val;
        if (!constant(t, is_num, "f32", &nm, &val) || !t.line_break() || !elut_with(t, nm))
            return false;
        out->scales.push_back(std::strtof(val.c_str(), nullptr));
        return true;
    });
}

}  // namespace tz

extern "C" {

TENZO_HIP_API int tenzo_hip_parse_model_mlir(const char* text, uint64_t* views, int max_views,
                                             float* scales, int max_scales, int* n_views,
                                             int* n_scales) {
    TZ_CHECK(text && n_views && n_scales, "parse_model_mlir: null pointer");
    tz::ModelFileIndex ix;
    tz::parse_model_mlir(text, std::strlen(text), &ix);
    *n_views = (int)ix.views.size();
    *n_scales = (int)ix.scales.size();
    for (int i = 0; i < *n_views && i < max_views && views; ++i) views[i] = ix.views[i];
    for (int i = 0; i < *n_scales && i < max_scales && scales; ++i) scales[i] = ix.scales[i];
    return TENZO_SUCCESS;
}

}  // extern "C"
