// The model files and the static plan (include/fhc_model.h): a small JSON reader, the loader with the reference's
// validation, and the graph walk into plan steps. Host code only.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstring>
#include <set>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "common.h"
#include "fhc_conv.h"
#include "fhc_model.h"

namespace fhc {
namespace {

// ---- JSON ------------------------------------------------------------------------------------------------------
struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    bool integral = false;  // written without fraction or exponent
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const std::string& key) const {
        if (kind != Obj) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    const Json& operator[](const std::string& key) const {
        static const Json null;
        const Json* j = get(key);
        return j ? *j : null;
    }
    bool is_str() const { return kind == Str; }
    bool is_u64() const { return kind == Num && integral && num >= 0 && num < 9.007199254740992e15; }
    uint64_t u64() const { return (uint64_t)num; }
};

class JsonParser {
  public:
    JsonParser(const char* p, size_t n) : p_(p), e_(p + n) {}
    Json parse() {
        Json v = value(0);
        ws();
        if (p_ != e_) err("trailing characters");
        return v;
    }

  private:
    const char *p_, *e_;
    [[noreturn]] void err(const char* what) { throw std::runtime_error(std::string("JSON: ") + what); }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) p_++;
    }
    bool lit(const char* s) {
        const size_t n = strlen(s);
        if ((size_t)(e_ - p_) >= n && memcmp(p_, s, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    static void utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (e_ - p_ < 4) err("short \\u escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else err("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        if (p_ >= e_ || *p_ != '"') err("expected a string");
        p_++;
        std::string s;
        while (true) {
            if (p_ >= e_) err("unterminated string");
            const char c = *p_++;
            if (c == '"') break;
            if ((unsigned char)c < 0x20) err("control character in a string");
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= e_) err("unterminated escape");
            const char x = *p_++;
            switch (x) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && lit("\\u")) {
                        const uint32_t lo = hex4();
                        if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(s, cp);
                    break;
                }
                default: err("bad escape");
            }
        }
        return s;
    }
    Json value(int depth) {
        if (depth > 64) err("nesting too deep");
        ws();
        if (p_ >= e_) err("unexpected end");
        Json v;
        const char c = *p_;
        if (c == '{') {
            p_++;
            v.kind = Json::Obj;
            ws();
            if (p_ < e_ && *p_ == '}') {
                p_++;
                return v;
            }
            while (true) {
                ws();
                std::string k = string();
                ws();
                if (p_ >= e_ || *p_ != ':') err("expected ':'");
                p_++;
                v.obj.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (p_ < e_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < e_ && *p_ == '}') {
                    p_++;
                    return v;
                }
                err("expected ',' or '}'");
            }
        }
        if (c == '[') {
            p_++;
            v.kind = Json::Arr;
            ws();
            if (p_ < e_ && *p_ == ']') {
                p_++;
                return v;
            }
            while (true) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (p_ < e_ && *p_ == ',') {
                    p_++;
                    continue;
                }
                if (p_ < e_ && *p_ == ']') {
                    p_++;
                    return v;
                }
                err("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Json::Str;
            v.str = string();
            return v;
        }
        if (lit("true")) {
            v.kind = Json::Bool;
            v.b = true;
            return v;
        }
        if (lit("false")) {
            v.kind = Json::Bool;
            return v;
        }
        if (lit("null")) return v;
        const char* s = p_;
        if (p_ < e_ && *p_ == '-') p_++;
        bool integral = true;
        while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                           *p_ == '-')) {
            if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') integral = false;
            p_++;
        }
        if (p_ == s) err("unexpected character");
        const std::string t(s, p_);
        char* end = nullptr;
        v.kind = Json::Num;
        v.num = strtod(t.c_str(), &end);
        if (!end || *end) err("bad number");
        v.integral = integral;
        return v;
    }
};

Json parse_json(const std::string& text) { return JsonParser(text.data(), text.size()).parse(); }

std::vector<std::string> names(const Json& op, const char* key) {
    std::vector<std::string> out;
    for (const Json& v : op[key].arr)
        if (v.is_str()) out.push_back(v.str);
    return out;
}

std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot read " + path);
    std::ostringstream s;
    s << f.rdbuf();
    return s.str();
}

std::string jstr(const std::string& s) {
    std::string o = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') o += '\\';
        o += c;
    }
    return o + "\"";
}

std::string jnum(double v) {
    char b[40];
    snprintf(b, sizeof b, "%.9g", v);
    return b;
}

}  // namespace
}  // namespace fhc

using namespace fhc;

struct fhc_model {
    Json ops;       // graph.json "ops"
    Json manifest;  // flyhighfg.json
    std::vector<uint8_t> blob;
    struct TensorInfo {
        std::vector<uint32_t> dims;
        uint64_t offset, count;
    };
    std::map<std::string, TensorInfo> tensors;
    uint32_t format_version = 1;
    uint64_t params = 0;
};

namespace fhc {
namespace {

// graph::validate (model/graph.rs:17-47): every op named, operand lists of strings, weights present, repeat bodies
// checked too, film_mlp's fixed weights present
void validate_ops(const Json& ops, const fhc_model& m) {
    if (ops.kind != Json::Arr) throw std::runtime_error("graph.json: ops is not a list");
    size_t i = 0;
    for (const Json& op : ops.arr) {
        const Json& nm = op["op"];
        if (!nm.is_str()) throw std::runtime_error("graph.json: op " + std::to_string(i) + " has no name");
        for (const char* key : {"in", "out", "w"}) {
            const Json* l = op.get(key);
            if (!l) continue;
            if (l->kind != Json::Arr) throw std::runtime_error("graph.json: " + nm.str + "." + key + " is not a list");
            for (const Json& v : l->arr)
                if (!v.is_str()) throw std::runtime_error("graph.json: " + nm.str + "." + key + " has a non-string entry");
        }
        for (const std::string& w : names(op, "w"))
            if (!m.tensors.count(w))
                throw std::runtime_error("graph.json: " + nm.str + " reads tensor " + w + ", which the manifest lacks");
        if (nm.str == "repeat") {
            if (op["body"].kind != Json::Arr) throw std::runtime_error("graph.json: repeat without a body");
            validate_ops(op["body"], m);
        }
        if (nm.str == "film_mlp")
            for (const char* w : {"film.film.0.weight", "film.film.0.bias", "film.film.2.weight", "film.film.2.bias"})
                if (!m.tensors.count(w))
                    throw std::runtime_error(std::string("graph.json: film_mlp needs tensor ") + w +
                                             ", which the manifest lacks");
        i++;
    }
}

// Model::from_shared (model/mod.rs:57-96) with check_tensor (:101-119)
void finish_load(fhc_model& m, const std::string& graph_text, const std::string& manifest_text) {
    const Json graph = parse_json(graph_text);
    m.manifest = parse_json(manifest_text);
    const Json* ops = graph.get("ops");
    if (!ops || ops->kind != Json::Arr || ops->arr.empty()) throw std::runtime_error("graph.json: no ops");
    m.ops = *ops;
    const Json& meta = m.manifest["meta"];
    const Json& fv = meta["format_version"];
    m.format_version = fv.is_u64() ? (uint32_t)fv.u64() : 1;
    if (m.format_version != 1)
        throw std::runtime_error("model format_version " + std::to_string(m.format_version) +
                                 " not supported, this engine reads 1..=1");
    const Json& ts = m.manifest["tensors"];
    if (ts.kind != Json::Obj) throw std::runtime_error("manifest has no tensors");
    for (const auto& kv : ts.obj) {
        const std::string& name = kv.first;
        const Json& off = kv.second["offset"];
        if (!off.is_u64()) throw std::runtime_error("tensor " + name + ": offset is not an unsigned integer");
        const Json& shape = kv.second["shape"];
        if (shape.kind != Json::Arr) throw std::runtime_error("tensor " + name + ": shape is not an array");
        fhc_model::TensorInfo t{{}, off.u64(), 1};
        for (const Json& d : shape.arr) {
            if (!d.is_u64()) throw std::runtime_error("tensor " + name + ": shape has a non-integer dimension");
            if (d.u64() < 1) throw std::runtime_error("tensor " + name + ": shape has a zero dimension");
            if (d.u64() > 0xFFFFFFFFull || t.count > (1ull << 40) / d.u64())
                throw std::runtime_error("tensor " + name + ": shape overflows");
            t.dims.push_back((uint32_t)d.u64());
            t.count *= d.u64();
        }
        if (t.offset > (1ull << 50) || (t.offset + t.count) * 2 > m.blob.size())
            throw std::runtime_error("tensor " + name + " runs past the end of the weight blob");
        m.params += t.count;
        m.tensors[name] = t;
    }
    validate_ops(m.ops, m);
}

// ---- the static plan (net/session.rs:26-66, net/build.rs:149-484, :532-736) ----------------------------------
struct Buf {
    uint32_t c, h, w;
    bool zeros;
    std::string name;
};
struct View {
    int buf = -1;
    uint32_t c = 0, h = 0, w = 0, c0 = 0;
    float scale = 1.0f;
    bool plain() const { return c0 == 0 && scale == 1.0f; }  // Tensor::is_plain (ops/tensor.rs:19-21)
    View sub(uint32_t a, uint32_t b) const {                 // Tensor::view (:22-24)
        View v = *this;
        v.c = b - a;
        v.c0 = c0 + a;
        return v;
    }
    View scaled(float f) const {  // Tensor::scaled (:25-27)
        View v = *this;
        v.scale = scale * f;
        return v;
    }
};

// one conv of the plan, as the reference's discovery build records it (ConvShape, ops/conv/autotune.rs:153-164)
struct ConvUse {
    std::string w, b, s;                  // weight, bias and slope tensors (s empty without an activation)
    uint32_t cin, cout, h, wd, stride;    // h, wd: the input size
    bool act, res;
};

struct Planner {
    const fhc_model& m;
    uint32_t k, hs, ws;  // the repeat count and the network size (interpolate's "HW")
    std::vector<Buf> bufs;
    std::vector<ConvUse> convs;
    std::map<std::string, View> env;
    std::map<std::string, size_t> uses;
    std::vector<std::string> steps;
    std::string stage = "pair";

    View alloc(uint32_t c, uint32_t h, uint32_t w, const std::string& name, bool zeros = false) {
        bufs.push_back(Buf{c, h, w, zeros, name});
        View v;
        v.buf = (int)bufs.size() - 1;
        v.c = c, v.h = h, v.w = w;
        return v;
    }
    static std::string vjson(const View& v) {
        return "{\"buf\":" + std::to_string(v.buf) + ",\"c0\":" + std::to_string(v.c0) + ",\"c\":" +
               std::to_string(v.c) + ",\"scale\":" + jnum(v.scale) + "}";
    }
    void step(const std::string& op, const std::vector<View>& ins, const View& out, const std::string& extra = "") {
        std::string s = "{\"stage\":\"" + stage + "\",\"op\":\"" + op + "\",\"in\":[";
        for (size_t i = 0; i < ins.size(); i++) s += (i ? "," : "") + vjson(ins[i]);
        s += "],\"out\":" + vjson(out);
        if (!extra.empty()) s += "," + extra;
        steps.push_back(s + "}");
    }
    const View& get(const std::string& n) {
        auto it = env.find(n);
        if (it == env.end()) throw std::runtime_error("graph.json: " + n + " is read before it is written");
        return it->second;
    }
    // a view a kernel needs plain is copied into a plain tensor first (Gpu::mat, ops/elementwise.rs:85-93)
    View mat(const View& x) {
        if (x.plain()) return x;
        View y = alloc(x.c, x.h, x.w, "");
        step("mat", {x}, y);
        return y;
    }
    void count_uses(const Json& ops) {  // model/graph.rs:49-60: the body of a repeat counted once
        for (const Json& op : ops.arr) {
            for (const std::string& n : names(op, "in")) uses[n]++;
            if (op["op"].str == "repeat") count_uses(op["body"]);
        }
    }
    size_t used(const std::string& n) const {
        auto it = uses.find(n);
        return it == uses.end() ? 0 : it->second;
    }
    const fhc_model::TensorInfo& tensor(const std::string& n) const {
        auto it = m.tensors.find(n);
        if (it == m.tensors.end()) throw std::runtime_error("the manifest has no tensor " + n);
        return it->second;
    }
    View conv(const View& xin, const std::string& w, const std::string& b, const std::string& s, uint32_t stride,
              uint32_t act, const View* res, const std::string& out_name) {
        const auto& t = tensor(w);
        if (t.dims.size() != 4 || t.dims[2] != 3 || t.dims[3] != 3)
            throw std::runtime_error("conv weight " + w + " is not [cout][cin][3][3]");
        const uint32_t cout = t.dims[0], cin = t.dims[1];
        if (xin.c != cin) throw std::runtime_error("conv " + w + ": input has " + std::to_string(xin.c) + " channels");
        const View x = mat(xin);
        const uint32_t ho = (x.h + 2 - 3) / stride + 1, wo = (x.w + 2 - 3) / stride + 1;
        View y = alloc(cout, ho, wo, out_name);
        std::vector<View> ins{x};
        std::string extra = "\"weight\":" + jstr(w) + ",\"bias\":" + jstr(b) + ",\"slope\":" +
                            (s.empty() ? std::string("null") : jstr(s)) + ",\"cin\":" + std::to_string(cin) +
                            ",\"cout\":" + std::to_string(cout) + ",\"stride\":" + std::to_string(stride) +
                            ",\"act\":" + std::to_string(act) + ",\"residual\":" + (res ? vjson(*res) : "null") +
                            ",\"name\":" + jstr(out_name);
        step("conv", ins, y, extra);
        convs.push_back(ConvUse{w, b, s, cin, cout, x.h, x.w, stride, act != 0, res != nullptr});
        return y;
    }

    void walk(const Json& ops, size_t from, size_t to) {
        size_t i = from;
        while (i < to) {
            const Json& op = ops.arr[i];
            i++;
            const std::string name = op["op"].str;
            const auto ins = names(op, "in"), outs = names(op, "out");
            if (name != "repeat" && name != "render_pix" && !outs.empty()) {
                bool dead = true;  // nobody reads it (build.rs:170-178)
                for (const std::string& o : outs) dead = dead && used(o) == 0;
                if (dead) continue;
            }
            auto in = [&](size_t j) -> const View& {
                if (j >= ins.size()) throw std::runtime_error("graph.json: " + name + " lacks input " + std::to_string(j));
                return get(ins[j]);
            };
            if (name == "repeat") {
                const Json& t = op["times"];
                const uint32_t times = t.is_u64() ? (uint32_t)t.u64() : k;
                for (uint32_t r = 0; r < times; r++) walk(op["body"], 0, op["body"].arr.size());
                continue;
            }
            if (outs.empty()) throw std::runtime_error("graph.json: " + name + " has no output");
            View res;
            if (name == "interpolate") {
                const View x = in(0);
                uint32_t oh, ow;
                if (op["size"].is_str() && op["size"].str == "HW") {
                    oh = hs, ow = ws;
                } else {
                    const float s = (float)op["scale"].num;
                    oh = (uint32_t)std::floor((float)x.h * s);
                    ow = (uint32_t)std::floor((float)x.w * s);
                }
                const bool aa = op["antialias"].kind == Json::Bool && op["antialias"].b;
                res = alloc(x.c, oh, ow, outs[0]);
                step("interp", {x}, res, std::string("\"antialias\":") + (aa ? "true" : "false"));
            } else if (name == "conv" || name == "conv2d") {
                const auto w = names(op, "w");
                const uint32_t act = name == "conv" ? 1 : 0;
                if (w.size() < (act ? 3u : 2u)) throw std::runtime_error("graph.json: " + name + " lacks weights");
                const Json& st = op["stride"];
                const uint32_t stride = st.is_u64() ? (uint32_t)st.u64() : 1;
                const auto& t = tensor(w[0]);
                const uint32_t cout = t.dims.empty() ? 0 : t.dims[0];
                const View x = in(0);
                const uint32_t ho = (x.h + 2 - 3) / stride + 1, wo = (x.w + 2 - 3) / stride + 1;
                // the residual peephole (build.rs:222-237)
                if (i < to && ops.arr[i]["op"].str == "add" && used(outs[0]) == 1) {
                    const auto ai = names(ops.arr[i], "in");
                    if (ai.size() == 2 && (ai[0] == outs[0] || ai[1] == outs[0])) {
                        const std::string& other = ai[0] == outs[0] ? ai[1] : ai[0];
                        auto it = env.find(other);
                        if (it != env.end() && it->second.plain() && it->second.c == cout && it->second.h == ho &&
                            it->second.w == wo) {
                            const View r = it->second;
                            const std::string fused = names(ops.arr[i], "out").at(0);
                            env[fused] = conv(x, w[0], w[1], act ? w[2] : "", stride, act, &r, fused);
                            i++;
                            continue;
                        }
                    }
                }
                res = conv(x, w[0], w[1], act ? w[2] : "", stride, act, nullptr, outs[0]);
            } else if (name == "avgpool") {
                const View x = mat(in(0));
                const uint32_t kk = (uint32_t)op["k"].num;
                if (kk == 0) throw std::runtime_error("graph.json: avgpool k 0");
                res = alloc(x.c, x.h / kk, x.w / kk, outs[0]);
                step("avgpool", {x}, res, "\"k\":" + std::to_string(kk));
            } else if (name == "warp") {
                const View img = in(0), fl = in(1);
                res = alloc(img.c, img.h, img.w, outs[0]);
                step("warp", {img, fl}, res);
            } else if (name == "concat") {
                std::vector<View> xs;
                uint32_t c = 0;
                for (size_t j = 0; j < ins.size(); j++) {
                    xs.push_back(in(j));
                    c += xs.back().c;
                }
                res = alloc(c, xs[0].h, xs[0].w, outs[0]);
                step("concat", xs, res);
            } else if (name == "slice") {
                res = in(0).sub((uint32_t)op["a"].num, (uint32_t)op["b"].num);
            } else if (name == "scale") {
                res = in(0).scaled((float)op["factor"].num);
            } else if (name == "neg") {
                res = in(0).scaled(-1.0f);
            } else if (name == "copy") {
                res = in(0);
            } else if (name == "mul_t") {
                const View x = in(0);
                res = alloc(x.c, x.h, x.w, outs[0]);
                step("unary", {x}, res, std::string("\"fn\":0,\"mode\":") + jstr(op["mode"].str) + ",\"t\":true");
            } else if (name == "add" || name == "mul") {
                const View a = in(0), b = in(1);
                res = alloc(a.c, a.h, a.w, outs[0]);
                step("binary", {a, b}, res, std::string("\"fn\":") + (name == "add" ? "0" : "1"));
            } else if (name == "zeros" || name == "zeros_like") {
                const View r = in(0);
                const uint32_t c = name == "zeros" ? (uint32_t)op["ch"].num : r.c;
                res = alloc(c, r.h, r.w, outs[0], true);
            } else if (name == "luma") {
                const View x = in(0);
                res = alloc(1, x.h, x.w, outs[0]);
                step("luma", {x}, res);
            } else if (name == "luma_grad") {
                const View x = mat(in(0));
                res = alloc(1, x.h, x.w, outs[0]);
                step("luma_grad", {x}, res);
            } else if (name == "sad_volume") {
                const View a = mat(in(0)), b = mat(in(1));
                const uint32_t r = (uint32_t)op["radius"].num;
                res = alloc((2 * r + 1) * (2 * r + 1), a.h, a.w, outs[0]);
                step("sad", {a, b}, res, "\"radius\":" + std::to_string(r));
            } else if (name == "affine_out") {
                const View x = in(0);
                res = alloc(x.c, x.h, x.w, outs[0]);
                step("unary", {x}, res, "\"fn\":2");
            } else if (name == "clamp") {
                const View x = in(0);
                res = alloc(x.c, x.h, x.w, outs[0]);
                step("unary", {x}, res, "\"fn\":1,\"lo\":" + jnum(op["lo"].num) + ",\"hi\":" + jnum(op["hi"].num));
            } else if (name == "film_mlp") {
                const auto& b2 = tensor("film.film.2.bias");
                res = alloc(b2.dims.empty() ? 0 : b2.dims[0], 1, 1, outs[0]);
                step("film_mlp", {}, res, "\"t\":true");
            } else if (name == "film_modulate") {
                const View h = mat(in(0)), g = mat(in(1));
                res = alloc(h.c, h.h, h.w, outs[0]);
                step("film", {h, g}, res);
            } else if (name == "render_pix") {
                const View a = mat(in(0)), b = mat(in(1)), rt = mat(in(4));
                const View fl = in(2), vis = in(3);
                res = alloc(3, a.h, a.w, outs[0]);
                step("render", {a, b, fl, vis, rt}, res, "\"fsx\":" + jnum(fl.scale) + ",\"fsy\":" + jnum(fl.scale));
            } else if (name == "convex_upsample") {
                // up.w (48 -> 36, no activation), then the convex upsample (build.rs:379-416)
                const View h = mat(in(0)), x = mat(in(1));
                const View wt = conv(h, "up.w.weight", "up.w.bias", "", 1, 0, nullptr, outs[0] + ":w");
                res = alloc(x.c, 2 * x.h, 2 * x.w, outs[0]);
                step("convex", {wt, x}, res);
            } else if (name == "blend_weights") {
                // the blendmix peephole (build.rs:417-450)
                bool fused = false;
                if (i + 3 <= to && outs.size() == 2) {
                    const Json &m1 = ops.arr[i], &m2 = ops.arr[i + 1], &ad = ops.arr[i + 2];
                    const auto i1 = names(m1, "in"), i2 = names(m2, "in"), ia = names(ad, "in");
                    const auto o1 = names(m1, "out"), o2 = names(m2, "out");
                    auto only = [&](const std::string& n) { return used(n) == 1; };
                    if (m1["op"].str == "mul" && m2["op"].str == "mul" && ad["op"].str == "add" && i1.size() == 2 &&
                        i2.size() == 2 && ia.size() == 2 && !o1.empty() && !o2.empty() && i1[1] == outs[0] &&
                        i2[1] == outs[1] && ia[0] == o1[0] && ia[1] == o2[0] && only(outs[0]) && only(outs[1]) &&
                        only(o1[0]) && only(o2[0])) {
                        const View wa = mat(get(i1[0])), wb = mat(get(i2[0]));
                        const std::string out = names(ad, "out").at(0);
                        View o = alloc(wa.c, wa.h, wa.w, out);
                        step("blendmix", {wa, wb, in(0)}, o);
                        env[out] = o;
                        i += 3;
                        fused = true;
                    }
                }
                if (fused) continue;
                const View v = in(0);
                View bw = alloc(2, v.h, v.w, outs[0]);
                step("blend", {v}, bw);
                env[outs[0]] = bw.sub(0, 1);
                if (outs.size() > 1) env[outs[1]] = bw.sub(1, 2);
                continue;
            } else {
                throw std::runtime_error("graph.json: unhandled op " + name);
            }
            env[outs[0]] = res;
        }
    }
};

// the first t-dependent op (model/graph.rs:180-186)
size_t mid_start(const Json& ops, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const Json& o = ops.arr[i];
        if (o["op"].str == "mul_t" || o["op"].str == "film_mlp") return i;
        for (const std::string& s : names(o, "in"))
            if (s == "t") return i;
    }
    return n;
}

std::string plan_json(const fhc_model& m, uint32_t k, uint32_t fw, uint32_t fh, uint32_t nw, uint32_t nh,
                      uint32_t repair, std::vector<ConvUse>* convs = nullptr) {
    const uint32_t hp = (fh + 31) / 32 * 32, wp = (fw + 31) / 32 * 32;
    const uint32_t ihp = (nh + 31) / 32 * 32, iwp = (nw + 31) / 32 * 32;
    if (ihp > hp || iwp > wp) throw std::runtime_error("the network size exceeds the frame");
    const bool internal = ihp != hp || iwp != wp;
    Planner p{m, k, ihp, iwp, {}, {}, {}, {}, {}, "pair"};
    p.count_uses(m.ops);
    p.uses["t"] = 0;
    // the Session's inputs (net/session.rs:56-60): both frames through rgba_in at the padded size
    View a = p.alloc(3, hp, wp, "A"), b = p.alloc(3, hp, wp, "B");
    p.step("rgba_in", {}, a, "\"frame\":0");
    p.step("rgba_in", {}, b, "\"frame\":1");
    if (internal) {  // build.rs:615-620: the network's inputs are the antialiased downscale
        View ai = p.alloc(3, ihp, iwp, "A"), bi = p.alloc(3, ihp, iwp, "B");
        p.step("interp", {a}, ai, "\"antialias\":true");
        p.step("interp", {b}, bi, "\"antialias\":true");
        p.env["A"] = ai;
        p.env["B"] = bi;
    } else {
        p.env["A"] = a;
        p.env["B"] = b;
    }
    // in the internal mode the graph's own render_pix (its last op) is replaced by the frame-size render
    const size_t n = m.ops.arr.size();
    size_t rend = n;
    for (size_t i = n; i-- > 0;)
        if (m.ops.arr[i]["op"].str == "render_pix") {
            rend = i;
            break;
        }
    const size_t body = internal && rend < n ? rend : n;
    const size_t ms = mid_start(m.ops, body);
    p.walk(m.ops, 0, ms);
    if (repair > 0) {  // build.rs:640-660: the periodic-structure repair of the pair's flow, in place
        auto it = p.env.find("flow");
        View f;
        if (it != p.env.end()) {
            f = it->second;
        } else {  // the flow's readers are built; its buffer lives on in the flowf view
            auto jt = p.env.find("flowf");
            if (jt == p.env.end()) throw std::runtime_error("graph.json: the pair flow is not found for the repair");
            f = jt->second;
            f.c = 4, f.c0 = 0, f.scale = 1.0f;
        }
        if (!f.plain() || f.c != 4) throw std::runtime_error("graph.json: the pair flow is not a plain 4-channel tensor");
        p.step("gmhs", {p.get("A"), p.get("B"), f}, f,
               "\"level\":" + std::to_string(repair) + ",\"full_w\":" + std::to_string(wp));
    }
    p.stage = "mid";
    p.walk(m.ops, ms, body);
    View render;
    if (internal && rend < n) {  // build.rs:717-736
        const Json& op = m.ops.arr[rend];
        const auto ins = names(op, "in");
        if (ins.size() < 5) throw std::runtime_error("graph.json: render_pix lacks inputs");
        const View ftq = p.get(ins[2]), vtq = p.get(ins[3]), rt = p.mat(p.get(ins[4]));
        const float fsx = ftq.scale * (float)wp / (float)iwp, fsy = ftq.scale * (float)hp / (float)ihp;
        render = p.alloc(3, hp, wp, "render");
        p.step("render", {a, b, ftq, vtq, rt}, render, "\"fsx\":" + jnum(fsx) + ",\"fsy\":" + jnum(fsy));
    } else {
        auto it = p.env.find("render");
        if (it == p.env.end()) throw std::runtime_error("graph.json: no render output");
        render = it->second;
    }
    p.step("rgba_out", {render}, render);  // net/session.rs:63: the crop to the frame
    if (convs) *convs = p.convs;
    std::ostringstream o;
    o << "{\"frame\":[" << fw << "," << fh << "],\"padded\":[" << wp << "," << hp << "],\"network\":[" << iwp << ","
      << ihp << "],\"internal\":" << (internal ? "true" : "false") << ",\"k\":" << k << ",\"mid_start\":" << ms
      << ",\"buffers\":[";
    for (size_t i = 0; i < p.bufs.size(); i++) {
        const Buf& bb = p.bufs[i];
        o << (i ? "," : "") << "{\"c\":" << bb.c << ",\"h\":" << bb.h << ",\"w\":" << bb.w
          << ",\"zeros\":" << (bb.zeros ? "true" : "false") << ",\"name\":" << jstr(bb.name) << "}";
    }
    o << "],\"steps\":[";
    for (size_t i = 0; i < p.steps.size(); i++) o << (i ? "," : "") << p.steps[i];
    o << "]}";
    return o.str();
}

}  // namespace
}  // namespace fhc

extern "C" int fhc_model_load_bytes(const char* graph_json, size_t graph_len, const char* manifest_json,
                                    size_t manifest_len, const void* blob, size_t blob_len, fhc_model** out) {
    return guard(-1, [&]() -> int {
        if (!out) return fail(-1, "fhc_model_load_bytes: NULL output handle");
        *out = nullptr;
        if (!graph_json || !manifest_json || (!blob && blob_len)) return fail(-1, "fhc_model_load_bytes: NULL input");
        auto m = std::make_unique<fhc_model>();
        const uint8_t* bp = static_cast<const uint8_t*>(blob);
        m->blob.assign(bp, bp + blob_len);
        try {
            finish_load(*m, std::string(graph_json, graph_len), std::string(manifest_json, manifest_len));
        } catch (const std::exception& e) {
            return fail(-1, "fhc_model_load: %s", e.what());
        }
        *out = m.release();
        clear_error();
        return 0;
    });
}

extern "C" int fhc_model_load(const char* dir, fhc_model** out) {
    return guard(-1, [&]() -> int {
        if (!out) return fail(-1, "fhc_model_load: NULL output handle");
        *out = nullptr;
        if (!dir) return fail(-1, "fhc_model_load: NULL directory");
        std::string g, man, bin;
        try {
            const std::string d(dir);
            g = read_file(d + "/graph.json");
            man = read_file(d + "/flyhighfg.json");
            bin = read_file(d + "/flyhighfg.bin");
        } catch (const std::exception& e) {
            return fail(-1, "fhc_model_load: %s", e.what());
        }
        return fhc_model_load_bytes(g.data(), g.size(), man.data(), man.size(), bin.data(), bin.size(), out);
    });
}

extern "C" void fhc_model_destroy(fhc_model* m) { delete m; }

extern "C" int fhc_model_info(const fhc_model* m, char* json, size_t cap) {
    return guard(-1, [&]() -> int {
        if (!m) return fail(-1, "fhc_model_info: NULL model");
        const Json& meta = m->manifest["meta"];
        const bool cubic = meta["render_sampling"].is_str() && meta["render_sampling"].str == "bicubic";
        const Json& dk = meta["default_K"];
        std::ostringstream o;
        o << "{\"model\":" << jstr(meta["model"].is_str() ? meta["model"].str : "?")
          << ",\"train_step\":" << (meta["train_step"].kind == Json::Num ? (long long)meta["train_step"].num : -1)
          << ",\"graph_ops\":" << m->ops.arr.size() << ",\"tensors\":" << m->tensors.size()
          << ",\"params\":" << m->params << ",\"render_sampling\":\"" << (cubic ? "bicubic" : "bilinear")
          << "\",\"format_version\":" << m->format_version
          << ",\"default_k\":" << (dk.is_u64() ? (long long)dk.u64() : 1) << "}";
        return write_string(o.str(), json, cap);
    });
}

extern "C" int fhc_model_tensor(const fhc_model* m, const char* name, uint32_t* dims, size_t cap, uint64_t* count) {
    return guard(-1, [&]() -> int {
        if (!m || !name) return fail(-1, "fhc_model_tensor: NULL argument");
        auto it = m->tensors.find(name);
        if (it == m->tensors.end()) return fail(-1, "fhc_model_tensor: no tensor %s", name);
        const auto& t = it->second;
        if (t.dims.size() > cap || (!dims && !t.dims.empty()))
            return fail(-1, "fhc_model_tensor: %zu dimensions do not fit", t.dims.size());
        for (size_t i = 0; i < t.dims.size(); i++) dims[i] = t.dims[i];
        if (count) *count = t.count;
        return (int)t.dims.size();
    });
}

extern "C" int64_t fhc_model_weight(const fhc_model* m, const char* name, uint16_t* out, size_t cap) {
    return guard((int64_t)-1, [&]() -> int64_t {
        if (!m || !name) return fail(-1, "fhc_model_weight: NULL argument");
        auto it = m->tensors.find(name);
        if (it == m->tensors.end()) return fail(-1, "fhc_model_weight: no tensor %s", name);
        const auto& t = it->second;
        if (t.count > cap || (!out && t.count))
            return fail(-1, "fhc_model_weight: %llu values do not fit", (unsigned long long)t.count);
        const uint8_t* p = m->blob.data() + t.offset * 2;
        for (uint64_t i = 0; i < t.count; i++) out[i] = (uint16_t)(p[2 * i] | (p[2 * i + 1] << 8));
        return (int64_t)t.count;
    });
}

extern "C" int fhc_model_plan(const fhc_model* m, uint32_t k, uint32_t frame_w, uint32_t frame_h, uint32_t net_w,
                              uint32_t net_h, uint32_t repair, char* json, size_t cap) {
    return guard(-1, [&]() -> int {
        if (!m) return fail(-1, "fhc_model_plan: NULL model");
        if (!frame_w || !frame_h || !net_w || !net_h || frame_w > 16384 || frame_h > 16384)
            return fail(-1, "fhc_model_plan: bad sizes (frame %u x %u, network %u x %u)", frame_w, frame_h, net_w,
                        net_h);
        if (k == 0 || k > 16) return fail(-1, "fhc_model_plan: k must be 1..16");
        if (repair > 2) return fail(-1, "fhc_model_plan: repair level %u (0 off, 1 safe, 2 aggressive)", repair);
        std::string s;
        try {
            s = plan_json(*m, k, frame_w, frame_h, net_w, net_h, repair);
        } catch (const std::exception& e) {
            return fail(-1, "fhc_model_plan: %s", e.what());
        }
        return write_string(s, json, cap);
    });
}

namespace fhc {
namespace {

struct ShapeKey {
    uint32_t v[7];
    bool operator<(const ShapeKey& o) const { return std::memcmp(v, o.v, sizeof v) < 0; }
};

// the plan's distinct conv shapes at batch n, in plan order, with the first use of each
std::vector<std::pair<ShapeKey, ConvUse>> conv_shapes(const fhc_model& m, uint32_t k, uint32_t fw, uint32_t fh,
                                                      uint32_t nw, uint32_t nh, uint32_t n) {
    std::vector<ConvUse> convs;
    plan_json(m, k, fw, fh, nw, nh, 0, &convs);
    std::vector<std::pair<ShapeKey, ConvUse>> out;
    std::set<ShapeKey> seen;
    for (const ConvUse& c : convs) {
        const ShapeKey key{{c.cin, c.cout, c.h, c.wd, c.stride, n, 3}};
        if (seen.insert(key).second) out.emplace_back(key, c);
    }
    return out;
}

int plan_args(const fhc_model* m, uint32_t k, uint32_t fw, uint32_t fh, uint32_t nw, uint32_t nh, const char* what) {
    if (!m) return fail(-1, "%s: NULL model", what);
    if (!fw || !fh || !nw || !nh || fw > 16384 || fh > 16384)
        return fail(-1, "%s: bad sizes (frame %u x %u, network %u x %u)", what, fw, fh, nw, nh);
    if (k == 0 || k > 16) return fail(-1, "%s: k must be 1..16", what);
    return 0;
}

// seeded f16 values of magnitude 2^-5 .. 2^-1 with random signs and mantissas (finite, no conversion needed)
void seeded_f16(std::vector<uint16_t>& v, uint32_t seed) {
    uint32_t x = seed * 2654435761u + 12345u;
    for (uint16_t& h : v) {
        x = x * 1664525u + 1013904223u;
        h = (uint16_t)(((x >> 31) << 15) | ((10u + (x >> 24) % 5u) << 10) | ((x >> 8) & 0x3ffu));
    }
}

std::vector<uint16_t> weight_bits(const fhc_model& m, const std::string& name) {
    const auto& t = m.tensors.at(name);
    std::vector<uint16_t> out(t.count);
    const uint8_t* p = m.blob.data() + t.offset * 2;
    for (uint64_t i = 0; i < t.count; i++) out[i] = (uint16_t)(p[2 * i] | (p[2 * i + 1] << 8));
    return out;
}

}  // namespace
}  // namespace fhc

extern "C" int fhc_model_conv_shapes(const fhc_model* m, uint32_t k, uint32_t frame_w, uint32_t frame_h,
                                     uint32_t net_w, uint32_t net_h, uint32_t n, uint32_t* out, size_t cap) {
    return guard(-1, [&]() -> int {
        clear_error();
        const int rc = plan_args(m, k, frame_w, frame_h, net_w, net_h, "fhc_model_conv_shapes");
        if (rc < 0) return rc;
        if (n == 0) return fail(-1, "fhc_model_conv_shapes: batch 0");
        std::vector<std::pair<ShapeKey, ConvUse>> shapes;
        try {
            shapes = conv_shapes(*m, k, frame_w, frame_h, net_w, net_h, n);
        } catch (const std::exception& e) {
            return fail(-1, "fhc_model_conv_shapes: %s", e.what());
        }
        for (size_t i = 0; i < shapes.size() && (i + 1) * 7 <= cap; i++)
            std::memcpy(out + 7 * i, shapes[i].first.v, sizeof shapes[i].first.v);
        return (int)shapes.size();
    });
}

extern "C" int fhc_model_autotune(const fhc_model* m, uint32_t k, uint32_t frame_w, uint32_t frame_h, uint32_t net_w,
                                  uint32_t net_h, uint32_t n, int reps) {
    return guard(-1, [&]() -> int {
        clear_error();
        const int rc = plan_args(m, k, frame_w, frame_h, net_w, net_h, "fhc_model_autotune");
        if (rc < 0) return rc;
        if (n == 0 || n > 64) return fail(-1, "fhc_model_autotune: batch %u (1..64)", n);
        std::vector<std::pair<ShapeKey, ConvUse>> shapes;
        try {
            shapes = conv_shapes(*m, k, frame_w, frame_h, net_w, net_h, n);
        } catch (const std::exception& e) {
            return fail(-1, "fhc_model_autotune: %s", e.what());
        }
        auto pad8 = [](uint32_t c) { return (c + 7) / 8 * 8; };
        int tuned = 0;
        for (const auto& [key, c] : shapes) {
            fhc_conv_desc d{};
            d.n = n, d.h = c.h, d.w = c.wd, d.cin = c.cin, d.cout = c.cout, d.kh = d.kw = 3, d.stride = c.stride;
            d.pad = 1, d.act = c.act ? FHC_ACT_PRELU : FHC_ACT_NONE, d.residual = c.res ? 1 : 0, d.ref_cand = 0xFF;
            d.x_cstride = pad8(c.cin), d.y_cstride = pad8(c.cout), d.r_cstride = c.res ? pad8(c.cout) : 0;
            const uint32_t ho = (c.h + 2 - 3) / c.stride + 1, wo = (c.wd + 2 - 3) / c.stride + 1;
            const size_t xe = (size_t)n * c.h * c.wd * d.x_cstride, ye = (size_t)n * ho * wo * d.y_cstride;
            std::vector<uint16_t> xh(xe), rh(c.res ? ye : 0);
            seeded_f16(xh, key.v[0] * 31u + key.v[2]);
            seeded_f16(rh, key.v[1] * 37u + key.v[3]);
            const std::vector<uint16_t> w = weight_bits(*m, c.w), b = weight_bits(*m, c.b);
            const std::vector<uint16_t> sl = c.act ? weight_bits(*m, c.s) : std::vector<uint16_t>();
            void *x = nullptr, *y = nullptr, *r = nullptr;
            auto release = [&]() {
                if (x) (void)hipFree(x);
                if (y) (void)hipFree(y);
                if (r) (void)hipFree(r);
            };
            if (hipMalloc(&x, xe * 2) != hipSuccess || hipMalloc(&y, ye * 2) != hipSuccess ||
                (c.res && hipMalloc(&r, ye * 2) != hipSuccess) ||
                hipMemcpy(x, xh.data(), xe * 2, hipMemcpyHostToDevice) != hipSuccess ||
                (c.res && hipMemcpy(r, rh.data(), ye * 2, hipMemcpyHostToDevice) != hipSuccess)) {
                release();
                return fail(-2, "fhc_model_autotune: device buffers for %s (%u -> %u at %u x %u, batch %u)",
                            c.w.c_str(), c.cin, c.cout, c.wd, c.h, n);
            }
            float us = 0.0f;
            const int code = fhc_conv_autotune(&d, w.data(), b.data(), c.act ? sl.data() : nullptr, x, y, r,
                                               reps, &us);
            release();
            if (code < 0) return code;
            tuned++;
        }
        return tuned;
    });
}
