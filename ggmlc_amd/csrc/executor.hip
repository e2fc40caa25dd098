// The executor handle of libgq: a ggmlc .gguf (GGUF v3 with the `ggmlc.graph_spec`
// execution graph) loaded, matched against the LLaMA-family decoder layout, and run on
// this library's kernels with one HIP graph per (s, n_kv, output rows) bucket. It is
// ggmlc's ModelExecutor (runtime/include/ggmlc/executor.h:25-289, bound to Python at
// runtime/bindings/python_bindings.cpp:137-216) for the graphs this path executes:
// create from file bytes and a device, prepare(symbols), set_input, run, outputs and
// their concrete shapes, the persistent KV cache (init/reset/has), logits_last_only.
// Host code only; no torch. Every launch goes through the validated gq_* entry points.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace gq {
namespace {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void raise(int code, const std::string& m) { throw Error(code, m); }

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) raise(GQ_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

// a gq_* call: its message is already set; rethrown so the handle's call unwinds
void gq_ok(int rc) {
    if (rc != GQ_OK) throw Error(rc, gq_last_error());
}

// ------------------------------------------------------------------------ JSON
// The subset of JSON the graph spec uses (objects, arrays, strings with the usual escapes,
// numbers, true/false/null). Numbers keep their double value and, for integer literals,
// the exact int64.
struct JVal {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    int64_t i = 0;
    bool integral = false;
    std::string s;
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;

    const JVal* get(const std::string& k) const {
        for (const auto& kv : o)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    int64_t as_int(int64_t def = 0) const {
        if (kind == Bool) return b ? 1 : 0;
        if (kind == Num) return integral ? i : (int64_t)num;
        return def;
    }
    double as_double(double def = 0.0) const {
        if (kind == Bool) return b ? 1.0 : 0.0;
        if (kind == Num) return num;
        return def;
    }
};

struct JParser {
    const char* p;
    const char* e;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    [[noreturn]] void bad(const char* what) { raise(GQ_ERR_INVALID, std::string("graph_spec JSON: ") + what); }
    void lit(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(e - p) < n || strncmp(p, w, n) != 0) bad("bad literal");
        p += n;
    }
    static void utf8(std::string& out, uint32_t c) {
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
    uint32_t hex4() {
        if (e - p < 4) bad("short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else bad("bad \\u escape");
        }
        return v;
    }
    std::string str() {
        if (p >= e || *p != '"') bad("expected a string");
        ++p;
        std::string out;
        while (p < e && *p != '"') {
            char c = *p++;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p >= e) bad("bad escape");
            c = *p++;
            switch (c) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        const uint32_t lo = hex4();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(out, cp);
                    break;
                }
                default: bad("bad escape");
            }
        }
        if (p >= e) bad("unterminated string");
        ++p;
        return out;
    }
    void value(JVal& v, int depth) {
        if (depth > 200) bad("nesting too deep");
        ws();
        if (p >= e) bad("unexpected end");
        const char c = *p;
        if (c == '{') {
            ++p;
            v.kind = JVal::Obj;
            ws();
            if (p < e && *p == '}') {
                ++p;
                return;
            }
            for (;;) {
                ws();
                std::string k = str();
                ws();
                if (p >= e || *p != ':') bad("expected ':'");
                ++p;
                v.o.emplace_back(std::move(k), JVal());
                value(v.o.back().second, depth + 1);
                ws();
                if (p < e && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < e && *p == '}') {
                    ++p;
                    return;
                }
                bad("expected ',' or '}'");
            }
        } else if (c == '[') {
            ++p;
            v.kind = JVal::Arr;
            ws();
            if (p < e && *p == ']') {
                ++p;
                return;
            }
            for (;;) {
                v.a.emplace_back();
                value(v.a.back(), depth + 1);
                ws();
                if (p < e && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < e && *p == ']') {
                    ++p;
                    return;
                }
                bad("expected ',' or ']'");
            }
        } else if (c == '"') {
            v.kind = JVal::Str;
            v.s = str();
        } else if (c == 't') {
            lit("true");
            v.kind = JVal::Bool;
            v.b = true;
        } else if (c == 'f') {
            lit("false");
            v.kind = JVal::Bool;
        } else if (c == 'n') {
            lit("null");
        } else {
            const char* s0 = p;
            bool integral = true;
            if (p < e && (*p == '-' || *p == '+')) ++p;
            while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' ||
                             *p == '+')) {
                if (*p == '.' || *p == 'e' || *p == 'E') integral = false;
                ++p;
            }
            if (p == s0) bad("unexpected character");
            const std::string t(s0, p);
            v.kind = JVal::Num;
            v.num = strtod(t.c_str(), nullptr);
            v.integral = integral;
            v.i = integral ? (int64_t)strtoll(t.c_str(), nullptr, 10) : (int64_t)v.num;
        }
    }
};

JVal parse_json(const std::string& text) {
    JParser ps{text.data(), text.data() + text.size()};
    JVal v;
    ps.value(v, 0);
    ps.ws();
    if (ps.p != ps.e) raise(GQ_ERR_INVALID, "graph_spec JSON: trailing characters");
    return v;
}

// ------------------------------------------------------------------ dimensions
// DimExpr of runtime/include/ggmlc/types.h:24-75: static | symbol | add | sub | mul |
// floordiv | ceildiv over int64 (division truncates toward zero; ceildiv is
// (l + r - 1) / r); unknown kinds read as static 1 (loader.cpp:218-250).
struct Dim {
    enum Kind { Static, Symbol, Add, Sub, Mul, FloorDiv, CeilDiv } kind = Static;
    int64_t val = 1;
    std::string name;
    std::shared_ptr<Dim> l, r;

    static Dim from_json(const JVal& j) {
        Dim d;
        const JVal* t = j.get("type");
        const std::string ty = t && t->kind == JVal::Str ? t->s : "static";
        if (ty == "static") {
            const JVal* v = j.get("val");
            d.val = v ? v->as_int(1) : 1;
            return d;
        }
        if (ty == "symbol") {
            d.kind = Symbol;
            const JVal* n = j.get("name");
            d.name = n && n->kind == JVal::Str ? n->s : "";
            return d;
        }
        static const std::map<std::string, Kind> ops = {
            {"add", Add}, {"sub", Sub}, {"mul", Mul}, {"floordiv", FloorDiv}, {"ceildiv", CeilDiv}};
        auto it = ops.find(ty);
        const JVal* lj = j.get("left");
        const JVal* rj = j.get("right");
        if (it == ops.end() || !lj || !rj) return d;
        d.kind = it->second;
        d.l = std::make_shared<Dim>(from_json(*lj));
        d.r = std::make_shared<Dim>(from_json(*rj));
        return d;
    }

    int64_t eval(const std::map<std::string, int64_t>& env) const {
        switch (kind) {
            case Static: return val;
            case Symbol: {
                auto it = env.find(name);
                if (it == env.end()) raise(GQ_ERR_INVALID, "symbol not set: " + name);
                return it->second;
            }
            default: break;
        }
        const int64_t a = l->eval(env), b = r->eval(env);
        switch (kind) {
            case Add: return a + b;
            case Sub: return a - b;
            case Mul: return a * b;
            case FloorDiv:
                if (b == 0) raise(GQ_ERR_INVALID, "division by zero in a dimension");
                return a / b;
            case CeilDiv:
                if (b == 0) raise(GQ_ERR_INVALID, "division by zero in a dimension");
                return (a + b - 1) / b;
            default: return 1;
        }
    }
};

// ---------------------------------------------------------------------- graph
enum Storage { S_INPUT = 0, S_PARAMETER = 1, S_CONSTANT = 2, S_ACTIVATION = 3, S_STATE = 4, S_OUTPUT = 5 };
// ggml 0.20.2 enum ggml_op values of the nodes the decoder layout uses
enum Op {
    OP_ADD = 2, OP_RMS_NORM = 25, OP_MUL_MAT = 29, OP_RESHAPE = 36, OP_VIEW = 37, OP_PERMUTE = 38,
    OP_GET_ROWS = 40, OP_ROPE = 48, OP_FLASH_ATTN_EXT = 74, OP_GLU = 100
};

struct GTensor {
    uint32_t id = 0;
    std::string name;
    int type = 0;
    Dim ne[4];
    int storage = S_ACTIVATION;
};

struct GNode {
    uint32_t id = 0;
    int opcode = 0;
    std::vector<uint32_t> in, out;
    std::map<std::string, JVal> attr;
    std::string name;
    bool has(const std::string& k) const { return attr.count(k) != 0; }
    int64_t attr_int(const std::string& k, int64_t def) const {
        auto it = attr.find(k);
        return it == attr.end() ? def : it->second.as_int(def);
    }
    double attr_f(const std::string& k, double def) const {
        auto it = attr.find(k);
        return it == attr.end() ? def : it->second.as_double(def);
    }
};

struct Graph {
    std::string name = "main";
    std::vector<uint32_t> inputs, outputs, parameters;
    std::vector<std::string> symbols;
    std::map<uint32_t, GTensor> tensors;
    std::vector<GNode> nodes;

    const GTensor& t(uint32_t id) const {
        auto it = tensors.find(id);
        if (it == tensors.end()) raise(GQ_ERR_INVALID, "graph_spec: unknown tensor id " + std::to_string(id));
        return it->second;
    }
};

std::vector<uint32_t> ids_of(const JVal* a) {
    std::vector<uint32_t> out;
    if (a && a->kind == JVal::Arr)
        for (const auto& v : a->a) out.push_back((uint32_t)v.as_int());
    return out;
}

Graph parse_graph(const std::string& text) {
    const JVal j = parse_json(text);
    if (j.kind != JVal::Obj) raise(GQ_ERR_INVALID, "graph_spec: not an object");
    Graph g;
    if (const JVal* n = j.get("name"); n && n->kind == JVal::Str) g.name = n->s;
    g.inputs = ids_of(j.get("inputs"));
    g.outputs = ids_of(j.get("outputs"));
    g.parameters = ids_of(j.get("parameters"));
    if (const JVal* st = j.get("symbol_table"); st && st->kind == JVal::Arr)
        for (const auto& v : st->a) g.symbols.push_back(v.s);
    if (const JVal* ts = j.get("tensors"); ts && ts->kind == JVal::Obj) {
        for (const auto& kv : ts->o) {
            const JVal& td = kv.second;
            GTensor t;
            const JVal* idv = td.get("id");
            t.id = idv ? (uint32_t)idv->as_int() : (uint32_t)strtoul(kv.first.c_str(), nullptr, 10);
            if (const JVal* n = td.get("name"); n && n->kind == JVal::Str) t.name = n->s;
            if (const JVal* ty = td.get("type")) t.type = (int)ty->as_int();
            if (const JVal* st = td.get("storage")) t.storage = (int)st->as_int(S_ACTIVATION);
            if (const JVal* ne = td.get("ne"); ne && ne->kind == JVal::Arr)
                for (size_t i = 0; i < ne->a.size() && i < 4; ++i) t.ne[i] = Dim::from_json(ne->a[i]);
            g.tensors[t.id] = std::move(t);
        }
    }
    if (const JVal* ns = j.get("nodes"); ns && ns->kind == JVal::Arr) {
        for (const auto& nd : ns->a) {
            GNode n;
            if (const JVal* v = nd.get("id")) n.id = (uint32_t)v->as_int();
            if (const JVal* v = nd.get("opcode")) n.opcode = (int)v->as_int();
            n.in = ids_of(nd.get("inputs"));
            n.out = ids_of(nd.get("outputs"));
            if (const JVal* a = nd.get("attributes"); a && a->kind == JVal::Obj)
                for (const auto& kv : a->o) n.attr[kv.first] = kv.second;
            if (const JVal* v = nd.get("name"); v && v->kind == JVal::Str) n.name = v->s;
            g.nodes.push_back(std::move(n));
        }
    }
    return g;
}

// ----------------------------------------------------------------------- GGUF
// GGUF v3 (ggml gguf.cpp; ggmlc serialization/gguf.py:225-362): "GGUF", u32 version,
// u64 n_tensors, u64 n_kv, the key/values, the tensor infos, padding to
// general.alignment (default 32), then the data section.
struct GgufTensor {
    std::string name;
    int64_t ne[4] = {1, 1, 1, 1};
    int type = 0;
    uint64_t offset = 0, nbytes = 0;
};

struct Gguf {
    std::vector<uint8_t> buf;
    size_t pos = 0;
    std::map<std::string, std::string> strings;  // string-valued metadata
    uint64_t alignment = 32;
    std::map<std::string, GgufTensor> tensors;
    uint64_t data_start = 0;

    void need(size_t n) {
        if (pos + n > buf.size()) raise(GQ_ERR_INVALID, "GGUF: truncated file");
    }
    template <typename T>
    T rd() {
        need(sizeof(T));
        T v;
        memcpy(&v, buf.data() + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string rstr() {
        const uint64_t n = rd<uint64_t>();
        need(n);
        std::string s(reinterpret_cast<const char*>(buf.data() + pos), n);
        pos += n;
        return s;
    }
    static size_t scalar_size(uint32_t t) {
        switch (t) {
            case 0: case 1: case 7: return 1;   // u8 i8 bool
            case 2: case 3: return 2;           // u16 i16
            case 4: case 5: case 6: return 4;   // u32 i32 f32
            case 10: case 11: case 12: return 8;  // u64 i64 f64
            default: return 0;
        }
    }
    void skip_value(uint32_t t, int depth) {
        if (depth > 8) raise(GQ_ERR_INVALID, "GGUF: arrays nested too deep");
        if (t == 8) {
            rstr();
            return;
        }
        if (t == 9) {
            const uint32_t et = rd<uint32_t>();
            const uint64_t n = rd<uint64_t>();
            if (et == 8 || et == 9) {
                for (uint64_t k = 0; k < n; ++k) skip_value(et, depth + 1);
                return;
            }
            const size_t sz = scalar_size(et);
            if (!sz) raise(GQ_ERR_INVALID, "GGUF: bad array element type");
            if (n > buf.size() / sz) raise(GQ_ERR_INVALID, "GGUF: truncated file");
            need((size_t)(n * sz));
            pos += (size_t)(n * sz);
            return;
        }
        const size_t sz = scalar_size(t);
        if (!sz) raise(GQ_ERR_INVALID, "GGUF: bad value type " + std::to_string(t));
        need(sz);
        pos += sz;
    }
    // bytes of a tensor of ne elements (ne already checked: non-negative, a product that
    // fits int64), refusing sizes that do not fit a size_t; 0 for types this loader
    // does not know
    static uint64_t type_nbytes(int type, const int64_t* ne) {
        int64_t blk = 1, bs = 0;
        switch (type) {
            case GQ_TYPE_F32: case GQ_TYPE_I32: bs = 4; break;
            case GQ_TYPE_F16: bs = 2; break;
            case GQ_TYPE_I64: bs = 8; break;
            case GQ_TYPE_Q8_0: blk = 32, bs = Q8_BYTES; break;
            case GQ_TYPE_Q4_0: blk = 32, bs = Q4_BYTES; break;
            case 24: bs = 1; break;   // I8
            case 25: case 30: bs = 2; break;  // I16, BF16
            case 28: bs = 8; break;   // F64
            default: return 0;
        }
        if (ne[0] % blk) raise(GQ_ERR_INVALID, "GGUF: rows of partial blocks");
        uint64_t n = (uint64_t)(ne[0] / blk);
        for (int i = 1; i < 4; ++i) n *= (uint64_t)ne[i];  // <= the element count: no wrap
        if (n > (uint64_t)SIZE_MAX / (uint64_t)bs) raise(GQ_ERR_INVALID, "GGUF: tensor byte size overflows");
        return n * (uint64_t)bs;
    }

    void parse() {
        pos = 0;
        need(4);
        if (memcmp(buf.data(), "GGUF", 4) != 0) raise(GQ_ERR_INVALID, "GGUF: magic header mismatch");
        pos = 4;
        const uint32_t version = rd<uint32_t>();
        if (version != 2 && version != 3) raise(GQ_ERR_INVALID, "GGUF: unsupported version");
        const uint64_t n_tensors = rd<uint64_t>(), n_kv = rd<uint64_t>();
        for (uint64_t k = 0; k < n_kv; ++k) {
            const std::string key = rstr();
            const uint32_t t = rd<uint32_t>();
            if (t == 8) {
                strings[key] = rstr();
            } else if (key == "general.alignment" && t == 4) {
                alignment = rd<uint32_t>();
            } else {
                skip_value(t, 0);
            }
        }
        if (!alignment || (alignment & (alignment - 1))) raise(GQ_ERR_INVALID, "GGUF: bad alignment");
        for (uint64_t k = 0; k < n_tensors; ++k) {
            GgufTensor ti;
            ti.name = rstr();
            const uint32_t nd = rd<uint32_t>();
            if (nd > 4) raise(GQ_ERR_INVALID, "GGUF: more than 4 dimensions");
            for (uint32_t d = 0; d < nd; ++d) {
                ti.ne[d] = (int64_t)rd<uint64_t>();
                if (ti.ne[d] < 0) raise(GQ_ERR_INVALID, "GGUF: negative dimension in tensor " + ti.name);
            }
            // the element count must be an int64 (ggml_nelements)
            int64_t nel = 1;
            for (int d = 0; d < 4; ++d) {
                if (ti.ne[d] != 0 && nel > INT64_MAX / ti.ne[d])
                    raise(GQ_ERR_INVALID, "GGUF: element count of tensor " + ti.name + " overflows");
                nel *= ti.ne[d];
            }
            ti.type = (int)rd<uint32_t>();
            ti.offset = rd<uint64_t>();
            ti.nbytes = type_nbytes(ti.type, ti.ne);
            if (tensors.count(ti.name)) raise(GQ_ERR_INVALID, "GGUF: duplicate tensor " + ti.name);
            tensors[ti.name] = ti;
        }
        data_start = (pos + alignment - 1) / alignment * alignment;
        // every comparison below is free of wrap-around: data = bytes after data_start
        const uint64_t data = data_start <= buf.size() ? buf.size() - data_start : 0;
        for (const auto& kv : tensors) {
            const GgufTensor& ti = kv.second;
            if (ti.offset % alignment) raise(GQ_ERR_INVALID, "GGUF: unaligned tensor " + ti.name);
            if (ti.offset > data || ti.nbytes > data - ti.offset)
                raise(GQ_ERR_INVALID, "GGUF: tensor " + ti.name + " runs past the end of the file");
        }
    }
    const GgufTensor& tensor(const std::string& name) const {
        auto it = tensors.find(name);
        if (it == tensors.end()) raise(GQ_ERR_INVALID, "GGUF: no tensor named " + name);
        return it->second;
    }
    const uint8_t* data(const GgufTensor& t) const { return buf.data() + data_start + t.offset; }
};

// ---------------------------------------------------------------- the matcher
// The decoder layout ggmlc's runtime executes for LLaMA-family models (the graph
// ggmlc_amd/llama_gguf.py writes and ggmlc's compiler emits after its fusion passes):
// GET_ROWS embedding, per layer RMS_NORM -> QKV MUL_MAT (one fused product with three
// VIEWs, or three products; optional F32 bias inputs) -> RESHAPE [hd, H, s] -> NEOX ROPE
// of q and k -> PERMUTE -> FLASH_ATTN_EXT -> RESHAPE -> output MUL_MAT -> ADD, RMS_NORM ->
// gate|up MUL_MAT -> GLU SWIGLU -> down MUL_MAT -> ADD; final RMS_NORM -> head MUL_MAT.
struct WeightRef {
    std::vector<std::string> names;  // row blocks concatenated in order
    std::vector<std::string> bias;   // matching bias tensors (empty: none)
    int type = 0;
    int64_t K = 0, N = 0;
};

struct Match {
    uint32_t input_tid = 0, output_tid = 0;
    std::string embed, lm_head;
    int embed_type = 0, lm_type = 0;
    int64_t n_embd = 0, n_vocab = 0, hd = 0, n_head = 0, n_head_kv = 0, n_ff = 0;
    float rms_eps = 1e-5f, rope_base = 10000.0f;
    struct Layer {
        WeightRef qkv, o, gate_up, down;
    };
    std::vector<Layer> layers;
};

[[noreturn]] void unmapped(const GNode& n, const std::string& why) {
    raise(GQ_ERR_UNSUPPORTED, "graph node " + std::to_string(n.id) + " (opcode " + std::to_string(n.opcode) + " '" +
                                  n.name + "'): " + why);
}

Match match_llama(const Graph& g, const Gguf& f) {
    std::map<uint32_t, const GNode*> prod;
    std::map<uint32_t, std::vector<const GNode*>> cons;
    for (const GNode& n : g.nodes) {
        for (uint32_t o : n.out) prod[o] = &n;
        for (uint32_t i : n.in) cons[i].push_back(&n);
    }
    Match m;
    std::vector<uint32_t> ins;
    for (uint32_t t : g.inputs)
        if (g.t(t).storage == S_INPUT) ins.push_back(t);
    if (ins.size() != 1 || (g.t(ins[0]).type != GQ_TYPE_I32 && g.t(ins[0]).type != GQ_TYPE_I64))
        raise(GQ_ERR_UNSUPPORTED, "expected one integer input (token ids)");
    m.input_tid = ins[0];
    if (g.outputs.size() != 1) raise(GQ_ERR_UNSUPPORTED, "expected one output (logits)");
    m.output_tid = g.outputs[0];
    static const std::vector<const GNode*> none;
    auto consumers = [&](uint32_t t) -> const std::vector<const GNode*>& {
        auto it = cons.find(t);
        return it == cons.end() ? none : it->second;
    };
    auto only = [&](uint32_t t, int op, const char* what, const GNode& from) -> const GNode& {
        const GNode* sel = nullptr;
        int n = 0;
        for (const GNode* c : consumers(t))
            if (c->opcode == op) sel = c, ++n;
        if (n != 1) unmapped(from, std::string("expected one ") + what + " consumer, found " + std::to_string(n));
        return *sel;
    };
    auto weight = [&](const GNode& node) {
        const GTensor& t = g.t(node.in.at(0));
        if ((t.type != GQ_TYPE_Q8_0 && t.type != GQ_TYPE_Q4_0) || !f.tensors.count(t.name))
            unmapped(node, "weight '" + t.name + "' must be a Q8_0/Q4_0 tensor stored in the file");
        const GgufTensor& ft = f.tensor(t.name);
        if (ft.type != t.type) unmapped(node, "weight '" + t.name + "' type differs from the file");
        WeightRef w;
        w.names = {t.name};
        w.type = t.type;
        w.K = ft.ne[0];
        w.N = ft.ne[1];
        return w;
    };
    auto bias_of = [&](const GNode& node, int64_t n) -> std::string {
        if (node.in.size() < 3) return "";
        if (node.in.size() > 3) unmapped(node, "MUL_MAT with more than three inputs");
        const GTensor& t = g.t(node.in[2]);
        if (t.type != GQ_TYPE_F32 || !f.tensors.count(t.name))
            unmapped(node, "bias '" + t.name + "' must be an F32 tensor stored in the file");
        const GgufTensor& ft = f.tensor(t.name);
        if (ft.ne[0] * ft.ne[1] * ft.ne[2] * ft.ne[3] != n) unmapped(node, "bias '" + t.name + "' size");
        return t.name;
    };
    auto rms_eps = [&](const GNode& node) {
        if (node.in.size() != 1) unmapped(node, "RMS_NORM with a weight input (expected it baked into the next MUL_MAT)");
        // the runtime reads eps through its integer map (executor.cpp:2024)
        return node.has("eps") ? (float)node.attr_int("eps", 0) : 1e-5f;
    };

    const GNode* emb = nullptr;
    for (const GNode& n : g.nodes)
        if (n.opcode == OP_GET_ROWS && std::find(n.in.begin(), n.in.end(), m.input_tid) != n.in.end()) {
            if (emb) raise(GQ_ERR_UNSUPPORTED, "expected the token ids to feed one GET_ROWS (embedding)");
            emb = &n;
        }
    if (!emb) raise(GQ_ERR_UNSUPPORTED, "expected the token ids to feed one GET_ROWS (embedding)");
    {
        WeightRef w = weight(*emb);
        m.embed = w.names[0], m.embed_type = w.type, m.n_embd = w.K, m.n_vocab = w.N;
    }
    uint32_t x = emb->out.at(0);
    std::vector<float> eps, bases;
    for (;;) {
        auto pit = prod.find(x);
        const GNode& norm = only(x, OP_RMS_NORM, "RMS_NORM", pit == prod.end() ? *emb : *pit->second);
        eps.push_back(rms_eps(norm));
        const uint32_t h = norm.out.at(0);
        std::vector<const GNode*> mms;
        for (const GNode* c : consumers(h))
            if (c->opcode == OP_MUL_MAT) mms.push_back(c);
        if (mms.size() == 1 && mms[0]->out.at(0) == m.output_tid) {  // final norm -> output head
            WeightRef w = weight(*mms[0]);
            if (w.K != m.n_embd || w.N != m.n_vocab) unmapped(*mms[0], "output head shape");
            if (mms[0]->in.size() > 2) unmapped(*mms[0], "an output head with a bias is not mapped");
            m.lm_head = w.names[0], m.lm_type = w.type;
            break;
        }
        Match::Layer L;
        std::vector<const GNode*> srcs;
        bool fused = false;
        if (mms.size() == 1) {
            fused = true;
            L.qkv = weight(*mms[0]);
            std::vector<const GNode*> views;
            for (const GNode* c : consumers(mms[0]->out.at(0)))
                if (c->opcode == OP_VIEW) views.push_back(c);
            if (views.size() != 3) unmapped(*mms[0], "fused QKV product must feed three VIEWs");
            std::sort(views.begin(), views.end(),
                      [](const GNode* a, const GNode* b) { return a->attr_int("start", 0) < b->attr_int("start", 0); });
            for (const GNode* v : views)
                if (v->attr_int("ggml_dim", 0) != 0 || v->attr_int("step", 1) != 1)
                    unmapped(*v, "QKV views must slice ne[0]");
            srcs = views;
        } else if (mms.size() == 3) {
            srcs = mms;
        } else {
            unmapped(norm, "expected 1 (fused) or 3 QKV products, found " + std::to_string(mms.size()));
        }
        struct Path {
            int64_t slot, hd, H;
            const GNode *src, *rope, *fa;
        };
        std::vector<Path> paths;
        const std::map<std::string, int64_t> one = {{"s", 1}};
        for (const GNode* sn : srcs) {
            const GNode& r = only(sn->out.at(0), OP_RESHAPE, "head RESHAPE", *sn);
            const GTensor& rt = g.t(r.out.at(0));
            const auto& nx = consumers(r.out.at(0));
            const GNode* rope = nx.size() == 1 && nx[0]->opcode == OP_ROPE ? nx[0] : nullptr;
            const GNode& src = rope ? *rope : r;
            const GNode& pm = only(src.out.at(0), OP_PERMUTE, "attention PERMUTE", src);
            const GNode& fa = only(pm.out.at(0), OP_FLASH_ATTN_EXT, "FLASH_ATTN_EXT", pm);
            const auto it = std::find(fa.in.begin(), fa.in.end(), pm.out.at(0));
            paths.push_back({(int64_t)(it - fa.in.begin()), rt.ne[0].eval(one), rt.ne[1].eval(one), sn, rope, &fa});
        }
        std::sort(paths.begin(), paths.end(), [](const Path& a, const Path& b) { return a.slot < b.slot; });
        if (paths[0].slot != 0 || paths[1].slot != 1 || paths[2].slot != 2 || paths[0].fa != paths[1].fa ||
            paths[1].fa != paths[2].fa)
            unmapped(*srcs[0], "q, k, v must be the inputs 0, 1, 2 of one attention node");
        if (!paths[0].rope || !paths[1].rope || paths[2].rope) unmapped(*srcs[0], "rope must apply to q and k only");
        const int64_t hd = paths[0].hd, Hq = paths[0].H, Hkv = paths[1].H;
        if (paths[1].hd != hd || paths[2].hd != hd) unmapped(*srcs[0], "q, k, v head sizes differ");
        if (paths[2].H != Hkv) unmapped(*srcs[2], "k and v head counts differ");
        if (fused) {
            if (L.qkv.N != (Hq + 2 * Hkv) * hd || paths[0].src->attr_int("start", -1) != 0 ||
                paths[1].src->attr_int("start", -1) != Hq * hd || paths[2].src->attr_int("start", -1) != (Hq + Hkv) * hd)
                unmapped(*srcs[0], "fused QKV rows are not q | k | v");
            const std::string b = bias_of(*mms[0], L.qkv.N);
            if (!b.empty()) L.qkv.bias = {b};
        } else {  // three products, concatenated in q | k | v order (exact: whole rows)
            L.qkv = WeightRef();
            int nb = 0;
            for (const Path& pth : paths) {
                WeightRef w = weight(*pth.src);
                if (L.qkv.names.empty()) L.qkv.type = w.type, L.qkv.K = w.K;
                if (w.type != L.qkv.type || w.K != L.qkv.K) unmapped(*pth.src, "q/k/v weights of different types");
                L.qkv.names.push_back(w.names[0]);
                L.qkv.N += w.N;
                const std::string b = bias_of(*pth.src, w.N);
                if (!b.empty()) ++nb;
                L.qkv.bias.push_back(b);
            }
            if (nb == 0) L.qkv.bias.clear();
            else if (nb != 3) unmapped(*srcs[0], "biases on some of q, k, v only");
        }
        for (int k = 0; k < 2; ++k) {
            const GNode& rn = *paths[k].rope;
            if (rn.attr_int("mode", 2) != 2 || rn.attr_int("n_dims", hd) != hd)
                unmapped(rn, "only NEOX rope over the whole head is mapped");
            if (rn.attr_f("ext_factor", 0.0) != 0.0 || rn.attr_f("freq_scale", 1.0) != 1.0)
                unmapped(rn, "rope scaling is not mapped");
            bases.push_back((float)rn.attr_f("freq_base", 10000.0));
        }
        const GNode& fa = *paths[0].fa;
        const double scale = fa.attr_f("scale", 1.0 / std::sqrt((double)hd));
        if (std::fabs(scale - 1.0 / std::sqrt((double)hd)) > 1e-7 * scale || fa.attr_f("max_bias", 0.0) != 0.0 ||
            fa.attr_f("logit_softcap", 0.0) != 0.0)
            unmapped(fa, "attention scale must be 1/sqrt(head_dim), no ALiBi/softcap");
        if (!fa.attr_int("fused_transpose", 0)) unmapped(fa, "expected the fused-transpose attention output [hd, H, s]");
        const GNode& a2 = only(fa.out.at(0), OP_RESHAPE, "attention output RESHAPE", fa);
        const GNode& o = only(a2.out.at(0), OP_MUL_MAT, "output projection", a2);
        L.o = weight(o);
        if (std::string b = bias_of(o, L.o.N); !b.empty()) L.o.bias = {b};
        const GNode& add1 = only(o.out.at(0), OP_ADD, "residual ADD", o);
        if (std::find(add1.in.begin(), add1.in.end(), x) == add1.in.end()) unmapped(add1, "residual must add the layer input");
        const uint32_t x1 = add1.out.at(0);
        const GNode& norm2 = only(x1, OP_RMS_NORM, "ffn RMS_NORM", add1);
        eps.push_back(rms_eps(norm2));
        const GNode& gu = only(norm2.out.at(0), OP_MUL_MAT, "gate|up projection", norm2);
        L.gate_up = weight(gu);
        if (std::string b = bias_of(gu, L.gate_up.N); !b.empty()) L.gate_up.bias = {b};
        const GNode& glu = only(gu.out.at(0), OP_GLU, "GLU SWIGLU", gu);
        if (glu.attr_int("op", 2) != 2 || glu.attr_int("swapped", 0) != 0) unmapped(glu, "only SWIGLU is mapped");
        const GNode& dn = only(glu.out.at(0), OP_MUL_MAT, "down projection", glu);
        L.down = weight(dn);
        if (std::string b = bias_of(dn, L.down.N); !b.empty()) L.down.bias = {b};
        const GNode& add2 = only(dn.out.at(0), OP_ADD, "residual ADD", dn);
        if (std::find(add2.in.begin(), add2.in.end(), x1) == add2.in.end())
            unmapped(add2, "residual must add the attention block's output");
        if (m.layers.empty()) {
            m.hd = hd, m.n_head = Hq, m.n_head_kv = Hkv, m.n_ff = L.gate_up.N / 2;
        } else if (m.hd != hd || m.n_head != Hq || m.n_head_kv != Hkv || m.n_ff != L.gate_up.N / 2) {
            unmapped(norm, "layers differ in shape");
        }
        if (L.qkv.K != m.n_embd || L.o.K != Hq * hd || L.o.N != m.n_embd || L.gate_up.K != m.n_embd ||
            L.down.K != m.n_ff || L.down.N != m.n_embd)
            unmapped(norm, "projection shapes do not chain");
        m.layers.push_back(std::move(L));
        x = add2.out.at(0);
    }
    if (m.layers.empty()) raise(GQ_ERR_UNSUPPORTED, "no decoder layer found");
    for (float e : eps)
        if (e != eps[0]) raise(GQ_ERR_UNSUPPORTED, "layers differ in RMS_NORM eps");
    for (float b : bases)
        if (b != bases[0]) raise(GQ_ERR_UNSUPPORTED, "layers differ in rope base");
    m.rms_eps = eps[0];
    m.rope_base = bases[0];
    return m;
}

// --------------------------------------------------------------- descriptors
size_t elem_size(int type) {
    switch (type) {
        case GQ_TYPE_F32: case GQ_TYPE_I32: return 4;
        case GQ_TYPE_F16: return 2;
        case GQ_TYPE_I64: return 8;
        default: return 0;
    }
}

// a tensor with rows of ne0 elements, strides given in elements of the type (0: packed)
gq_tensor desc(const void* p, int type, int64_t ne0, int64_t ne1 = 1, int64_t ne2 = 1, int64_t s1 = 0,
               int64_t s2 = 0) {
    gq_tensor t{};
    t.data = const_cast<void*>(p);
    t.type = type;
    const size_t es = elem_size(type);
    t.ne[0] = ne0, t.ne[1] = ne1, t.ne[2] = ne2, t.ne[3] = 1;
    t.nb[0] = es;
    t.nb[1] = es * (size_t)(s1 ? s1 : ne0);
    t.nb[2] = es * (size_t)(s2 ? s2 : (s1 ? s1 : ne0) * ne1);
    t.nb[3] = t.nb[2] * (size_t)ne2;
    return t;
}

struct QW {  // a device-resident block-quantized weight
    void* data = nullptr;
    int type = 0;
    int64_t K = 0, N = 0;
    float* bias = nullptr;
    gq_tensor d() const {
        gq_tensor t{};
        const size_t bb = type == GQ_TYPE_Q8_0 ? Q8_BYTES : Q4_BYTES;
        t.data = data;
        t.type = type;
        t.ne[0] = K, t.ne[1] = N, t.ne[2] = 1, t.ne[3] = 1;
        t.nb[0] = bb, t.nb[1] = (size_t)(K / QK) * bb;
        t.nb[2] = t.nb[1] * (size_t)N, t.nb[3] = t.nb[2];
        return t;
    }
};

// the batched decode's attention launches are sized for max_len rounded up to this many rows
constexpr int64_t PAGED_BUCKET = 512;

int64_t pad_kv_len(int64_t n, int64_t max_ctx, int64_t n_pad) {  // executor.cpp:58-64
    n = std::max<int64_t>(n, 1);
    if (n_pad <= 1) return std::min(n, max_ctx);
    return std::min(std::max<int64_t>(n_pad, (n + n_pad - 1) / n_pad * n_pad), max_ctx);
}

// the graph's surface and the matched decoder as JSON (gq_exec_describe / gq_exec_inspect)
std::string describe_json(const Graph& graph, const Match& m, const std::string& device) {
    auto ids = [](const std::vector<uint32_t>& v) {
        std::string s = "[";
        for (size_t i = 0; i < v.size(); ++i) s += (i ? "," : "") + std::to_string(v[i]);
        return s + "]";
    };
    auto esc = [](const std::string& s) {
        std::string o = "\"";
        for (char c : s) {
            if (c == '"' || c == '\\') o += '\\';
            if ((unsigned char)c < 0x20) {
                char u[8];
                snprintf(u, sizeof(u), "\\u%04x", c);
                o += u;
            } else {
                o += c;
            }
        }
        return o + "\"";
    };
    std::string syms = "[";
    for (size_t i = 0; i < graph.symbols.size(); ++i) syms += (i ? "," : "") + esc(graph.symbols[i]);
    syms += "]";
    std::string names = "{";
    bool first = true;
    for (const auto* v : {&graph.inputs, &graph.outputs})
        for (uint32_t t : *v) {
            names += (first ? "" : ",") + esc(std::to_string(t)) + ":" + esc(graph.t(t).name);
            first = false;
        }
    names += "}";
    std::string layers = "[";
    for (size_t l = 0; l < m.layers.size(); ++l) {
        const auto& L = m.layers[l];
        auto w = [&](const WeightRef& r) {
            std::string s = "{\"names\":[";
            for (size_t i = 0; i < r.names.size(); ++i) s += (i ? "," : "") + esc(r.names[i]);
            s += "],\"bias\":[";
            for (size_t i = 0; i < r.bias.size(); ++i) s += (i ? "," : "") + esc(r.bias[i]);
            return s + "],\"type\":" + std::to_string(r.type) + ",\"K\":" + std::to_string(r.K) +
                   ",\"N\":" + std::to_string(r.N) + "}";
        };
        layers += std::string(l ? "," : "") + "{\"qkv\":" + w(L.qkv) + ",\"o\":" + w(L.o) +
                  ",\"gate_up\":" + w(L.gate_up) + ",\"down\":" + w(L.down) + "}";
    }
    layers += "]";
    char cfg[640];
    snprintf(cfg, sizeof(cfg),
             "{\"n_layer\":%zu,\"n_embd\":%lld,\"n_head\":%lld,\"n_head_kv\":%lld,\"head_dim\":%lld,"
             "\"n_ff\":%lld,\"n_vocab\":%lld,\"rms_eps\":%.9g,\"rope_base\":%.9g,\"tied\":%d,"
             "\"qkv_bias\":%d,\"embed_type\":%d,\"lm_type\":%d,\"input\":%u,\"output\":%u}",
             m.layers.size(), (long long)m.n_embd, (long long)m.n_head, (long long)m.n_head_kv, (long long)m.hd,
             (long long)m.n_ff, (long long)m.n_vocab, (double)m.rms_eps, (double)m.rope_base,
             m.lm_head == m.embed ? 1 : 0, m.layers.empty() || m.layers[0].qkv.bias.empty() ? 0 : 1, m.embed_type,
             m.lm_type, m.input_tid, m.output_tid);
    return "{\"name\":" + esc(graph.name) + ",\"device\":" + esc(device) + ",\"inputs\":" + ids(graph.inputs) +
           ",\"outputs\":" + ids(graph.outputs) + ",\"parameters\":" + ids(graph.parameters) +
           ",\"symbol_table\":" + syms + ",\"names\":" + names + ",\"embed\":" + esc(m.embed) +
           ",\"lm_head\":" + esc(m.lm_head) + ",\"layers\":" + layers + ",\"config\":" + cfg + "}";
}

}  // namespace

// -------------------------------------------------------------- the executor
struct Executor {
    int dev = 0;
    std::string device;
    hipStream_t stream = nullptr;
    Gguf file;
    Graph graph;
    Match m;
    std::vector<void*> allocs;          // every device allocation, freed with the handle
    std::vector<void*> retired_ws;      // workspaces replaced while graphs may hold them
    QW embed, lm_head;
    struct Layer {
        QW qkv, o, gate_up, down;
    };
    std::vector<Layer> layers;
    // KV cache: per layer K then V, each F16 [Hkv][max_ctx][hd]
    uint16_t* kv = nullptr;
    int64_t max_ctx = 0;
    bool kv_on = false;
    int32_t* pos_dev = nullptr;
    int32_t pos_host = 0;  // source of the position upload (outlives the async copy)
    void* ws = nullptr;
    size_t ws_bytes = 0;
    bool logits_last_only = false;
    bool use_graphs = true;
    // prepared step
    int64_t s = 0, pos = 0;
    bool prepared = false;
    std::vector<int32_t> ids_host;
    // per-s buffers
    struct Bufs {
        int32_t* ids;
        float *x, *x_alt, *h, *qkv, *q, *attn, *proj, *gu, *act, *logits;
        int32_t *next, *pos_ids;
        int64_t* kv_idx;
        float* rope_cs;
        uint16_t* mask;
        int64_t rows_cap;  // logits rows allocated
        int32_t* seq_len;       // paged decode: each row's rows to attend
        uint8_t *q8_o, *q8_d;   // int8 path: the o and down projections' quantized input rows
    };
    std::map<int64_t, Bufs> bufs;
    std::map<std::tuple<int64_t, int64_t, int64_t>, std::pair<hipGraphExec_t, int64_t>> graphs;  // and its node count
    std::vector<hipGraph_t> graph_defs;
    std::vector<float> out_host;  // the last run's logits, [rows][vocab]
    int64_t out_rows = 0;
    // the n_kv bucket pad: GGMLC_KV_PAD when init_kv_cache runs (executor.cpp:501-503), else 256
    int64_t kv_n_pad = 256;

    // -- paged KV (executor.cpp:634-920) -------------------------------------------------
    // Per layer one K and one V pool, F16 [Hkv][n_pages * P][hd]: page p is rows
    // [p P, (p + 1) P) of every layer's pools, so one page id names a token range in all
    // layers. Slot tables list each slot's pages (device I32 [max_batch][max_pages], -1:
    // none); page 0 takes the KV writes of batch rows whose slot has no page. Pages are
    // reference counted: a slot holds one reference per listed page, and callers that
    // keep pages beyond their slot (a prefix cache) take their own. A slot's prompt is
    // computed on the contiguous cache (the single-sequence step and its graphs), with
    // the slot's earlier rows copied in and the computed rows copied out to its pages;
    // a batched decode step runs every slot of [0, b) at its own position.
    struct Paged {
        bool on = false;
        int64_t P = 128, max_batch = 0, max_ctx = 0, max_pages = 0, n_pages = 0;
        uint16_t* pool = nullptr;
        int32_t* table = nullptr;
        std::vector<int32_t> table_host;
        std::vector<std::vector<int32_t>> pages;
        std::vector<char> active, dirty;
        std::vector<int32_t> refs;
        std::vector<int32_t> free_pages;  // popped from the back: lowest ids first
        int32_t* pos = nullptr;           // device: each slot's next position
        std::vector<int32_t> pos_host;
        int32_t* list = nullptr;          // device: one slot's page ids (row copies)
        std::vector<int32_t> list_host;
        int contig_slot = -1;             // the slot whose rows [0, contig_rows) the contiguous cache holds
        int64_t contig_rows = 0;
    } pg;
    int slot = -1;       // prepared paged step: >= 0 a prompt step of that slot, -1 a batched decode
    int64_t nb = 1;      // prepared paged step: batch rows (symbol b)
    bool paged_step = false;
    std::map<std::tuple<int64_t, int64_t>, std::pair<hipGraphExec_t, int64_t>> paged_graphs;  // (b, max_len)

    // -- profiling (set_enable_profile / get_profile / runtime_graph_summary /
    // runtime_mul_mat_shape_summary, executor.h:101-118) -----------------------------------
    bool profile_on = false;
    double prof_prepare_ms = 0.0, prof_run_ms = 0.0;
    int64_t prof_n_prepare = 0, prof_n_run = 0;
    std::map<std::string, int64_t> op_hist, mm_shapes, fa_shapes;  // launches of the last issued step
    int64_t last_nodes = -1;  // kernel nodes of the graph the last run replayed (-1: eager)
    void count(const std::string& op) { ++op_hist[op]; }

    int64_t E() const { return m.n_embd; }
    int64_t nq() const { return (m.n_head + 2 * m.n_head_kv) * m.hd; }
    int64_t qd() const { return m.n_head * m.hd; }

    void* dmalloc(size_t n) {
        void* p = nullptr;
        hip_ok(hipMalloc(&p, std::max<size_t>(n, 256)), "hipMalloc");
        allocs.push_back(p);
        return p;
    }
    void dfree(void* p) {
        if (!p) return;
        auto it = std::find(allocs.begin(), allocs.end(), p);
        if (it != allocs.end()) allocs.erase(it);
        (void)hipFree(p);
    }

    QW upload(const WeightRef& w) {
        QW q;
        q.type = w.type, q.K = w.K, q.N = w.N;
        size_t total = 0;
        for (const auto& n : w.names) total += file.tensor(n).nbytes;
        q.data = dmalloc(total);
        size_t off = 0;
        for (const auto& n : w.names) {
            const GgufTensor& t = file.tensor(n);
            hip_ok(hipMemcpy(static_cast<uint8_t*>(q.data) + off, file.data(t), t.nbytes, hipMemcpyHostToDevice),
                   "weight upload");
            off += t.nbytes;
        }
        if (!w.bias.empty()) {
            q.bias = static_cast<float*>(dmalloc((size_t)q.N * 4));
            size_t boff = 0;
            for (const auto& n : w.bias) {
                const GgufTensor& t = file.tensor(n);
                hip_ok(hipMemcpy(reinterpret_cast<uint8_t*>(q.bias) + boff, file.data(t), t.nbytes,
                                 hipMemcpyHostToDevice),
                       "bias upload");
                boff += t.nbytes;
            }
        }
        return q;
    }

    void load() {
        const auto it = file.strings.find("ggmlc.graph_spec");
        if (it == file.strings.end()) raise(GQ_ERR_INVALID, "GGUF metadata missing 'ggmlc.graph_spec'");
        graph = parse_graph(it->second);
        m = match_llama(graph, file);
        if (m.hd != 64 && m.hd != 128) raise(GQ_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
        embed = upload(WeightRef{{m.embed}, {}, m.embed_type, m.n_embd, m.n_vocab});
        lm_head = m.lm_head == m.embed ? embed : upload(WeightRef{{m.lm_head}, {}, m.lm_type, m.n_embd, m.n_vocab});
        for (const auto& L : m.layers) layers.push_back({upload(L.qkv), upload(L.o), upload(L.gate_up), upload(L.down)});
        pos_dev = static_cast<int32_t*>(dmalloc(4));
        hip_ok(hipMemsetAsync(pos_dev, 0, 4, stream), "hipMemsetAsync");
    }

    // -- KV cache (executor.cpp:498-620): F16 rows written at pos..pos+s-1 ----------------
    void init_kv(int64_t ctx) {
        if (ctx <= 0) raise(GQ_ERR_INVALID, "init_kv_cache: max_ctx must be positive");
        if (kv_on) return;
        if (const char* env = std::getenv("GGMLC_KV_PAD")) kv_n_pad = std::max<int64_t>(1, std::atoll(env));
        drop_graphs();
        const size_t bytes = 2 * layers.size() * (size_t)m.n_head_kv * ctx * m.hd * 2;
        kv = static_cast<uint16_t*>(dmalloc(bytes));
        hip_ok(hipMemsetAsync(kv, 0, bytes, stream), "hipMemsetAsync");
        max_ctx = ctx;
        kv_on = true;
        bufs_free();
    }
    void reset_kv() {
        if (!kv) return;
        hip_ok(hipMemsetAsync(kv, 0, 2 * layers.size() * (size_t)m.n_head_kv * max_ctx * m.hd * 2, stream),
               "hipMemsetAsync");
        hip_ok(hipMemsetAsync(pos_dev, 0, 4, stream), "hipMemsetAsync");
        hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
        pg.contig_slot = -1;  // the contiguous cache no longer holds a slot's rows
    }
    uint16_t* kc(size_t l) const { return kv + (2 * l) * (size_t)m.n_head_kv * max_ctx * m.hd; }
    uint16_t* vc(size_t l) const { return kv + (2 * l + 1) * (size_t)m.n_head_kv * max_ctx * m.hd; }
    size_t pool_elems() const { return (size_t)m.n_head_kv * pg.n_pages * pg.P * m.hd; }
    uint16_t* kp(size_t l) const { return pg.pool + (2 * l) * pool_elems(); }
    uint16_t* vp(size_t l) const { return pg.pool + (2 * l + 1) * pool_elems(); }

    void set_tokens_per_page(int64_t n) {
        if (pg.on) raise(GQ_ERR_INVALID, "set_tokens_per_page: the paged cache is already initialised");
        // the attention kernels take pages of a power of two >= 64 rows (>= 128 for 64-dim heads)
        if (n < 64 || (n & (n - 1)) || (m.hd == 64 && n < 128))
            raise(GQ_ERR_INVALID, "tokens_per_page must be a power of two >= 64 (>= 128 for head_dim 64)");
        pg.P = n;
    }

    void init_paged(int64_t max_batch, int64_t ctx) {
        if (pg.on) return;  // executor.cpp:635
        if (max_batch <= 0 || max_batch > 256) raise(GQ_ERR_INVALID, "init_paged_kv_cache: max_batch must be 1..256");
        if (ctx <= 0) raise(GQ_ERR_INVALID, "init_paged_kv_cache: max_ctx must be positive");
        if (kv_on && max_ctx < ctx)
            raise(GQ_ERR_INVALID, "init_paged_kv_cache: max_ctx above the contiguous cache's (" +
                                      std::to_string(max_ctx) + ")");
        if (!kv_on) init_kv(ctx);  // the prompt steps' contiguous cache
        Paged& p = pg;
        p.max_batch = max_batch, p.max_ctx = ctx;
        p.max_pages = (ctx + p.P - 1) / p.P;
        p.n_pages = max_batch * p.max_pages + 1;
        if ((int64_t)p.n_pages * p.P * m.hd * 2 >= ((int64_t)1 << 31))
            raise(GQ_ERR_UNSUPPORTED, "init_paged_kv_cache: one head of a pool must stay below 2 GiB");
        drop_graphs();
        p.pool = static_cast<uint16_t*>(dmalloc(2 * layers.size() * pool_elems() * 2));
        hip_ok(hipMemsetAsync(p.pool, 0, 2 * layers.size() * pool_elems() * 2, stream), "hipMemsetAsync");
        p.table = static_cast<int32_t*>(dmalloc((size_t)max_batch * p.max_pages * 4));
        hip_ok(hipMemsetAsync(p.table, 0xff, (size_t)max_batch * p.max_pages * 4, stream), "hipMemsetAsync");
        p.pos = static_cast<int32_t*>(dmalloc((size_t)max_batch * 4));
        hip_ok(hipMemsetAsync(p.pos, 0, (size_t)max_batch * 4, stream), "hipMemsetAsync");
        p.list = static_cast<int32_t*>(dmalloc((size_t)p.max_pages * 4));
        p.table_host.assign((size_t)max_batch * p.max_pages, -1);
        p.pages.assign((size_t)max_batch, {});
        p.active.assign((size_t)max_batch, 0);
        p.dirty.assign((size_t)max_batch, 0);
        p.pos_host.assign((size_t)max_batch, 0);
        p.list_host.assign((size_t)p.max_pages, -1);
        p.refs.assign((size_t)p.n_pages, 0);
        p.refs[0] = 1;  // the trash page is never handed out
        p.free_pages.clear();
        for (int64_t i = p.n_pages - 1; i >= 1; --i) p.free_pages.push_back((int32_t)i);
        hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
        p.on = true;
    }
    void need_paged() const {
        if (!pg.on) raise(GQ_ERR_INVALID, "init_paged_kv_cache first");
    }
    void check_slot(int64_t sl) const {
        need_paged();
        if (sl < 0 || sl >= pg.max_batch)
            raise(GQ_ERR_INVALID, "slot " + std::to_string(sl) + " outside [0, " + std::to_string(pg.max_batch) + ")");
    }
    void set_slot_pos(int64_t sl, int64_t p) {
        pg.pos_host[(size_t)sl] = (int32_t)p;
        hip_ok(hipMemcpyAsync(pg.pos + sl, &pg.pos_host[(size_t)sl], 4, hipMemcpyHostToDevice, stream), "pos upload");
        hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");  // the host value may change next
    }
    void set_row(int64_t sl) {
        int32_t* row = &pg.table_host[(size_t)sl * pg.max_pages];
        std::fill(row, row + pg.max_pages, -1);
        std::copy(pg.pages[(size_t)sl].begin(), pg.pages[(size_t)sl].end(), row);
        pg.dirty[(size_t)sl] = 1;
    }
    void sync_tables() {
        bool any = false;
        for (int64_t sl = 0; sl < pg.max_batch; ++sl) {
            if (!pg.dirty[(size_t)sl]) continue;
            hip_ok(hipMemcpyAsync(pg.table + sl * pg.max_pages, &pg.table_host[(size_t)sl * pg.max_pages],
                                  (size_t)pg.max_pages * 4, hipMemcpyHostToDevice, stream),
                   "page table upload");
            pg.dirty[(size_t)sl] = 0;
            any = true;
        }
        if (any) hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
    }
    void release_page(int32_t id) {
        if (id <= 0 || id >= pg.n_pages || pg.refs[(size_t)id] <= 0)
            raise(GQ_ERR_INVALID, "page " + std::to_string(id) + " is not in use");
        if (--pg.refs[(size_t)id] == 0) pg.free_pages.push_back(id);
    }
    void retain_page(int32_t id) {
        if (id <= 0 || id >= pg.n_pages || pg.refs[(size_t)id] <= 0)
            raise(GQ_ERR_INVALID, "page " + std::to_string(id) + " is not in use");
        ++pg.refs[(size_t)id];
    }
    void alloc_slot(int64_t sl) {  // executor.cpp:738-765
        check_slot(sl);
        if (pg.active[(size_t)sl]) free_slot(sl);
        pg.active[(size_t)sl] = 1;
        set_slot_pos(sl, 0);
    }
    void free_slot(int64_t sl) {  // executor.cpp:767-803
        check_slot(sl);
        for (int32_t id : pg.pages[(size_t)sl]) release_page(id);
        pg.pages[(size_t)sl].clear();
        pg.active[(size_t)sl] = 0;
        set_row(sl);
        if (pg.contig_slot == sl) pg.contig_slot = -1;
    }
    void ensure_tokens(int64_t sl, int64_t total) {  // executor.cpp:812-851
        check_slot(sl);
        if (!pg.active[(size_t)sl]) raise(GQ_ERR_INVALID, "slot " + std::to_string(sl) + " is not allocated");
        if (total < 0 || total > pg.max_ctx)
            raise(GQ_ERR_INVALID, std::to_string(total) + " tokens exceed the slots' max_ctx (" +
                                      std::to_string(pg.max_ctx) + ")");
        auto& pl = pg.pages[(size_t)sl];
        const size_t need = (size_t)((total + pg.P - 1) / pg.P);
        if (pl.size() >= need) return;
        if (pg.free_pages.size() < need - pl.size())
            raise(GQ_ERR_WORKSPACE, "the page pool has " + std::to_string(pg.free_pages.size()) + " free pages, " +
                                        std::to_string(need - pl.size()) + " needed");
        while (pl.size() < need) {
            const int32_t id = pg.free_pages.back();
            pg.free_pages.pop_back();
            pg.refs[(size_t)id] = 1;
            pl.push_back(id);
        }
        set_row(sl);
    }
    void map_pages(int64_t sl, int64_t start, const int32_t* ids, int64_t n) {  // executor.cpp:853-897
        check_slot(sl);
        if (!pg.active[(size_t)sl]) raise(GQ_ERR_INVALID, "slot " + std::to_string(sl) + " is not allocated");
        auto& pl = pg.pages[(size_t)sl];
        if (start != (int64_t)pl.size()) raise(GQ_ERR_INVALID, "shared pages must continue the slot's page list");
        if (n < 0 || (n && !ids) || (int64_t)pl.size() + n > pg.max_pages)
            raise(GQ_ERR_INVALID, "map_existing_pages: bad page list");
        for (int64_t i = 0; i < n; ++i) retain_page(ids[i]);  // validates every id first
        for (int64_t i = 0; i < n; ++i) pl.push_back(ids[i]);
        set_row(sl);
        if (pg.contig_slot == sl) pg.contig_slot = -1;
    }
    int32_t page_of(int64_t sl, int64_t idx) const {  // executor.cpp:899-920
        check_slot(sl);
        const auto& pl = pg.pages[(size_t)sl];
        if (idx < 0 || idx >= (int64_t)pl.size())
            raise(GQ_ERR_INVALID, "slot " + std::to_string(sl) + " has no page " + std::to_string(idx));
        return pl[(size_t)idx];
    }
    size_t active_bytes() const {
        if (!pg.on) return 0;
        int64_t used = 0;
        for (int64_t i = 1; i < pg.n_pages; ++i) used += pg.refs[(size_t)i] > 0;
        return (size_t)used * 2 * layers.size() * m.n_head_kv * pg.P * m.hd * 2;
    }
    // rows [r0, r1) of slot sl between its pages and the contiguous cache, every layer
    void copy_rows(int64_t sl, int64_t r0, int64_t r1, int to_pool) {
        if (r1 <= r0) return;
        const auto& pl = pg.pages[(size_t)sl];
        std::fill(pg.list_host.begin(), pg.list_host.end(), -1);
        std::copy(pl.begin(), pl.end(), pg.list_host.begin());
        hip_ok(hipMemcpyAsync(pg.list, pg.list_host.data(), (size_t)pg.max_pages * 4, hipMemcpyHostToDevice, stream),
               "page list upload");
        const int64_t rows = pg.n_pages * pg.P, hd = m.hd, Hkv = m.n_head_kv;
        for (size_t l = 0; l < layers.size(); ++l) {
            for (int kvi = 0; kvi < 2; ++kvi) {
                gq_tensor pool = desc(kvi ? vp(l) : kp(l), GQ_TYPE_F16, hd, rows, Hkv);
                gq_tensor cache = desc(kvi ? vc(l) : kc(l), GQ_TYPE_F16, hd, max_ctx, Hkv);
                gq_ok(gq_kv_pages_copy(&pool, &cache, pg.list, (int64_t)pl.size(), pg.P, r0, r1, to_pool, stream));
            }
        }
        hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");  // the page list may change next
    }

    void drop_graphs() {
        for (auto& kvp : graphs) (void)hipGraphExecDestroy(kvp.second.first);
        graphs.clear();
        for (auto& kvp : paged_graphs) (void)hipGraphExecDestroy(kvp.second.first);
        paged_graphs.clear();
        for (hipGraph_t g : graph_defs) (void)hipGraphDestroy(g);
        graph_defs.clear();
    }
    void bufs_free() {
        drop_graphs();
        for (auto& kvp : bufs) {
            Bufs& b = kvp.second;
            for (void* p : {(void*)b.ids, (void*)b.x, (void*)b.x_alt, (void*)b.h, (void*)b.qkv, (void*)b.q,
                            (void*)b.attn, (void*)b.proj, (void*)b.gu, (void*)b.act, (void*)b.logits, (void*)b.next,
                            (void*)b.pos_ids, (void*)b.kv_idx, (void*)b.rope_cs, (void*)b.mask, (void*)b.seq_len,
                            (void*)b.q8_o, (void*)b.q8_d})
                dfree(p);
        }
        bufs.clear();
    }

    Bufs& buffers(int64_t n) {
        auto it = bufs.find(n);
        if (it != bufs.end()) return it->second;
        Bufs b{};
        const int64_t e = E(), F = m.n_ff;
        b.ids = static_cast<int32_t*>(dmalloc((size_t)n * 4));
        b.x = static_cast<float*>(dmalloc((size_t)n * e * 4));
        b.x_alt = static_cast<float*>(dmalloc((size_t)n * e * 4));
        b.h = static_cast<float*>(dmalloc((size_t)n * e * 4));
        b.qkv = static_cast<float*>(dmalloc((size_t)n * nq() * 4));
        b.q = static_cast<float*>(dmalloc((size_t)n * qd() * 4));
        b.attn = static_cast<float*>(dmalloc((size_t)n * qd() * 4));
        b.proj = static_cast<float*>(dmalloc((size_t)2 * n * e * 4));  // room for a product's two halves of K
        b.gu = static_cast<float*>(dmalloc((size_t)n * 2 * F * 4));
        b.act = static_cast<float*>(dmalloc((size_t)n * F * 4));
        b.logits = static_cast<float*>(dmalloc((size_t)n * m.n_vocab * 4));
        b.rows_cap = n;
        b.next = static_cast<int32_t*>(dmalloc(4));
        b.pos_ids = static_cast<int32_t*>(dmalloc((size_t)n * 4));
        b.kv_idx = static_cast<int64_t*>(dmalloc((size_t)n * 8));
        b.rope_cs = static_cast<float*>(dmalloc((size_t)n * m.hd * 4));
        b.mask = static_cast<uint16_t*>(dmalloc((size_t)n * max_ctx * 2));
        b.seq_len = static_cast<int32_t*>(dmalloc((size_t)n * 4));
        b.q8_o = static_cast<uint8_t*>(dmalloc(gq_q8_rows_bytes(qd())));
        b.q8_d = static_cast<uint8_t*>(dmalloc(gq_q8_rows_bytes(m.n_ff)));
        return bufs.emplace(n, b).first->second;
    }

    // the largest workspace any op of an n-row step asks for (attention's plan is not
    // monotonic in n_kv: every bucket is checked), grown outside capture; a replaced
    // buffer stays allocated because graphs captured before may still use it
    void size_workspace(int64_t n, int64_t rows) {
        size_t need = 0;
        auto mm = [&](const QW& w, int64_t M) {
            gq_tensor a = w.d();
            gq_tensor b = desc(nullptr, GQ_TYPE_F32, w.K, M);
            gq_mul_mat_fusion f{};
            need = std::max(need, gq_mul_mat_fused_workspace_size(&a, &b, &f));
            gq_tensor b2 = desc(nullptr, GQ_TYPE_F32, 2 * w.K, M);  // the down projection's SWIGLU input
            f.b_swiglu = 1;
            need = std::max(need, gq_mul_mat_fused_workspace_size(&a, &b2, &f));
        };
        const Layer& L = layers[0];
        for (const QW* w : {&L.qkv, &L.o, &L.gate_up, &L.down}) mm(*w, n);
        mm(lm_head, rows);
        const int64_t step = std::max<int64_t>(kv_n_pad, 1);
        for (int64_t nk = step; nk < max_ctx + step; nk += step) {  // every n_kv bucket
            const int64_t nkv = std::min(nk, max_ctx);
            gq_tensor q = desc(nullptr, GQ_TYPE_F32, m.hd, n, m.n_head);
            gq_tensor k = desc(nullptr, GQ_TYPE_F16, m.hd, nkv, m.n_head_kv);
            need = std::max(need, gq_flash_attn_ext_workspace_size(&q, &k));
        }
        if (pg.on && n <= pg.max_batch) {  // the batched decode's paged attention
            for (int64_t ml = PAGED_BUCKET; ml < pg.max_ctx + PAGED_BUCKET; ml += PAGED_BUCKET) {
                gq_tensor q = desc(nullptr, GQ_TYPE_F32, m.hd, n, m.n_head, m.n_head * m.hd, m.hd);
                gq_tensor k = desc(nullptr, GQ_TYPE_F16, m.hd, pg.n_pages * pg.P, m.n_head_kv);
                need = std::max(need, gq_flash_attn_paged_workspace_size(&q, &k, std::min(ml, pg.max_ctx), pg.P));
            }
        }
        if (need <= ws_bytes) return;
        if (ws) retired_ws.push_back(ws);
        ws_bytes = std::max<size_t>(need, (size_t)1 << 20);
        ws = dmalloc(ws_bytes);
    }

    // -- one step: embedding -> layers -> RMS_NORM -> head on rows [r0, n) -> argmax ----
    void mm_fused(const QW& w, const float* x, int64_t xK, int64_t rows, float* dst, int64_t dN,
                  gq_mul_mat_fusion& f) {
        std::string op = "MUL_MAT";
        if (f.b_add) op = "ADD+" + op;
        if (f.rms_norm) op = "RMS_NORM+" + op;
        if (f.b_swiglu) op = "SWIGLU+" + op;
        if (f.b_q8) op = "Q8_ROWS+" + op;
        if (f.rope_kv) op += "+ROPE+SET_ROWS";
        if (f.swiglu) op += "+SWIGLU";
        if (f.out_q8) op += "+Q8_ROWS";
        if (w.bias) op += "+ADD(bias)";
        if (f.out_halves) op += "(K halves)";
        count(op);
        ++mm_shapes[std::string(w.type == GQ_TYPE_Q8_0 ? "q8_0" : "q4_0") + " K=" + std::to_string(w.K) + " N=" +
                    std::to_string(w.N) + " M=" + std::to_string(rows) + (f.int8 ? " int8" : "")];
        gq_tensor a = w.d();
        gq_tensor b = desc(x, GQ_TYPE_F32, xK, rows);
        gq_tensor d = desc(dst, GQ_TYPE_F32, dN, rows, f.out_halves ? 2 : 1);
        gq_tensor bias = desc(w.bias, GQ_TYPE_F32, w.N);
        if (w.bias) f.bias = &bias;
        f.workspace = ws;
        f.workspace_bytes = ws_bytes;
        gq_ok(gq_mul_mat_fused(&a, &b, dst ? &d : nullptr, &f, stream));
    }

    // whether the int8 path takes the plain product w x in two halves of K, so that its
    // output may stay two slabs for the next prologue's ADD (gq_mul_mat_fused_halves)
    bool mm_halves(const QW& w, const float* x, int64_t xK, int64_t rows) {
        gq_tensor a = w.d();
        gq_tensor b = desc(x, GQ_TYPE_F32, xK, rows);
        gq_tensor bias = desc(w.bias, GQ_TYPE_F32, w.N);
        gq_mul_mat_fusion f{};
        f.int8 = 1;
        if (w.bias) f.bias = &bias;
        const int rc = gq_mul_mat_fused_halves(&a, &b, &f);
        gq_ok(rc < 0 ? rc : GQ_OK);
        return rc == 1;
    }

    void forward(int64_t n, int64_t n_kv, int64_t r0) {
        Bufs& b = buffers(n);
        op_hist.clear(), mm_shapes.clear(), fa_shapes.clear();
        const bool fused = n <= 4;  // one GEMV launch per projection with its graph neighbours
        const int64_t e = E(), hd = m.hd, Hq = m.n_head, Hkv = m.n_head_kv, F = m.n_ff, QD = qd(), NQ = nq();
        {
            gq_tensor mk = desc(b.mask, GQ_TYPE_F16, n_kv, n, 1, max_ctx);
            gq_ok(gq_kv_step_inputs(pos_dev, n, b.pos_ids, b.kv_idx, &mk, stream));
            count("KV_STEP_INPUTS");
        }
        gq_tensor pos_t = desc(b.pos_ids, GQ_TYPE_I32, n);
        gq_tensor idx_t = desc(b.kv_idx, GQ_TYPE_I64, n);
        gq_tensor rcs = desc(b.rope_cs, GQ_TYPE_F32, hd, n);
        if (fused) gq_ok(gq_rope_cache(&pos_t, (int)hd, m.rope_base, 1.0f, 1.0f, &rcs, stream)), count("ROPE_CACHE");
        {
            gq_tensor tab = embed.d();
            gq_tensor ids = desc(b.ids, GQ_TYPE_I32, n);
            gq_tensor xo = desc(b.x, GQ_TYPE_F32, e, n);
            gq_ok(gq_get_rows(&tab, &ids, &xo, stream));
            count("GET_ROWS");
        }
        float* x = b.x;
        auto other = [&](float* p) { return p == b.x ? b.x_alt : b.x; };
        float* pending = nullptr;  // a projection still to be added to x (by the next prologue)
        const float scale = 1.0f / std::sqrt((float)hd);
        for (size_t l = 0; l < layers.size(); ++l) {
            const Layer& L = layers[l];
            gq_tensor kcache = desc(kc(l), GQ_TYPE_F16, hd, max_ctx, Hkv);
            gq_tensor vcache = desc(vc(l), GQ_TYPE_F16, hd, max_ctx, Hkv);
            gq_tensor pend = desc(pending, GQ_TYPE_F32, e, n);
            float* nx = pending ? other(x) : nullptr;
            gq_tensor nxt = desc(nx, GQ_TYPE_F32, e, n);
            gq_mul_mat_fusion f{};
            f.rms_norm = 1, f.rms_eps = m.rms_eps;
            if (pending) f.b_add = &pend, f.b_sum = &nxt;
            gq_tensor qo = desc(b.q, GQ_TYPE_F32, hd, Hq, n);
            if (fused) {  // ADD + RMS_NORM + QKV (+ bias) + ROPE x2 + SET_ROWS x2 in one launch
                gq_rope_kv_epilogue ep{};
                ep.n_head = (int32_t)Hq, ep.n_head_kv = (int32_t)Hkv, ep.head_dim = (int32_t)hd;
                ep.pos = &pos_t, ep.n_dims = (int32_t)hd, ep.mode = 2;
                ep.freq_base = m.rope_base, ep.freq_scale = 1.0f, ep.attn_factor = 1.0f;
                ep.kv_idx = &idx_t, ep.q_out = &qo, ep.k_cache = &kcache, ep.v_cache = &vcache;
                ep.rope_cache = &rcs;
                f.rope_kv = &ep;
                mm_fused(L.qkv, x, e, n, nullptr, NQ, f);
            } else {  // ADD + RMS_NORM in the QKV GEMM's prologue, then ROPE + SET_ROWS in one launch
                mm_fused(L.qkv, x, e, n, b.qkv, NQ, f);
                gq_tensor qv = desc(b.qkv, GQ_TYPE_F32, hd, Hq, n, hd, NQ);
                gq_tensor kv_ = desc(b.qkv + QD, GQ_TYPE_F32, hd, Hkv, n, hd, NQ);
                gq_tensor vv = desc(b.qkv + QD + Hkv * hd, GQ_TYPE_F32, hd, Hkv, n, hd, NQ);
                gq_ok(gq_rope_kv_store(&qv, &kv_, &vv, &pos_t, (int)hd, 2, m.rope_base, 1.0f, 1.0f, &idx_t, &qo,
                                       &kcache, &vcache, nullptr, stream));
                count("ROPE+SET_ROWS");
            }
            if (nx) x = nx;
            {  // FLASH_ATTN_EXT over the padded view [0, n_kv) of the cache
                count("FLASH_ATTN_EXT");
                ++fa_shapes["D=" + std::to_string(hd) + " Hq=" + std::to_string(Hq) + " Hkv=" + std::to_string(Hkv) +
                            " S=" + std::to_string(n) + " n_kv=" + std::to_string(n_kv)];
                gq_tensor q = desc(b.q, GQ_TYPE_F32, hd, n, Hq, Hq * hd, hd);
                gq_tensor kview = desc(kc(l), GQ_TYPE_F16, hd, n_kv, Hkv, hd, max_ctx * hd);
                gq_tensor vview = desc(vc(l), GQ_TYPE_F16, hd, n_kv, Hkv, hd, max_ctx * hd);
                gq_tensor mk = desc(b.mask, GQ_TYPE_F16, n_kv, n, 1, max_ctx);
                gq_tensor out = desc(b.attn, GQ_TYPE_F32, hd, Hq, n);
                gq_ok(gq_flash_attn_ext(&q, &kview, &vview, &mk, scale, 0.0f, 0.0f, &out, ws, ws_bytes, stream));
            }
            float* x2 = other(x);
            gq_tensor o_t = desc(b.proj, GQ_TYPE_F32, e, n);
            gq_tensor x2_t = desc(x2, GQ_TYPE_F32, e, n);
            {
                gq_mul_mat_fusion fo{};
                mm_fused(L.o, b.attn, QD, n, b.proj, e, fo);
            }
            if (fused) {  // ADD + RMS_NORM + gate|up (+ bias) + SWIGLU, then down
                gq_mul_mat_fusion fg{};
                fg.rms_norm = 1, fg.rms_eps = m.rms_eps, fg.swiglu = 1, fg.b_add = &o_t, fg.b_sum = &x2_t;
                mm_fused(L.gate_up, x, e, n, b.act, F, fg);
                x = x2;
                gq_mul_mat_fusion fd{};
                mm_fused(L.down, b.act, F, n, b.proj, e, fd);
            } else {  // ADD + RMS_NORM before gate_up, SWIGLU before down, in the GEMM prologues
                gq_mul_mat_fusion fg{};
                fg.rms_norm = 1, fg.rms_eps = m.rms_eps, fg.b_add = &o_t, fg.b_sum = &x2_t;
                mm_fused(L.gate_up, x, e, n, b.gu, 2 * F, fg);
                x = x2;
                gq_mul_mat_fusion fd{};
                fd.b_swiglu = 1;
                mm_fused(L.down, b.gu, 2 * F, n, b.proj, e, fd);
            }
            pending = b.proj;
        }
        // the head over rows [r0, n): residual ADD + RMS_NORM in its prologue
        const int64_t rows = n - r0;
        gq_tensor pend = desc(pending + r0 * e, GQ_TYPE_F32, e, rows);
        gq_mul_mat_fusion fh{};
        fh.rms_norm = 1, fh.rms_eps = m.rms_eps, fh.b_add = &pend;
        mm_fused(lm_head, x + r0 * e, e, rows, b.logits, m.n_vocab, fh);
        gq_tensor last = desc(b.logits + (rows - 1) * m.n_vocab, GQ_TYPE_F32, m.n_vocab, 1);
        gq_tensor nt = desc(b.next, GQ_TYPE_I32, 1);
        gq_ok(gq_argmax(&last, &nt, stream));
        gq_ok(gq_kv_advance(pos_dev, n, stream));
        count("ARGMAX"), count("KV_ADVANCE");
    }

    // whether every product of a layer takes the int8 path with the quantized-row handoffs
    // (model.q8_chain_ok): K % 256 == 0, 16-byte aligned weights, gate|up rows % 64, QKV
    // rows % 16, a power-of-two head_dim >= 16
    bool q8_chain_ok() const {
        if (m.hd < 16 || (m.hd & (m.hd - 1))) return false;
        for (const Layer& L : layers) {
            for (const QW* w : {&L.qkv, &L.o, &L.gate_up, &L.down})
                if (w->K % 256 || reinterpret_cast<uintptr_t>(w->data) % 16) return false;
            if (L.gate_up.N % 64 || L.qkv.N % 16) return false;
        }
        return true;
    }

    // One decode token for slots [0, B) over the paged pools (paged.BatchDecoder.step):
    // row i runs the token ids[i] at position pg.pos[i], writes its K/V row into slot i's
    // pages (page 0 when the slot has none) and attends to its rows [0, pos[i]]; every
    // position then advances by one. 2..16 rows take the int8 chain where it applies (ROPE
    // + SET_ROWS and SWIGLU in the products' epilogues, the split merge writing the o
    // projection's quantized rows); up to 4 rows otherwise the fused GEMVs; the logits of
    // every row.
    void forward_paged(int64_t B, int64_t max_len) {
        Bufs& b = buffers(B);
        op_hist.clear(), mm_shapes.clear(), fa_shapes.clear();
        const int64_t e = E(), hd = m.hd, Hq = m.n_head, Hkv = m.n_head_kv, F = m.n_ff, QD = qd(), NQ = nq();
        const int64_t rows = pg.n_pages * pg.P;
        const bool q8 = B > 1 && B <= 16 && q8_chain_ok() && Hq % Hkv == 0 && Hq / Hkv > 1 && Hq / Hkv <= 16 &&
                        pg.P % 128 == 0 && max_len > 128;
        const bool fused = !q8 && B <= 4;
        gq_tensor tab_t = desc(pg.table, GQ_TYPE_I32, pg.max_pages, B);
        gq_ok(gq_paged_step_inputs(pg.pos, B, &tab_t, pg.P, 0, b.kv_idx, b.seq_len, stream));
        count("PAGED_STEP_INPUTS");
        gq_tensor pos_t = desc(pg.pos, GQ_TYPE_I32, B);
        gq_tensor idx_t = desc(b.kv_idx, GQ_TYPE_I64, B);
        gq_tensor len_t = desc(b.seq_len, GQ_TYPE_I32, B);
        gq_tensor rcs = desc(b.rope_cs, GQ_TYPE_F32, hd, B);
        if (fused || q8) gq_ok(gq_rope_cache(&pos_t, (int)hd, m.rope_base, 1.0f, 1.0f, &rcs, stream)), count("ROPE_CACHE");
        {
            gq_tensor tab = embed.d();
            gq_tensor ids = desc(b.ids, GQ_TYPE_I32, B);
            gq_tensor xo = desc(b.x, GQ_TYPE_F32, e, B);
            gq_ok(gq_get_rows(&tab, &ids, &xo, stream));
            count("GET_ROWS");
        }
        float* x = b.x;
        auto other = [&](float* p) { return p == b.x ? b.x_alt : b.x; };
        float* pending = nullptr;
        bool pend_halves = false;  // pending holds a product's two halves of K (2 slabs of B rows)
        const float scale = 1.0f / std::sqrt((float)hd);
        for (size_t l = 0; l < layers.size(); ++l) {
            const Layer& L = layers[l];
            gq_tensor kpool = desc(kp(l), GQ_TYPE_F16, hd, rows, Hkv);
            gq_tensor vpool = desc(vp(l), GQ_TYPE_F16, hd, rows, Hkv);
            gq_tensor pend = desc(pending, GQ_TYPE_F32, e, B, pend_halves ? 2 : 1);
            float* nx = pending ? other(x) : nullptr;
            gq_tensor nxt = desc(nx, GQ_TYPE_F32, e, B);
            gq_mul_mat_fusion f{};
            f.rms_norm = 1, f.rms_eps = m.rms_eps;
            if (pending) f.b_add = &pend, f.b_sum = &nxt, f.b_add_halves = pend_halves ? 1 : 0;
            gq_tensor qo = desc(b.q, GQ_TYPE_F32, hd, Hq, B);
            if (fused || q8) {  // ADD + RMS_NORM + QKV (+ bias) + ROPE x2 + SET_ROWS x2
                gq_rope_kv_epilogue ep{};
                ep.n_head = (int32_t)Hq, ep.n_head_kv = (int32_t)Hkv, ep.head_dim = (int32_t)hd;
                ep.pos = &pos_t, ep.n_dims = (int32_t)hd, ep.mode = 2;
                ep.freq_base = m.rope_base, ep.freq_scale = 1.0f, ep.attn_factor = 1.0f;
                ep.kv_idx = &idx_t, ep.q_out = &qo, ep.k_cache = &kpool, ep.v_cache = &vpool;
                ep.rope_cache = &rcs;
                f.rope_kv = &ep;
                f.int8 = q8 ? 1 : 0;
                mm_fused(L.qkv, x, e, B, nullptr, NQ, f);
            } else {  // ADD + RMS_NORM in the QKV GEMM's prologue, then ROPE + SET_ROWS in one launch
                mm_fused(L.qkv, x, e, B, b.qkv, NQ, f);
                gq_tensor qv = desc(b.qkv, GQ_TYPE_F32, hd, Hq, B, hd, NQ);
                gq_tensor kv_ = desc(b.qkv + QD, GQ_TYPE_F32, hd, Hkv, B, hd, NQ);
                gq_tensor vv = desc(b.qkv + QD + Hkv * hd, GQ_TYPE_F32, hd, Hkv, B, hd, NQ);
                gq_ok(gq_rope_kv_store(&qv, &kv_, &vv, &pos_t, (int)hd, 2, m.rope_base, 1.0f, 1.0f, &idx_t, &qo,
                                       &kpool, &vpool, nullptr, stream));
                count("ROPE+SET_ROWS");
            }
            if (nx) x = nx;
            {  // every row over its own slot's rows
                gq_tensor q = desc(b.q, GQ_TYPE_F32, hd, B, Hq, Hq * hd, hd);
                gq_tensor out = desc(b.attn, GQ_TYPE_F32, hd, Hq, B);
                if (q8)
                    gq_ok(gq_flash_attn_paged_q8(&q, &kpool, &vpool, &tab_t, &len_t, pg.P, max_len, scale, &out,
                                                 b.q8_o, ws, ws_bytes, stream));
                else
                    gq_ok(gq_flash_attn_paged(&q, &kpool, &vpool, &tab_t, &len_t, pg.P, max_len, scale, &out, ws,
                                              ws_bytes, stream));
                count(q8 ? "FLASH_ATTN_PAGED+Q8_ROWS" : "FLASH_ATTN_PAGED");
                ++fa_shapes["paged D=" + std::to_string(hd) + " Hq=" + std::to_string(Hq) + " Hkv=" +
                            std::to_string(Hkv) + " B=" + std::to_string(B) + " max_len=" + std::to_string(max_len)];
            }
            float* x2 = other(x);
            // int8 path: o and down in two halves of K where it splits them (narrow products),
            // their slabs added by the next prologue's ADD
            const bool o_halves = q8 && mm_halves(L.o, b.attn, QD, B);
            gq_tensor o_t = desc(b.proj, GQ_TYPE_F32, e, B, o_halves ? 2 : 1);
            gq_tensor x2_t = desc(x2, GQ_TYPE_F32, e, B);
            {
                gq_mul_mat_fusion fo{};
                if (q8) fo.b_q8 = b.q8_o, fo.int8 = 1, fo.out_halves = o_halves ? 1 : 0;
                mm_fused(L.o, b.attn, QD, B, b.proj, e, fo);
            }
            pend_halves = false;
            if (q8) {  // ADD + RMS_NORM + gate|up + SWIGLU writing down's quantized rows, then down
                gq_mul_mat_fusion fg{};
                fg.rms_norm = 1, fg.rms_eps = m.rms_eps, fg.swiglu = 1, fg.b_add = &o_t, fg.b_sum = &x2_t;
                fg.b_add_halves = o_halves ? 1 : 0;
                fg.out_q8 = b.q8_d, fg.int8 = 1;
                mm_fused(L.gate_up, x, e, B, nullptr, F, fg);
                x = x2;
                pend_halves = mm_halves(L.down, b.act, F, B);
                gq_mul_mat_fusion fd{};
                fd.b_q8 = b.q8_d, fd.int8 = 1, fd.out_halves = pend_halves ? 1 : 0;
                mm_fused(L.down, b.act, F, B, b.proj, e, fd);
            } else if (fused) {
                gq_mul_mat_fusion fg{};
                fg.rms_norm = 1, fg.rms_eps = m.rms_eps, fg.swiglu = 1, fg.b_add = &o_t, fg.b_sum = &x2_t;
                mm_fused(L.gate_up, x, e, B, b.act, F, fg);
                x = x2;
                gq_mul_mat_fusion fd{};
                mm_fused(L.down, b.act, F, B, b.proj, e, fd);
            } else {
                gq_mul_mat_fusion fg{};
                fg.rms_norm = 1, fg.rms_eps = m.rms_eps, fg.b_add = &o_t, fg.b_sum = &x2_t;
                mm_fused(L.gate_up, x, e, B, b.gu, 2 * F, fg);
                x = x2;
                gq_mul_mat_fusion fd{};
                fd.b_swiglu = 1;
                mm_fused(L.down, b.gu, 2 * F, B, b.proj, e, fd);
            }
            pending = b.proj;
        }
        gq_mul_mat_fusion fh{};
        fh.rms_norm = 1, fh.rms_eps = m.rms_eps;
        fh.int8 = q8 && lm_head.K % 256 == 0 && reinterpret_cast<uintptr_t>(lm_head.data) % 16 == 0 ? 1 : 0;
        if (pend_halves && !fh.int8 && B <= 4) {  // the GEMV path adds one tensor: the halves' sum first
            gq_tensor h0 = desc(pending, GQ_TYPE_F32, e, B), h1 = desc(pending + B * e, GQ_TYPE_F32, e, B);
            gq_ok(gq_add(&h0, &h1, &h0, stream));
            count("ADD");
            pend_halves = false;
        }
        gq_tensor pend = desc(pending, GQ_TYPE_F32, e, B, pend_halves ? 2 : 1);
        fh.b_add = &pend, fh.b_add_halves = pend_halves ? 1 : 0;
        mm_fused(lm_head, x, e, B, b.logits, m.n_vocab, fh);
        gq_ok(gq_paged_advance(pg.pos, nullptr, B, stream));
        count("PAGED_ADVANCE");
    }

    // a step's graph: replayed when its bucket has one; otherwise issued eagerly (which also
    // fills the kernels' per-shape attribute and occupancy caches) and, with graphs on,
    // captured afterwards without executing, for the bucket's next run
    template <typename Map, typename Key, typename Fwd>
    void launch_step(Map& cache, const Key& key, bool graphs_ok, Fwd fwd) {
        auto it = cache.find(key);
        if (graphs_ok && it != cache.end()) {
            hip_ok(hipGraphLaunch(it->second.first, stream), "hipGraphLaunch");
            last_nodes = it->second.second;
            return;
        }
        fwd();
        last_nodes = -1;
        if (!graphs_ok) return;
        hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
        hipGraph_t g = nullptr;
        hip_ok(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            fwd();
        } catch (...) {
            (void)hipStreamEndCapture(stream, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        hip_ok(hipStreamEndCapture(stream, &g), "hipStreamEndCapture");
        hipGraphExec_t ge = nullptr;
        const hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
        if (ie != hipSuccess) {
            (void)hipGraphDestroy(g);
            hip_ok(ie, "hipGraphInstantiate");
        }
        size_t nodes = 0;
        (void)hipGraphGetNodes(g, nullptr, &nodes);
        graph_defs.push_back(g);
        cache.emplace(key, std::make_pair(ge, (int64_t)nodes));
    }

    void check_ids(int64_t n) const {
        if ((int64_t)ids_host.size() != n) raise(GQ_ERR_INVALID, "run: input ids not set");
        for (int32_t id : ids_host)
            if (id < 0 || id >= m.n_vocab) raise(GQ_ERR_INVALID, "token id " + std::to_string(id) + " outside the vocabulary");
    }

    // s tokens at position p on the contiguous cache; the logits to the host
    void step_contig(int64_t p, int64_t n, bool scratch) {
        const int64_t n_kv = pad_kv_len(p + n, max_ctx, kv_n_pad);
        const int64_t r0 = logits_last_only ? n - 1 : 0;
        Bufs& b = buffers(n);
        size_workspace(n, n - r0);
        hip_ok(hipMemcpyAsync(b.ids, ids_host.data(), (size_t)n * 4, hipMemcpyHostToDevice, stream), "ids upload");
        pos_host = (int32_t)p;
        hip_ok(hipMemcpyAsync(pos_dev, &pos_host, 4, hipMemcpyHostToDevice, stream), "pos upload");
        launch_step(graphs, std::make_tuple(n, n_kv, r0), use_graphs && !scratch, [&] { forward(n, n_kv, r0); });
        out_rows = n - r0;
        out_host.resize((size_t)out_rows * m.n_vocab);
        hip_ok(hipMemcpyAsync(out_host.data(), b.logits, out_host.size() * 4, hipMemcpyDeviceToHost, stream),
               "logits download");
        hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
    }

    void run() {
        if (!prepared) raise(GQ_ERR_INVALID, "run: call prepare first");
        if (paged_step) return slot >= 0 ? run_prompt_slot() : run_batch();
        check_ids(s);
        bool scratch = false;
        if (!kv_on) {  // no persistent cache: the whole sequence from position 0 in a scratch cache
            if (pos != 0) raise(GQ_ERR_INVALID, "run: pos > 0 needs init_kv_cache");
            init_kv(pad_kv_len(s, INT64_MAX, kv_n_pad));
            scratch = true;
        }
        if (pos + s > max_ctx)
            raise(GQ_ERR_INVALID, "pos + s = " + std::to_string(pos + s) + " exceeds the KV cache (" +
                                      std::to_string(max_ctx) + ")");
        step_contig(pos, s, scratch);
        pos += s;
        if (pg.on) pg.contig_slot = -1;  // the contiguous cache no longer holds a slot's rows
        if (scratch) {  // the scratch cache lives for this call only
            bufs_free();
            dfree(kv);
            kv = nullptr;
            kv_on = false;
            max_ctx = 0;
        }
    }

    // a prompt step of one slot: rows [pos, pos + s) computed on the contiguous cache, after
    // its rows [0, pos) are there (copied from its pages unless the previous prompt step of
    // this slot left them), then stored into its pages; the slot continues at pos + s
    void run_prompt_slot() {
        check_ids(s);
        const auto& pl = pg.pages[(size_t)slot];
        if (!pg.active[(size_t)slot]) raise(GQ_ERR_INVALID, "slot " + std::to_string(slot) + " is not allocated");
        if (pos + s > (int64_t)pl.size() * pg.P)
            raise(GQ_ERR_INVALID, "slot " + std::to_string(slot) + " holds " + std::to_string(pl.size() * pg.P) +
                                      " rows, pos + s = " + std::to_string(pos + s) + " (paged_kv_ensure_tokens first)");
        sync_tables();
        if (pg.contig_slot != slot || pg.contig_rows < pos) copy_rows(slot, 0, pos, 0);
        pg.contig_slot = -1;  // until the rows below are in place
        step_contig(pos, s, false);
        copy_rows(slot, pos, pos + s, 1);
        pg.contig_slot = slot, pg.contig_rows = pos + s;
        set_slot_pos(slot, pos + s);
    }

    // one decode token for every slot of [0, nb), each at its own position
    void run_batch() {
        check_ids(nb);
        int64_t longest = 1;
        for (int64_t i = 0; i < nb; ++i) {
            if (!pg.active[(size_t)i]) continue;  // its row writes the trash page, attends to nothing
            const int64_t p = pg.pos_host[(size_t)i];
            if (p + 1 > (int64_t)pg.pages[(size_t)i].size() * pg.P)
                raise(GQ_ERR_INVALID, "slot " + std::to_string(i) + " has no row for position " + std::to_string(p) +
                                          " (paged_kv_ensure_tokens first)");
            longest = std::max(longest, p + 1);
        }
        const int64_t max_len = std::min(pg.max_ctx, (longest + PAGED_BUCKET - 1) / PAGED_BUCKET * PAGED_BUCKET);
        sync_tables();
        Bufs& b = buffers(nb);
        size_workspace(nb, nb);
        hip_ok(hipMemcpyAsync(b.ids, ids_host.data(), (size_t)nb * 4, hipMemcpyHostToDevice, stream), "ids upload");
        launch_step(paged_graphs, std::make_tuple(nb, max_len), use_graphs, [&] { forward_paged(nb, max_len); });
        out_rows = nb;
        out_host.resize((size_t)nb * m.n_vocab);
        hip_ok(hipMemcpyAsync(out_host.data(), b.logits, out_host.size() * 4, hipMemcpyDeviceToHost, stream),
               "logits download");
        hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize");
        for (int64_t i = 0; i < nb; ++i) ++pg.pos_host[(size_t)i];
        pg.contig_slot = -1;
    }

    std::map<std::string, int64_t> env() const {
        std::map<std::string, int64_t> en{{"s", s}, {"pos", pos}};
        if (paged_step) en["b"] = nb, en["slot"] = slot < 0 ? 0 : slot;
        return en;
    }

    void shape(uint32_t tid, int64_t ne[4]) const {
        const GTensor& t = graph.t(tid);
        const auto en = env();
        for (int i = 0; i < 4; ++i) ne[i] = t.ne[i].eval(en);
        if (tid == m.output_tid) ne[1] = out_rows ? out_rows : ne[1];
    }

    ~Executor() {
        if (dev >= 0) (void)hipSetDevice(dev);
        if (stream) (void)hipStreamSynchronize(stream);
        drop_graphs();
        for (void* p : allocs) (void)hipFree(p);  // retired workspaces included
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

int parse_device(const char* device, int* dev) {
    const std::string d = device ? device : "auto";
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(GQ_ERR_DEVICE, "no GPU visible: this runtime has no CPU path");
    if (d == "auto" || d == "gpu" || d == "cuda") {
        *dev = 0;
        return GQ_OK;
    }
    for (const char* pre : {"cuda:", "gpu:"}) {
        if (d.rfind(pre, 0) == 0) {
            char* end = nullptr;
            const long v = strtol(d.c_str() + strlen(pre), &end, 10);
            if (end && *end == '\0' && v >= 0 && v < n) {
                *dev = (int)v;
                return GQ_OK;
            }
        }
    }
    return fail(GQ_ERR_INVALID, "device '" + d + "': this runtime executes on the GPU only ('gpu[:N]', 'cuda[:N]', 'auto')");
}

// runs body with the handle's device current; C++ errors become return codes
template <typename F>
int guarded(Executor* h, const char* what, F body) {
    if (!h) return fail(GQ_ERR_INVALID, std::string(what) + ": null handle");
    try {
        hip_ok(hipSetDevice(h->dev), "hipSetDevice");
        body();
        return GQ_OK;
    } catch (const Error& e) {
        return fail(e.code, std::string(what) + ": " + e.what());
    } catch (const std::exception& e) {
        return fail(GQ_ERR_DEVICE, std::string(what) + ": " + e.what());
    }
}

}  // namespace
}  // namespace gq

using namespace gq;

struct gq_exec {
    Executor ex;
};

extern "C" {

int gq_exec_create(const void* gguf_bytes, size_t len, const char* device, gq_exec** out) {
    if (!out) return fail(GQ_ERR_INVALID, "exec_create: null out");
    *out = nullptr;
    if (!gguf_bytes || len == 0) return fail(GQ_ERR_INVALID, "exec_create: empty model");
    int dev = 0;
    int rc = parse_device(device, &dev);
    if (rc) return rc;
    auto h = std::make_unique<gq_exec>();
    h->ex.dev = dev;
    h->ex.device = "cuda:" + std::to_string(dev);
    rc = guarded(&h->ex, "exec_create", [&] {
        gq_ok(gq_init());
        hip_ok(hipStreamCreate(&h->ex.stream), "hipStreamCreate");
        h->ex.file.buf.assign(static_cast<const uint8_t*>(gguf_bytes), static_cast<const uint8_t*>(gguf_bytes) + len);
        h->ex.file.parse();
        h->ex.load();
        hip_ok(hipStreamSynchronize(h->ex.stream), "hipStreamSynchronize");
    });
    if (rc) return rc;
    *out = h.release();
    return GQ_OK;
}

void gq_exec_free(gq_exec* h) { delete h; }

static int copy_out(const std::string& j, char* buf, size_t len, size_t* needed) {
    if (needed) *needed = j.size() + 1;
    if (buf && len) {
        const size_t n = std::min(len - 1, j.size());
        memcpy(buf, j.data(), n);
        buf[n] = '\0';
    }
    return GQ_OK;
}

int gq_exec_available_devices(char* buf, size_t len, size_t* needed) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    std::string j = "[";
    for (int i = 0; i < n; ++i) j += (i ? ",\"cuda:" : "\"cuda:") + std::to_string(i) + "\"";
    return copy_out(j + "]", buf, len, needed);
}

int gq_exec_describe(gq_exec* h, char* buf, size_t len, size_t* needed) {
    std::string j;
    const int rc = guarded(h ? &h->ex : nullptr, "exec_describe",
                           [&] { j = describe_json(h->ex.graph, h->ex.m, h->ex.device); });
    return rc ? rc : copy_out(j, buf, len, needed);
}

int gq_exec_inspect(const void* gguf_bytes, size_t len, char* buf, size_t buf_len, size_t* needed) {
    std::string j;
    try {
        if (!gguf_bytes || len == 0) raise(GQ_ERR_INVALID, "empty model");
        Gguf f;
        f.buf.assign(static_cast<const uint8_t*>(gguf_bytes), static_cast<const uint8_t*>(gguf_bytes) + len);
        f.parse();
        const auto it = f.strings.find("ggmlc.graph_spec");
        if (it == f.strings.end()) raise(GQ_ERR_INVALID, "GGUF metadata missing 'ggmlc.graph_spec'");
        const Graph g = parse_graph(it->second);
        j = describe_json(g, match_llama(g, f), "");
    } catch (const Error& e) {
        return fail(e.code, std::string("exec_inspect: ") + e.what());
    } catch (const std::exception& e) {
        return fail(GQ_ERR_INVALID, std::string("exec_inspect: ") + e.what());
    }
    return copy_out(j, buf, buf_len, needed);
}

int gq_exec_prepare(gq_exec* h, const char* const* names, const int64_t* values, int64_t n) {
    const auto t0 = std::chrono::steady_clock::now();
    const int rc = guarded(h ? &h->ex : nullptr, "exec_prepare", [&] {
        Executor& e = h->ex;
        int64_t s = -1, pos = -1, b = -1, slot = -1;
        for (int64_t i = 0; i < n; ++i) {
            if (!names || !names[i]) raise(GQ_ERR_INVALID, "null symbol name");
            const std::string k = names[i];
            if (k == "s") s = values[i];
            else if (k == "pos") pos = values[i];
            else if (k == "b") b = values[i];
            else if (k == "slot") slot = values[i];
            else if (std::find(e.graph.symbols.begin(), e.graph.symbols.end(), k) == e.graph.symbols.end())
                raise(GQ_ERR_INVALID, "unknown symbol " + k);
        }
        if (s <= 0) raise(GQ_ERR_INVALID, "symbol s must be given and positive");
        if (b == 0 || b < -1) raise(GQ_ERR_INVALID, "symbol b must be positive");
        if (slot < -1) raise(GQ_ERR_INVALID, "symbol slot must not be negative");
        if (pos < -1) raise(GQ_ERR_INVALID, "symbol pos must not be negative");
        bool paged = false;
        if (e.pg.on && (slot >= 0 || b >= 1)) {
            // the reference scheduler's protocol (batch_scheduler.cpp:190-194, 318-321): a prompt
            // step names its slot (b = 1); a decode step gives b (s = 1) and runs slots [0, b)
            paged = true;
            if (slot >= 0) {
                e.check_slot(slot);
                if (b > 1) raise(GQ_ERR_INVALID, "a prompt step of one slot needs b = 1");
                if (pos < 0) pos = e.pg.pos_host[(size_t)slot];
                if (pos + s > e.pg.max_ctx)
                    raise(GQ_ERR_INVALID, "pos + s = " + std::to_string(pos + s) + " exceeds the slots' max_ctx (" +
                                              std::to_string(e.pg.max_ctx) + ")");
            } else {
                if (s != 1) raise(GQ_ERR_INVALID, "a batched step decodes one token per slot: s must be 1");
                if (b > e.pg.max_batch)
                    raise(GQ_ERR_INVALID, "b = " + std::to_string(b) + " exceeds max_batch (" +
                                              std::to_string(e.pg.max_batch) + ")");
                // each slot decodes at its own position; pos (the scheduler passes the
                // largest) only has to cover them
                for (int64_t i = 0; i < b && pos >= 0; ++i)
                    if (e.pg.active[(size_t)i] && e.pg.pos_host[(size_t)i] > pos)
                        raise(GQ_ERR_INVALID, "pos = " + std::to_string(pos) + " is below slot " + std::to_string(i) +
                                                  "'s position " + std::to_string(e.pg.pos_host[(size_t)i]));
            }
        } else {
            if ((b > 1 || slot > 0))
                raise(GQ_ERR_INVALID, "symbols b > 1 and slot > 0 need init_paged_kv_cache");
            if (pos < 0) pos = e.kv_on ? e.pos : 0;
            if (e.kv_on && pos + s > e.max_ctx)
                raise(GQ_ERR_INVALID, "pos + s = " + std::to_string(pos + s) + " exceeds the KV cache (" +
                                          std::to_string(e.max_ctx) + ")");
        }
        e.s = s, e.pos = pos < 0 ? 0 : pos, e.prepared = true;
        e.paged_step = paged, e.slot = paged ? (int)slot : -1, e.nb = paged && slot < 0 ? (b < 0 ? 1 : b) : 1;
        e.ids_host.clear();
        e.out_rows = 0;
    });
    if (rc == GQ_OK && h->ex.profile_on) {
        h->ex.prof_prepare_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        ++h->ex.prof_n_prepare;
    }
    return rc;
}

int gq_exec_set_input(gq_exec* h, uint32_t tensor_id, const void* data, size_t bytes) {
    return guarded(h ? &h->ex : nullptr, "exec_set_input", [&] {
        Executor& e = h->ex;
        if (!e.prepared) raise(GQ_ERR_INVALID, "call prepare first");
        if (tensor_id != e.m.input_tid) raise(GQ_ERR_INVALID, "tensor " + std::to_string(tensor_id) + " is not the graph input");
        const int type = e.graph.t(tensor_id).type;
        const size_t es = type == GQ_TYPE_I64 ? 8 : 4;
        const int64_t n_ids = e.s * e.nb;  // s token ids (b x 1 in a batched decode step)
        if (!data || bytes != (size_t)n_ids * es)
            raise(GQ_ERR_INVALID, "input holds " + std::to_string(bytes) + " bytes, expected " +
                                      std::to_string((size_t)n_ids * es) + " (s x b token ids)");
        e.ids_host.resize((size_t)n_ids);
        for (int64_t i = 0; i < n_ids; ++i) {
            int64_t v;
            if (es == 8) memcpy(&v, static_cast<const uint8_t*>(data) + 8 * i, 8);
            else {
                int32_t w;
                memcpy(&w, static_cast<const uint8_t*>(data) + 4 * i, 4);
                v = w;
            }
            if (v < INT32_MIN || v > INT32_MAX) raise(GQ_ERR_INVALID, "token id out of range");
            e.ids_host[(size_t)i] = (int32_t)v;
        }
    });
}

int gq_exec_set_input_by_name(gq_exec* h, const char* name, const void* data, size_t bytes) {
    uint32_t tid = 0;
    const int rc = guarded(h ? &h->ex : nullptr, "exec_set_input_by_name", [&] {
        bool found = false;
        for (uint32_t t : h->ex.graph.inputs)
            if (name && h->ex.graph.t(t).name == name) tid = t, found = true;
        if (!found) raise(GQ_ERR_INVALID, std::string("no input named ") + (name ? name : "(null)"));
    });
    if (rc) return rc;
    return gq_exec_set_input(h, tid, data, bytes);
}

int gq_exec_run(gq_exec* h) {
    const auto t0 = std::chrono::steady_clock::now();
    const int rc = guarded(h ? &h->ex : nullptr, "exec_run", [&] { h->ex.run(); });
    if (rc == GQ_OK && h->ex.profile_on) {
        h->ex.prof_run_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        ++h->ex.prof_n_run;
    }
    return rc;
}

int gq_exec_synchronize(gq_exec* h) {
    return guarded(h ? &h->ex : nullptr, "exec_synchronize",
                   [&] { hip_ok(hipStreamSynchronize(h->ex.stream), "hipStreamSynchronize"); });
}

int gq_exec_get_tensor_shape(gq_exec* h, uint32_t tensor_id, int64_t ne[4]) {
    return guarded(h ? &h->ex : nullptr, "exec_get_tensor_shape", [&] {
        if (!ne) raise(GQ_ERR_INVALID, "null ne");
        h->ex.shape(tensor_id, ne);
    });
}

int gq_exec_get_output(gq_exec* h, uint32_t tensor_id, void* dst, size_t bytes, size_t* written) {
    return guarded(h ? &h->ex : nullptr, "exec_get_output", [&] {
        Executor& e = h->ex;
        if (tensor_id != e.m.output_tid) raise(GQ_ERR_INVALID, "tensor " + std::to_string(tensor_id) + " is not the graph output");
        if (e.out_rows == 0) raise(GQ_ERR_INVALID, "no output yet: run first");
        const size_t n = e.out_host.size() * 4;
        if (written) *written = n;
        if (dst) {
            if (bytes < n) raise(GQ_ERR_INVALID, "output buffer holds " + std::to_string(bytes) + " bytes, needs " + std::to_string(n));
            memcpy(dst, e.out_host.data(), n);
        }
    });
}

int gq_exec_init_kv_cache(gq_exec* h, int64_t max_ctx) {
    return guarded(h ? &h->ex : nullptr, "exec_init_kv_cache", [&] {
        h->ex.init_kv(max_ctx);
        hip_ok(hipStreamSynchronize(h->ex.stream), "hipStreamSynchronize");
    });
}

int gq_exec_reset_kv_cache(gq_exec* h) {
    return guarded(h ? &h->ex : nullptr, "exec_reset_kv_cache", [&] {
        h->ex.reset_kv();
        h->ex.pos = 0;
    });
}

int gq_exec_has_kv_cache(gq_exec* h) { return h && h->ex.kv_on ? 1 : 0; }

int gq_exec_set_logits_last_only(gq_exec* h, int enable) {
    return guarded(h ? &h->ex : nullptr, "exec_set_logits_last_only", [&] { h->ex.logits_last_only = enable != 0; });
}

int gq_exec_logits_last_only(gq_exec* h) { return h && h->ex.logits_last_only ? 1 : 0; }

int gq_exec_set_enable_graphs(gq_exec* h, int enable) {
    return guarded(h ? &h->ex : nullptr, "exec_set_enable_graphs", [&] { h->ex.use_graphs = enable != 0; });
}

int64_t gq_exec_position(gq_exec* h) { return h ? h->ex.pos : -1; }

// ---- paged KV (executor.h:73-93) ----------------------------------------------------
int gq_exec_set_tokens_per_page(gq_exec* h, int64_t n) {
    return guarded(h ? &h->ex : nullptr, "exec_set_tokens_per_page", [&] { h->ex.set_tokens_per_page(n); });
}

int64_t gq_exec_get_tokens_per_page(gq_exec* h) { return h ? h->ex.pg.P : -1; }

int gq_exec_init_paged_kv_cache(gq_exec* h, int64_t max_batch, int64_t max_ctx) {
    return guarded(h ? &h->ex : nullptr, "exec_init_paged_kv_cache", [&] { h->ex.init_paged(max_batch, max_ctx); });
}

int gq_exec_is_paged_kv_cache_enabled(gq_exec* h) { return h && h->ex.pg.on ? 1 : 0; }

int gq_exec_paged_kv_alloc_slot(gq_exec* h, int64_t slot) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_kv_alloc_slot", [&] { h->ex.alloc_slot(slot); });
}

int gq_exec_paged_kv_free_slot(gq_exec* h, int64_t slot) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_kv_free_slot", [&] { h->ex.free_slot(slot); });
}

int gq_exec_is_paged_slot_allocated(gq_exec* h, int64_t slot) {
    if (!h || !h->ex.pg.on || slot < 0 || slot >= h->ex.pg.max_batch) return 0;
    return h->ex.pg.active[(size_t)slot] ? 1 : 0;
}

int gq_exec_paged_kv_ensure_tokens(gq_exec* h, int64_t slot, int64_t total_tokens) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_kv_ensure_tokens",
                   [&] { h->ex.ensure_tokens(slot, total_tokens); });
}

int gq_exec_paged_kv_map_existing_pages(gq_exec* h, int64_t slot, int64_t start_page, const int32_t* pages,
                                        int64_t n_pages) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_kv_map_existing_pages",
                   [&] { h->ex.map_pages(slot, start_page, pages, n_pages); });
}

int gq_exec_paged_kv_extract_page(gq_exec* h, int64_t slot, int64_t page_idx, int32_t* page) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_kv_extract_page", [&] {
        if (!page) raise(GQ_ERR_INVALID, "null page");
        *page = h->ex.page_of(slot, page_idx);
    });
}

int gq_exec_paged_page_retain(gq_exec* h, int32_t page) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_page_retain", [&] {
        h->ex.need_paged();
        h->ex.retain_page(page);
    });
}

int gq_exec_paged_page_release(gq_exec* h, int32_t page) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_page_release", [&] {
        h->ex.need_paged();
        h->ex.release_page(page);
    });
}

size_t gq_exec_get_paged_active_vram_bytes(gq_exec* h) { return h ? h->ex.active_bytes() : 0; }

int gq_exec_paged_slot_position(gq_exec* h, int64_t slot, int64_t* pos) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_slot_position", [&] {
        h->ex.check_slot(slot);
        if (!pos) raise(GQ_ERR_INVALID, "null pos");
        *pos = h->ex.pg.pos_host[(size_t)slot];
    });
}

int gq_exec_paged_set_slot_position(gq_exec* h, int64_t slot, int64_t pos) {
    return guarded(h ? &h->ex : nullptr, "exec_paged_set_slot_position", [&] {
        Executor& e = h->ex;
        e.check_slot(slot);
        if (pos < 0 || pos > e.pg.max_ctx) raise(GQ_ERR_INVALID, "position outside [0, max_ctx]");
        e.set_slot_pos(slot, pos);
        if (e.pg.contig_slot == slot) e.pg.contig_rows = std::min(e.pg.contig_rows, pos);
    });
}

// ---- profiling (executor.h:101-118) --------------------------------------------------
int gq_exec_set_enable_profile(gq_exec* h, int enable) {
    return guarded(h ? &h->ex : nullptr, "exec_set_enable_profile", [&] { h->ex.profile_on = enable != 0; });
}

int gq_exec_reset_profile(gq_exec* h) {
    return guarded(h ? &h->ex : nullptr, "exec_reset_profile", [&] {
        Executor& e = h->ex;
        e.prof_prepare_ms = e.prof_run_ms = 0.0;
        e.prof_n_prepare = e.prof_n_run = 0;
    });
}

int gq_exec_get_profile(gq_exec* h, gq_exec_profile* out) {
    return guarded(h ? &h->ex : nullptr, "exec_get_profile", [&] {
        if (!out) raise(GQ_ERR_INVALID, "null profile");
        const Executor& e = h->ex;
        *out = gq_exec_profile{};
        out->prepare_ms = e.prof_prepare_ms, out->run_ms = e.prof_run_ms;
        out->n_prepare = e.prof_n_prepare, out->n_run = e.prof_n_run;
    });
}

int gq_exec_runtime_graph_summary(gq_exec* h, char* buf, size_t len, size_t* needed) {
    std::string j;
    const int rc = guarded(h ? &h->ex : nullptr, "exec_runtime_graph_summary", [&] {
        const Executor& e = h->ex;
        int64_t n = 0, n_mm = 0, n_fa = 0, n_set = 0;
        std::string ops;
        for (const auto& kv : e.op_hist) {
            n += kv.second;
            if (kv.first.find("MUL_MAT") != std::string::npos) n_mm += kv.second;
            if (kv.first.find("FLASH_ATTN") != std::string::npos) n_fa += kv.second;
            if (kv.first.find("SET_ROWS") != std::string::npos) n_set += kv.second;
            ops += (ops.empty() ? "\"" : ",\"") + kv.first + "\":" + std::to_string(kv.second);
        }
        j = "{\"n_nodes\":" + std::to_string(n) + ",\"n_kernel_nodes\":" +
            std::to_string(e.last_nodes >= 0 ? e.last_nodes : n) + ",\"n_mul_mat\":" + std::to_string(n_mm) +
            ",\"n_flash_attn\":" + std::to_string(n_fa) + ",\"n_set_rows\":" + std::to_string(n_set) +
            ",\"kv_n_pad\":" + std::to_string(e.kv_n_pad) + ",\"graphs_captured\":" +
            std::to_string(e.graphs.size() + e.paged_graphs.size()) + ",\"last_run_replayed\":" +
            (e.last_nodes >= 0 ? "true" : "false") + ",\"paged_kv\":" + (e.pg.on ? "true" : "false") +
            ",\"ops\":{" + ops + "}}";
    });
    return rc ? rc : copy_out(j, buf, len, needed);
}

int gq_exec_runtime_mul_mat_shape_summary(gq_exec* h, char* buf, size_t len, size_t* needed) {
    std::string j;
    const int rc = guarded(h ? &h->ex : nullptr, "exec_runtime_mul_mat_shape_summary", [&] {
        auto list = [](const std::map<std::string, int64_t>& m) {
            std::vector<std::pair<std::string, int64_t>> v(m.begin(), m.end());
            std::stable_sort(v.begin(), v.end(), [](const auto& a, const auto& b) { return a.second > b.second; });
            std::string o = "[";
            for (size_t i = 0; i < v.size(); ++i)
                o += std::string(i ? "," : "") + "{\"n\":" + std::to_string(v[i].second) + ",\"shape\":\"" +
                     v[i].first + "\"}";
            return o + "]";
        };
        j = "{\"mul_mat\":" + list(h->ex.mm_shapes) + ",\"flash_attn\":" + list(h->ex.fa_shapes) + "}";
    });
    return rc ? rc : copy_out(j, buf, len, needed);
}

}  // extern "C"
