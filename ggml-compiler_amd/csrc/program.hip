// program.hip - ggml-compiler's runtime on this library: the GGUF program loader, its driver and
// the model C API of include/ggml_compiler_rt.h (reference: runtime/include/ggml_compiler_rt.h:91-172).
//
// A GGUF written by ggml-compiler holds weights and constants (tensors "w.N" / "c.N") and a program
// (JSON under "ggml_compiler.program", written by ggml_compiler/emit/gguf_runtime.py:104-207):
// symbols with ranges, driver values, stages whose nodes are already in ggml terms (innermost-first
// `ne`, ggml axes), entry points whose drivers call stages and run loops, and state values. Loading
// uploads every tensor into one HIP buffer (quantized ones in this library's packed layout),
// allocates every driver value in a second buffer (zeroed, so state starts at zero) and builds one
// graph per driver call site with the ggml API, placed by the graph allocator. A run walks the
// entry's driver; each call computes its site's graph with ggml_backend_graph_compute, which
// replays a captured HIP graph after the first run. Results reach their driver values through
// ggml_cpy nodes appended after every other node, except a result that already is its value's
// memory (set_rows into a KV cache the stage read).
//
// Semantics kept from the reference: the program schema and its checks (runtime/src/program.cpp:
// 61-300), symbolic dims as expression trees evaluated per binding, driver values of symbolic size
// held at their largest size with per-binding views (runtime/src/ggml_compiler_rt.cpp:481-548), the
// per-site graph build and its result copies (:566-700), the loop's order of carries, scalars,
// slices, counters, bound symbols, causal masks, body, collected rows and the until test (:376-441),
// and the C API's argument checks and messages (:812-1170). The JSON reader, GGUF reader, op
// dispatch and data structures are this file's own.
#include "gcq_common.h"
#include "ggml_impl.h"

#include "../../include/gcq.h"
#include "../../include/ggml_compiler_rt.h"

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <unordered_map>
#include <vector>

#include <fcntl.h>
#include <unistd.h>

namespace gcq {
namespace {

// ------------------------------------------------------------------------------------ JSON

struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    bool integral = false;  // a number written without fraction or exponent
    int64_t i = 0;
    std::string s;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json * find(const std::string & key) const {
        if (kind != Obj) return nullptr;
        for (const auto & kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    const Json & at(const std::string & key) const {
        const Json * j = find(key);
        if (!j) fail("malformed program: missing key '" + key + "'");
        return *j;
    }
    int64_t as_int() const {
        if (kind != Num || !integral) fail("malformed program: expected an integer");
        return i;
    }
    double as_num() const {
        if (kind != Num) fail("malformed program: expected a number");
        return num;
    }
    const std::string & as_str() const {
        if (kind != Str) fail("malformed program: expected a string");
        return s;
    }
    const std::vector<Json> & items() const {
        if (kind != Arr) fail("malformed program: expected an array");
        return arr;
    }
    std::vector<std::string> strings() const {
        std::vector<std::string> out;
        for (const auto & e : items()) out.push_back(e.as_str());
        return out;
    }
};

class JsonReader {
  public:
    JsonReader(const std::string & text) : p_(text.data()), end_(text.data() + text.size()) {}

    Json document() {
        Json v = value(0);
        ws();
        if (p_ != end_) error("trailing characters");
        return v;
    }

  private:
    const char * p_;
    const char * end_;

    [[noreturn]] void error(const char * what) { fail(std::string("program JSON does not parse: ") + what); }
    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool eat(char c) {
        ws();
        if (p_ < end_ && *p_ == c) {
            p_++;
            return true;
        }
        return false;
    }
    void expect(char c) {
        if (!eat(c)) error("unexpected character");
    }
    bool word(const char * w) {
        const size_t n = std::strlen(w);
        if ((size_t) (end_ - p_) >= n && std::memcmp(p_, w, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    static void put_utf8(std::string & out, uint32_t cp) {
        if (cp < 0x80) {
            out += (char) cp;
        } else if (cp < 0x800) {
            out += (char) (0xC0 | (cp >> 6));
            out += (char) (0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += (char) (0xE0 | (cp >> 12));
            out += (char) (0x80 | ((cp >> 6) & 0x3F));
            out += (char) (0x80 | (cp & 0x3F));
        } else {
            out += (char) (0xF0 | (cp >> 18));
            out += (char) (0x80 | ((cp >> 12) & 0x3F));
            out += (char) (0x80 | ((cp >> 6) & 0x3F));
            out += (char) (0x80 | (cp & 0x3F));
        }
    }
    uint32_t hex4() {
        if (end_ - p_ < 4) error("short \\u escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; k++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t) (c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t) (c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t) (c - 'A' + 10);
            else error("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        // after the opening quote
        std::string out;
        while (true) {
            if (p_ >= end_) error("unterminated string");
            const char c = *p_++;
            if (c == '"') return out;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ >= end_) error("unterminated escape");
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
                    uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                        p_ += 2;
                        const uint32_t lo = hex4();
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: error("bad escape");
            }
        }
    }
    Json value(int depth) {
        if (depth > 256) error("nesting too deep");
        ws();
        if (p_ >= end_) error("unexpected end");
        Json v;
        const char c = *p_;
        if (c == '{') {
            p_++;
            v.kind = Json::Obj;
            if (eat('}')) return v;
            do {
                ws();
                if (p_ >= end_ || *p_ != '"') error("expected a key");
                p_++;
                std::string k = string();
                expect(':');
                v.obj.emplace_back(std::move(k), value(depth + 1));
            } while (eat(','));
            expect('}');
        } else if (c == '[') {
            p_++;
            v.kind = Json::Arr;
            if (eat(']')) return v;
            do {
                v.arr.push_back(value(depth + 1));
            } while (eat(','));
            expect(']');
        } else if (c == '"') {
            p_++;
            v.kind = Json::Str;
            v.s = string();
        } else if (word("true")) {
            v.kind = Json::Bool;
            v.b = true;
        } else if (word("false")) {
            v.kind = Json::Bool;
        } else if (word("null")) {
            v.kind = Json::Null;
        } else if (word("NaN")) {
            v.kind = Json::Num;
            v.num = NAN;
        } else if (word("Infinity")) {
            v.kind = Json::Num;
            v.num = INFINITY;
        } else if (word("-Infinity")) {
            v.kind = Json::Num;
            v.num = -INFINITY;
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            const char * s = p_;
            bool integral = true;
            if (*p_ == '-') p_++;
            while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                                 *p_ == '+' || *p_ == '-')) {
                if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') integral = false;
                p_++;
            }
            const std::string text(s, p_);
            char * stop = nullptr;
            v.kind = Json::Num;
            v.num = std::strtod(text.c_str(), &stop);
            if (!stop || *stop) error("bad number");
            if (integral) {
                errno = 0;
                v.i = std::strtoll(text.c_str(), &stop, 10);
                v.integral = errno == 0 && stop && !*stop;
            }
        } else {
            error("unexpected character");
        }
        return v;
    }
};

// ------------------------------------------------------------------------------------ GGUF

// The parts of a GGUF (v2 / v3) the loader reads: string values, tensor infos, the data offset.
struct GgufFile {
    struct Info {
        std::string name;
        int type = 0;
        int64_t ne[4] = {1, 1, 1, 1};
        uint64_t offset = 0;
    };
    std::string path;
    std::map<std::string, std::string> strings;
    std::vector<Info> tensors;
    uint64_t data_offset = 0;

    void open(const std::string & p) {
        path = p;
        FILE * f = std::fopen(p.c_str(), "rb");
        if (!f) fail("cannot read GGUF '" + p + "'");
        std::unique_ptr<FILE, int (*)(FILE *)> hold(f, std::fclose);
        auto raw = [&](void * dst, size_t n) {
            if (n && std::fread(dst, 1, n, f) != n) fail("cannot read GGUF '" + p + "': truncated");
        };
        auto u32 = [&] {
            uint32_t v;
            raw(&v, 4);
            return v;
        };
        auto u64 = [&] {
            uint64_t v;
            raw(&v, 8);
            return v;
        };
        auto str = [&] {
            const uint64_t n = u64();
            if (n > (1ull << 32)) fail("cannot read GGUF '" + p + "': string of " + std::to_string(n) + " bytes");
            std::string s(n, '\0');
            raw(s.data(), n);
            return s;
        };
        char magic[4];
        raw(magic, 4);
        if (std::memcmp(magic, "GGUF", 4) != 0) fail("cannot read GGUF '" + p + "': not a GGUF file");
        const uint32_t version = u32();
        if (version < 2 || version > 3) fail("cannot read GGUF '" + p + "': version " + std::to_string(version));
        const uint64_t n_tensors = u64(), n_kv = u64();
        uint64_t alignment = 32;
        static const int kScalar[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};  // bytes per GGUF value type
        std::function<void(uint32_t)> skip = [&](uint32_t t) {
            if (t == 8) {
                (void) str();
            } else if (t == 9) {
                const uint32_t et = u32();
                const uint64_t n = u64();
                for (uint64_t k = 0; k < n; k++) skip(et);
            } else if (t < 13) {
                char buf[8];
                raw(buf, (size_t) kScalar[t]);
            } else {
                fail("cannot read GGUF '" + p + "': value type " + std::to_string(t));
            }
        };
        for (uint64_t k = 0; k < n_kv; k++) {
            const std::string key = str();
            const uint32_t t = u32();
            if (t == 8) {
                strings[key] = str();
            } else if (key == "general.alignment" && t == 4) {
                alignment = u32();
            } else {
                skip(t);
            }
        }
        if (alignment == 0 || (alignment & (alignment - 1))) fail("cannot read GGUF '" + p + "': bad alignment");
        for (uint64_t k = 0; k < n_tensors; k++) {
            Info in;
            in.name = str();
            const uint32_t nd = u32();
            if (nd > 4) fail("GGUF tensor '" + in.name + "' has " + std::to_string(nd) + " dims");
            for (uint32_t d = 0; d < nd; d++) in.ne[d] = (int64_t) u64();
            in.type = (int) u32();
            in.offset = u64();
            tensors.push_back(std::move(in));
        }
        const long pos = std::ftell(f);
        data_offset = ((uint64_t) pos + alignment - 1) / alignment * alignment;
    }
};

// ---------------------------------------------------------------------------------- program

struct Symbol {
    std::string name;
    int64_t min = 1, max = 1;
};

// An integer dim: a constant, symbol `v`, or an operation folded left over its arguments.
struct Expr {
    enum Kind { Const, Sym, Add, Mul, FloorDiv, Mod, Max, Min } kind = Const;
    int64_t v = 0;
    std::vector<Expr> args;

    bool constant() const { return kind == Const; }
    int64_t eval(const std::vector<int64_t> & b) const {
        if (kind == Const) return v;
        if (kind == Sym) return b.at((size_t) v);
        int64_t acc = args.at(0).eval(b);
        for (size_t k = 1; k < args.size(); k++) {
            const int64_t x = args[k].eval(b);
            switch (kind) {
                case Add: acc += x; break;
                case Mul: acc *= x; break;
                case FloorDiv: {  // Python's //: rounds toward minus infinity
                    if (x == 0) fail("division by zero in a symbolic dim");
                    const int64_t q = acc / x;
                    acc = (q * x != acc && ((acc < 0) != (x < 0))) ? q - 1 : q;
                    break;
                }
                case Mod: {  // Python's %: the sign of the divisor
                    if (x == 0) fail("modulo by zero in a symbolic dim");
                    int64_t r = acc % x;
                    if (r != 0 && ((r < 0) != (x < 0))) r += x;
                    acc = r;
                    break;
                }
                case Max: acc = std::max(acc, x); break;
                case Min: acc = std::min(acc, x); break;
                default: break;
            }
        }
        return acc;
    }
    void uses(std::vector<bool> & used) const {
        if (kind == Sym) used.at((size_t) v) = true;
        for (const auto & a : args) a.uses(used);
    }
};

Expr parse_dim(const Json & j, const std::vector<Symbol> & syms) {
    Expr e;
    if (j.kind == Json::Num) {
        e.v = j.as_int();
        return e;
    }
    if (j.kind == Json::Str) {
        for (size_t k = 0; k < syms.size(); k++)
            if (syms[k].name == j.s) {
                e.kind = Expr::Sym;
                e.v = (int64_t) k;
                return e;
            }
        fail("dim refers to unknown symbol '" + j.s + "'");
    }
    if (j.kind != Json::Arr || j.arr.size() < 2 || j.arr[0].kind != Json::Str) fail("malformed dim");
    static const std::pair<const char *, Expr::Kind> ops[] = {{"+", Expr::Add},       {"*", Expr::Mul},
                                                               {"//", Expr::FloorDiv}, {"%", Expr::Mod},
                                                               {"max", Expr::Max},     {"min", Expr::Min}};
    bool known = false;
    for (const auto & o : ops)
        if (j.arr[0].s == o.first) {
            e.kind = o.second;
            known = true;
        }
    if (!known) fail("unknown dim operator '" + j.arr[0].s + "'");
    for (size_t k = 1; k < j.arr.size(); k++) e.args.push_back(parse_dim(j.arr[k], syms));
    return e;
}

int parse_type_name(const std::string & name) {
    for (int t = 0; t < GGML_TYPE_COUNT; t++) {
        const char * tn = ggml_type_name((ggml_type) t);
        if (tn && name == tn) return t;
    }
    fail("unknown tensor type '" + name + "'");
}

struct TensorSpec {
    std::string name;
    int type = GGML_TYPE_F32;
    Expr ne_x[4];
    std::vector<Expr> shape_x;
    int64_t ne[4] = {1, 1, 1, 1};  // for the current binding
    std::vector<int64_t> shape;

    bool symbolic() const {
        for (const auto & d : ne_x)
            if (!d.constant()) return true;
        return false;
    }
    void bind(const std::vector<int64_t> & b) {
        for (int k = 0; k < 4; k++) {
            ne[k] = ne_x[k].eval(b);
            if (ne[k] < 1) fail("value '" + name + "' gets a dim of " + std::to_string(ne[k]));
        }
        shape.clear();
        for (const auto & d : shape_x) shape.push_back(d.eval(b));
    }
    size_t nbytes(const std::vector<int64_t> & b) const {
        int64_t n[4];
        for (int k = 0; k < 4; k++) n[k] = ne_x[k].eval(b);
        return ggml_row_size((ggml_type) type, n[0]) * (size_t) (n[1] * n[2] * n[3]);
    }
};

void parse_ne(const Json & j, const std::vector<Symbol> & syms, Expr (&ne)[4]) {
    if (j.kind != Json::Arr || j.arr.size() != 4) fail("'ne' must be an array of 4 dims");
    for (int k = 0; k < 4; k++) ne[k] = parse_dim(j.arr[k], syms);
}

TensorSpec parse_tensor(const Json & j, const std::vector<Symbol> & syms) {
    TensorSpec t;
    t.name = j.at("name").as_str();
    t.type = parse_type_name(j.at("type").as_str());
    parse_ne(j.at("ne"), syms, t.ne_x);
    for (const auto & d : j.at("shape").items()) t.shape_x.push_back(parse_dim(d, syms));
    return t;
}

struct NodeSpec {
    std::string id, op, loc;
    std::vector<std::string> src;
    int type = GGML_TYPE_F32;
    Expr ne_x[4];
    int64_t ne[4] = {1, 1, 1, 1};
    Json p;                                    // op parameters
    std::vector<std::pair<std::string, Expr>> p_x;  // symbolic ones (a view's start)
    std::map<std::string, int64_t> p_bound;         // their values for the binding

    bool has(const char * key) const { return p_bound.count(key) || p.find(key); }
    double num(const char * key) const {
        auto it = p_bound.find(key);
        if (it != p_bound.end()) return (double) it->second;
        const Json * v = p.find(key);
        if (!v) fail(id + " (" + op + "): missing parameter '" + key + "'");
        return v->as_num();
    }
    double num_or(const char * key, double dflt) const { return has(key) ? num(key) : dflt; }
    int64_t integer(const char * key) const {
        auto it = p_bound.find(key);
        if (it != p_bound.end()) return it->second;
        const Json * v = p.find(key);
        if (!v) fail(id + " (" + op + "): missing parameter '" + key + "'");
        return v->as_int();
    }
};

struct StageSpec {
    std::string name;
    std::vector<TensorSpec> params;
    std::vector<std::string> outputs;
    std::vector<NodeSpec> nodes;
    bool symbolic = false;  // any shape of the stage reads a symbol
};

struct DriverOp {
    bool loop = false;
    // call
    std::string stage;
    std::vector<std::string> args, out;
    int site = -1;
    // loop
    int n = 0, n_symbol = -1;
    std::vector<std::pair<std::string, std::string>> counters, collect, carry, slices;
    std::vector<std::pair<int, Expr>> bind;
    std::vector<std::pair<std::string, int>> masks;
    std::vector<std::pair<std::string, std::vector<int>>> until;
    std::vector<std::pair<std::string, std::vector<float>>> scalars;
    std::vector<DriverOp> body;
    std::vector<std::vector<ggml_tensor *>> slice_rows;  // per slice, n row views (made at bind)
};

struct EntrySpec {
    std::string name;
    std::vector<std::string> inputs, outputs;
    std::vector<DriverOp> driver;
};

struct Program {
    int format = 0;
    std::vector<Symbol> symbols;
    std::vector<TensorSpec> values;
    std::vector<StageSpec> stages;
    std::vector<EntrySpec> entries;
    std::vector<std::string> state;

    int symbol(const std::string & name) const {
        for (size_t k = 0; k < symbols.size(); k++)
            if (symbols[k].name == name) return (int) k;
        return -1;
    }
    void bind(const std::vector<int64_t> & b) {
        if (b.size() != symbols.size()) fail("binding has the wrong number of symbols");
        for (size_t k = 0; k < symbols.size(); k++)
            if (b[k] < symbols[k].min || b[k] > symbols[k].max)
                fail("symbol '" + symbols[k].name + "' = " + std::to_string(b[k]) + " is outside [" +
                     std::to_string(symbols[k].min) + ", " + std::to_string(symbols[k].max) + "]");
        for (auto & v : values) v.bind(b);
        for (auto & s : stages) {
            for (auto & p : s.params) p.bind(b);
            for (auto & n : s.nodes) {
                for (int k = 0; k < 4; k++) n.ne[k] = n.ne_x[k].eval(b);
                for (const auto & kv : n.p_x) n.p_bound[kv.first] = kv.second.eval(b);
            }
        }
    }
};

DriverOp parse_driver(const Json & j, const std::vector<Symbol> & syms) {
    DriverOp d;
    const std::string & kind = j.at("op").as_str();
    if (kind == "call") {
        d.stage = j.at("stage").as_str();
        d.args = j.at("args").strings();
        d.out = j.at("out").strings();
        return d;
    }
    if (kind != "loop") fail("driver op '" + kind + "' is not supported by this runtime");
    d.loop = true;
    const Json & n = j.at("n");
    if (n.kind == Json::Str) {  // a trip count bound at run time
        for (size_t k = 0; k < syms.size(); k++)
            if (syms[k].name == n.s) d.n_symbol = (int) k;
        if (d.n_symbol < 0) fail("loop count refers to unknown symbol '" + n.s + "'");
        d.n = (int) syms[d.n_symbol].max;
    } else {
        d.n = (int) n.as_int();
    }
    auto pairs = [&](const char * key, std::vector<std::pair<std::string, std::string>> & out, bool required) {
        const Json * a = j.find(key);
        if (!a) {
            if (required) fail(std::string("malformed program: loop without '") + key + "'");
            return;
        }
        for (const auto & e : a->items()) {
            if (e.items().size() != 2) fail(std::string("malformed program: loop '") + key + "' entry");
            out.emplace_back(e.arr[0].as_str(), e.arr[1].as_str());
        }
    };
    pairs("counters", d.counters, false);
    std::vector<Symbol> ext = syms;  // counters extend the symbols of the bind expressions
    for (const auto & c : d.counters) ext.push_back({c.first, 0, INT64_MAX});
    if (const Json * b = j.find("bind"))
        for (const auto & e : b->items()) {
            const int k = [&] {
                for (size_t q = 0; q < syms.size(); q++)
                    if (syms[q].name == e.items().at(0).as_str()) return (int) q;
                fail("loop binds unknown symbol '" + e.arr[0].as_str() + "'");
            }();
            d.bind.emplace_back(k, parse_dim(e.arr.at(1), ext));
        }
    if (const Json * m = j.find("masks"))
        for (const auto & e : m->items()) {
            int k = -1;
            for (size_t q = 0; q < d.counters.size(); q++)
                if (d.counters[q].first == e.items().at(1).as_str()) k = (int) q;
            if (k < 0) fail("loop mask uses unknown counter '" + e.arr[1].as_str() + "'");
            d.masks.emplace_back(e.arr[0].as_str(), k);
        }
    if (const Json * u = j.find("until"))
        for (const auto & e : u->items()) {
            std::vector<int> ids;
            for (const auto & x : e.items().at(1).items()) ids.push_back((int) x.as_int());
            d.until.emplace_back(e.arr[0].as_str(), ids);
        }
    pairs("collect", d.collect, false);
    pairs("carry", d.carry, true);
    for (const auto & sc : j.at("scalars").items()) {
        std::vector<float> vals;
        for (const auto & x : sc.at("values").items()) vals.push_back((float) x.as_num());
        if ((int) vals.size() != d.n)
            fail("loop scalar has " + std::to_string(vals.size()) + " entries for " + std::to_string(d.n) +
                 " iterations");
        d.scalars.emplace_back(sc.at("value").as_str(), std::move(vals));
    }
    pairs("slices", d.slices, false);
    for (const auto & b : j.at("body").items()) d.body.push_back(parse_driver(b, syms));
    return d;
}

Program parse_program(const std::string & text) {
    const Json j = JsonReader(text).document();
    Program prog;
    prog.format = (int) j.at("format_version").as_int();
    if (prog.format < 1 || prog.format > 3)
        fail("program format_version " + std::to_string(prog.format) +
             " is not supported (this runtime reads 1 to 3)");
    if (const Json * s = j.find("symbols"))
        for (const auto & e : s->items())
            prog.symbols.push_back({e.at("name").as_str(), e.at("min").as_int(), e.at("max").as_int()});
    for (const auto & v : j.at("values").items()) prog.values.push_back(parse_tensor(v, prog.symbols));
    for (const auto & js : j.at("stages").items()) {
        StageSpec s;
        s.name = js.at("name").as_str();
        std::vector<bool> used(prog.symbols.size(), false);
        for (const auto & p : js.at("params").items()) {
            s.params.push_back(parse_tensor(p, prog.symbols));
            for (const auto & d : s.params.back().ne_x) d.uses(used);
        }
        s.outputs = js.at("outputs").strings();
        for (const auto & jn : js.at("nodes").items()) {
            NodeSpec n;
            n.id = jn.at("id").as_str();
            n.op = jn.at("op").as_str();
            n.src = jn.at("src").strings();
            n.type = parse_type_name(jn.at("type").as_str());
            parse_ne(jn.at("ne"), prog.symbols, n.ne_x);
            if (const Json * p = jn.find("p")) n.p = *p;
            if (const Json * l = jn.find("loc"); l && l->kind == Json::Str) n.loc = l->s;
            for (const auto & d : n.ne_x) d.uses(used);
            for (const char * key : {"start", "stop"})
                if (const Json * v = n.p.find(key); v && v->kind != Json::Num) {
                    n.p_x.emplace_back(key, parse_dim(*v, prog.symbols));
                    n.p_x.back().second.uses(used);
                }
            s.nodes.push_back(std::move(n));
        }
        s.symbolic = std::find(used.begin(), used.end(), true) != used.end();
        prog.stages.push_back(std::move(s));
    }
    auto entry = [&](const Json & je, const std::string & name) {
        EntrySpec e;
        e.name = name;
        e.inputs = je.at("inputs").strings();
        e.outputs = je.at("outputs").strings();
        for (const auto & d : je.at("driver").items()) e.driver.push_back(parse_driver(d, prog.symbols));
        return e;
    };
    if (const Json * es = j.find("entries"))
        for (const auto & je : es->items()) prog.entries.push_back(entry(je, je.at("name").as_str()));
    else
        prog.entries.push_back(entry(j, "main"));
    if (prog.entries.empty()) fail("program has no entry point");
    if (const Json * st = j.find("state")) prog.state = st->strings();
    std::vector<int64_t> lo;
    for (const auto & sy : prog.symbols) lo.push_back(sy.min);
    prog.bind(lo);
    return prog;
}

}  // namespace
}  // namespace gcq

// ------------------------------------------------------------------------------------ model

namespace gcq {
namespace {

struct Site {
    const StageSpec * stage = nullptr;
    int stage_index = -1;
    ggml_context * ctx = nullptr;
    ggml_cgraph * gf = nullptr;
    ggml_gallocr_t ga = nullptr;
    bool stale = false;
};

struct StageStat {
    double ms = 0.0;
    int calls = 0;
};

// A ggml API call that reports failure through the library's error record (the void tensor
// functions), turned into an exception.
template <class F>
void must(const std::string & what, F && f) {
    const uint64_t before = error_count();
    f();
    if (error_count() != before) fail(what + ": " + last_error());
}

std::string ne_str(const int64_t * ne) {
    return "[" + std::to_string(ne[0]) + ", " + std::to_string(ne[1]) + ", " + std::to_string(ne[2]) + ", " +
           std::to_string(ne[3]) + "]";
}

[[noreturn]] void node_fail(const NodeSpec & n, const std::string & msg) {
    std::string where = n.id + " (" + n.op + ")";
    if (!n.loc.empty()) where += " at " + n.loc;
    fail(where + ": " + msg);
}

// A step-1 slice of x along ggml dim `dim` from `start`, of shape ne. A size-1 dim gets the packed
// stride (it never moves an address, and layout checks compare strides across size-1 dims).
ggml_tensor * slice_of(ggml_context * ctx, ggml_tensor * x, int dim, int64_t start, const int64_t * ne) {
    size_t nb[4] = {x->nb[0], x->nb[1], x->nb[2], x->nb[3]};
    for (int k = 1; k < 4; k++)
        if (ne[k] == 1) nb[k] = nb[k - 1] * (size_t) ne[k - 1];
    return ggml_view_4d(ctx, x, ne[0], ne[1], ne[2], ne[3], nb[1], nb[2], nb[3], (size_t) start * x->nb[dim]);
}

// A reshape: ggml_reshape_4d of a contiguous x; of a strided x only one that adds or drops size-1
// dims (the other dims keep order and strides); NULL otherwise.
ggml_tensor * reshape_of(ggml_context * ctx, ggml_tensor * x, const int64_t * ne) {
    if (ggml_is_contiguous(x)) return ggml_reshape_4d(ctx, x, ne[0], ne[1], ne[2], ne[3]);
    size_t nb[4] = {x->nb[0], 0, 0, 0};
    int k = 0;  // next dim of x
    for (int i = 0; i < 4; i++) {
        if (ne[i] == 1) {
            if (i > 0) nb[i] = nb[i - 1] * (size_t) ne[i - 1];
            continue;
        }
        while (k < 4 && x->ne[k] == 1) k++;
        if (k == 4 || x->ne[k] != ne[i]) return nullptr;
        nb[i] = x->nb[k++];
    }
    while (k < 4 && x->ne[k] == 1) k++;
    if (k != 4 || nb[0] != x->nb[0]) return nullptr;
    return ggml_view_4d(ctx, x, ne[0], ne[1], ne[2], ne[3], nb[1], nb[2], nb[3], 0);
}

// One program node as ggml calls (the op surface of runtime/src/ops.cpp:56-309 that this library
// runs: binaries and unaries as ops.cpp:76-100, and the rest below; the others fail here with the
// node's name).
ggml_tensor * emit(ggml_context * ctx, const NodeSpec & n, const std::vector<ggml_tensor *> & s) {
    auto need = [&](size_t lo, size_t hi) {
        if (s.size() < lo || s.size() > hi)
            node_fail(n, "expected " + std::to_string(lo) + (lo == hi ? "" : "-" + std::to_string(hi)) +
                             " inputs, got " + std::to_string(s.size()));
    };
    const std::string & op = n.op;
    ggml_tensor * t = nullptr;
    using Binary = ggml_tensor * (*)(ggml_context *, ggml_tensor *, ggml_tensor *);
    using Unary = ggml_tensor * (*)(ggml_context *, ggml_tensor *);
    static const std::map<std::string, Binary> binaries = {
        {"add", ggml_add}, {"sub", ggml_sub}, {"mul", ggml_mul}, {"div", ggml_div}};
    // gelu_tanh is the tanh form, which is what ggml_gelu computes here.
    static const std::map<std::string, Unary> unaries = {
        {"relu", ggml_relu}, {"gelu", ggml_gelu},       {"gelu_tanh", ggml_gelu}, {"gelu_erf", ggml_gelu_erf},
        {"silu", ggml_silu}, {"tanh", ggml_tanh},       {"sigmoid", ggml_sigmoid}, {"exp", ggml_exp},
        {"log", ggml_log},   {"neg", ggml_neg},         {"abs", ggml_abs},         {"sqr", ggml_sqr},
        {"sqrt", ggml_sqrt}, {"sin", ggml_sin},         {"cos", ggml_cos},         {"softplus", ggml_softplus}};
    if (const auto b = binaries.find(op); b != binaries.end()) {
        need(2, 2);
        if (!ggml_can_repeat(s[1], s[0])) node_fail(n, "cannot broadcast " + ne_str(s[1]->ne) + " into " + ne_str(s[0]->ne));
        t = b->second(ctx, s[0], s[1]);
    } else if (const auto u = unaries.find(op); u != unaries.end()) {
        need(1, 1);
        t = u->second(ctx, s[0]);
    } else if (op == "mean" || op == "sum_rows") {
        need(1, 1);
        t = op == "mean" ? ggml_mean(ctx, s[0]) : ggml_sum_rows(ctx, s[0]);
    } else if (op == "clamp") {
        need(1, 1);
        t = ggml_clamp(ctx, s[0], (float) n.num("min"), (float) n.num("max"));
    } else if (op == "repeat") {
        need(1, 1);
        for (int k = 0; k < 4; k++)
            if (s[0]->ne[k] <= 0 || n.ne[k] % s[0]->ne[k] != 0) node_fail(n, "cannot tile " + ne_str(s[0]->ne) + " to " + ne_str(n.ne));
        t = ggml_repeat_4d(ctx, s[0], n.ne[0], n.ne[1], n.ne[2], n.ne[3]);
    } else if (op == "concat") {
        need(2, 2);
        t = ggml_concat(ctx, s[0], s[1], (int) n.integer("dim"));
    } else if (op == "norm") {
        need(1, 1);
        t = ggml_norm(ctx, s[0], (float) n.num("eps"));
    } else if (op == "cont") {
        need(1, 1);
        t = ggml_cont(ctx, s[0]);
    } else if (op == "mul_mat") {
        need(2, 2);
        ggml_tensor *a = s[0], *b = s[1];
        if (a->ne[0] != b->ne[0] || b->ne[2] % a->ne[2] != 0 || b->ne[3] % a->ne[3] != 0)
            node_fail(n, "cannot multiply " + ne_str(a->ne) + " by " + ne_str(b->ne));
        if (ggml_is_transposed(a)) node_fail(n, "weight operand is transposed; it needs a cont first");
        t = ggml_mul_mat(ctx, a, b);
        if (t && n.has("acc") && n.integer("acc") != 0) ggml_prec_set_acc(t, GGML_PREC_F32);
    } else if (op == "scale") {
        need(1, 1);
        const ggml_tensor * x = s[0];
        if (x->nb[0] != ggml_type_size(x->type) || x->nb[2] != x->nb[1] * x->ne[1] || x->nb[3] != x->nb[2] * x->ne[2])
            node_fail(n, "input " + ne_str(x->ne) + " is a strided view; it needs a cont first");
        const float sc = (float) n.num("s"), b = (float) n.num_or("b", 0.0);
        t = b == 0.0f ? ggml_scale(ctx, s[0], sc) : ggml_scale_bias(ctx, s[0], sc, b);
    } else if (op == "rms_norm") {
        need(1, 1);
        t = ggml_rms_norm(ctx, s[0], (float) n.num("eps"));
    } else if (op == "soft_max") {
        need(1, 2);
        t = ggml_soft_max_ext(ctx, s[0], s.size() > 1 ? s[1] : nullptr, (float) n.num_or("scale", 1.0),
                              (float) n.num_or("max_bias", 0.0));
    } else if (op == "reshape") {
        need(1, 1);
        if (ggml_nelements(s[0]) != n.ne[0] * n.ne[1] * n.ne[2] * n.ne[3])
            node_fail(n, "cannot reshape " + ne_str(s[0]->ne) + " to " + ne_str(n.ne));
        t = reshape_of(ctx, s[0], n.ne);
        if (!t)
            node_fail(n, "input is a strided view and the reshape does more than add or drop size-1 dims; it needs a "
                         "cont first");
    } else if (op == "permute") {
        need(1, 1);
        const Json * ax = n.p.find("axes");
        if (!ax || ax->items().size() != 4) node_fail(n, "'axes' must have 4 entries");
        t = ggml_permute(ctx, s[0], (int) ax->arr[0].as_int(), (int) ax->arr[1].as_int(), (int) ax->arr[2].as_int(),
                         (int) ax->arr[3].as_int());
    } else if (op == "view") {
        need(1, 1);
        const int64_t dim = n.integer("dim"), start = n.integer("start");
        if (dim < 0 || dim > 3 || start < 0 || start + n.ne[dim] > s[0]->ne[dim])
            node_fail(n, "slice out of range of " + ne_str(s[0]->ne));
        t = slice_of(ctx, s[0], (int) dim, start, n.ne);
    } else if (op == "flash_attn") {
        need(3, 4);
        ggml_tensor *q = s[0], *k = s[1], *v = s[2];
        ggml_tensor * mask = s.size() > 3 ? s[3] : nullptr;
        if (k->ne[0] != q->ne[0] || k->ne[1] != v->ne[1] || q->ne[3] != k->ne[3] || q->ne[3] != v->ne[3] ||
            q->ne[2] % k->ne[2] != 0)
            node_fail(n, "q " + ne_str(q->ne) + ", k " + ne_str(k->ne) + ", v " + ne_str(v->ne) + " do not line up");
        if (mask && (mask->type != GGML_TYPE_F16 || !ggml_is_contiguous(mask) || q->ne[2] % mask->ne[2] != 0))
            node_fail(n, "mask must be a contiguous f16 tensor broadcastable over heads");
        t = ggml_flash_attn_ext(ctx, q, k, v, mask, (float) n.num("scale"), 0.0f, 0.0f);
        if (t) ggml_prec_set_acc(t, GGML_PREC_F32);
    } else if (op == "swiglu") {
        need(2, 2);
        if (!ggml_are_same_shape(s[0], s[1]) || !ggml_is_contiguous(s[0]) || !ggml_is_contiguous(s[1]))
            node_fail(n, "swiglu needs a gate and an up of one shape, both contiguous");
        t = ggml_swiglu_split(ctx, s[0], s[1]);
    } else if (op == "set_rows") {
        need(3, 3);
        ggml_tensor *dst = s[0], *src = s[1], *idx = s[2];
        if (dst->ne[0] != src->ne[0] || dst->ne[2] != src->ne[2] || dst->ne[3] != src->ne[3] ||
            src->ne[1] != idx->ne[0] || idx->ne[1] != 1 || idx->type != GGML_TYPE_I32 ||
            (src->type != GGML_TYPE_F32 && src->type != GGML_TYPE_F16))
            node_fail(n, "cannot write rows " + ne_str(src->ne) + " at indices " + ne_str(idx->ne) + " into " +
                             ne_str(dst->ne));
        if (dst->nb[0] != ggml_type_size(dst->type) || src->nb[0] != ggml_type_size(src->type))
            node_fail(n, "set_rows needs rows that are contiguous");
        t = ggml_set_rows(ctx, dst, src, idx);
    } else if (op == "rope") {
        need(2, 3);
        ggml_tensor *x = s[0], *pos = s[1];
        ggml_tensor * ff = s.size() > 2 ? s[2] : nullptr;
        const int n_dims = (int) n.integer("n_dims");
        if (x->type != GGML_TYPE_F32 || x->nb[0] != ggml_type_size(x->type) || pos->type != GGML_TYPE_I32 ||
            !ggml_is_vector(pos) || pos->ne[0] != x->ne[2] || n_dims % 2 || n_dims > x->ne[0] ||
            (ff && (ff->type != GGML_TYPE_F32 || ff->ne[0] < n_dims / 2)))
            node_fail(n, "cannot rotate " + ne_str(x->ne) + " at positions " + ne_str(pos->ne));
        t = ggml_rope_ext(ctx, x, pos, ff, n_dims, (int) n.integer("mode"), 0, (float) n.num("freq_base"),
                          (float) n.num("freq_scale"), 0.0f, (float) n.num("attn_factor"), 32.0f, 1.0f);
    } else if (op == "argmax") {
        need(1, 1);
        if (!ggml_is_matrix(s[0])) node_fail(n, "argmax needs a matrix, got " + ne_str(s[0]->ne));
        t = ggml_argmax(ctx, s[0]);
    } else if (op == "get_rows") {
        need(2, 2);
        if (s[1]->type != GGML_TYPE_I32) node_fail(n, "row indices must be i32");
        t = ggml_get_rows(ctx, s[0], s[1]);
    } else if (op == "cast") {
        need(1, 1);
        t = ggml_cast(ctx, s[0], (ggml_type) n.type);
    } else {
        node_fail(n, "op is not supported by this runtime");
    }
    if (!t) node_fail(n, std::string("ggml could not build it: ") + ggml_last_error());
    if (t->type != n.type)
        node_fail(n, std::string("produced type ") + ggml_type_name(t->type) + ", program expects " +
                         ggml_type_name((ggml_type) n.type));
    for (int k = 0; k < 4; k++)
        if (t->ne[k] != n.ne[k]) node_fail(n, "produced shape " + ne_str(t->ne) + ", program expects " + ne_str(n.ne));
    ggml_set_name(t, n.id.c_str());
    return t;
}

}  // namespace
}  // namespace gcq

using namespace gcq;

struct ggml_compiler_stage_build {
    ggml_context * ctx = nullptr;
    ggml_backend_t backend = nullptr;
    ggml_context * wctx = nullptr;
    const std::vector<int64_t> * binding = nullptr;
    std::vector<ggml_tensor *> params, outputs;
    std::string error;
};

struct ggml_compiler_model {
    Program prog;
    std::map<std::string, ggml_compiler_build_fn> builders;
    GgufFile file;
    ggml_backend_t backend = nullptr;
    ggml_context * wctx = nullptr;  // weights and constants
    ggml_backend_buffer_t wbuf = nullptr;
    ggml_context * vctx = nullptr;  // driver values
    ggml_backend_buffer_t vbuf = nullptr;
    ggml_context * bctx = nullptr;  // per binding: views of symbolic values
    std::vector<ggml_context *> slice_ctxs;  // per binding: row views of loop slice sources
    std::vector<int64_t> binding;   // the next run's
    std::vector<int64_t> built;     // the views' and graphs'
    std::unordered_map<std::string, ggml_tensor *> store;  // each value's memory
    std::unordered_map<std::string, ggml_tensor *> view;   // each value as the bound graphs see it
    std::unordered_map<std::string, const TensorSpec *> spec;
    struct Entry {
        const EntrySpec * spec = nullptr;
        std::vector<const TensorSpec *> inputs, outputs;
    };
    std::vector<Entry> entries;
    std::map<std::string, bool> input_set;
    std::vector<Site> sites;
    std::vector<StageStat> stage_stats;
    ggml_compiler_stats last{};

    ~ggml_compiler_model() {
        for (auto & c : sites) {
            if (c.ga) ggml_gallocr_free(c.ga);
            if (c.ctx) ggml_free(c.ctx);
        }
        for (auto * c : slice_ctxs) ggml_free(c);
        if (bctx) ggml_free(bctx);
        if (vbuf) ggml_backend_buffer_free(vbuf);
        if (vctx) ggml_free(vctx);
        if (wbuf) ggml_backend_buffer_free(wbuf);
        if (wctx) ggml_free(wctx);
        if (backend) ggml_backend_free(backend);
    }

    ggml_tensor * value(const std::string & name) const {
        auto it = view.find(name);
        if (it == view.end()) fail("driver value '" + name + "' is not declared");
        return it->second;
    }

    void load(const char * path, const ggml_compiler_options & o) {
        if (o.allow_cpu_fallback) fail("allow_cpu_fallback is not available: this runtime runs on HIP devices only");
        if (o.backend != GGML_COMPILER_BACKEND_HIP && o.backend != GGML_COMPILER_BACKEND_AUTO)
            fail("backend " + std::to_string((int) o.backend) + " is not available: this runtime has the HIP backend "
                 "(GGML_COMPILER_BACKEND_HIP or _AUTO)");
        file.open(path);
        auto it = file.strings.find("ggml_compiler.program");
        if (it == file.strings.end())
            fail(std::string("'") + path + "' has no ggml_compiler.program; it was not written by ggml-compiler compile");
        prog = parse_program(it->second);
        const int n_dev = gcq_device_count();
        if (n_dev == 0) fail("no HIP device");
        if (o.device < 0 || o.device >= n_dev)
            fail("device index " + std::to_string(o.device) + " out of range; " + std::to_string(n_dev) +
                 " HIP device(s) found");
        backend = ggml_backend_hip_init(o.device);
        if (!backend) fail(std::string("cannot start the HIP backend: ") + last_error());
        load_weights();
        for (const auto & sy : prog.symbols) binding.push_back(sy.max);
        prog.bind(binding);
        alloc_values();
        stage_stats.assign(prog.stages.size(), StageStat{});
        bind_values();
        for (auto & e : prog.entries) build_ops(e.driver);
        built = binding;
    }

    void load_weights() {
        if (file.tensors.empty()) return;
        ggml_init_params ip{};
        ip.mem_size = ggml_tensor_overhead() * (file.tensors.size() + 1);
        ip.no_alloc = true;
        wctx = ggml_init(ip);
        for (const auto & in : file.tensors) {
            if (in.type < 0 || in.type >= GGML_TYPE_COUNT || !ggml_type_name((ggml_type) in.type))
                fail("GGUF tensor '" + in.name + "' has unknown type " + std::to_string(in.type));
            ggml_tensor * t = ggml_new_tensor_4d(wctx, (ggml_type) in.type, in.ne[0], in.ne[1], in.ne[2], in.ne[3]);
            if (!t) fail("GGUF tensor '" + in.name + "': " + last_error());
            ggml_set_name(t, in.name.c_str());
        }
        wbuf = ggml_backend_alloc_ctx_tensors(wctx, backend);
        if (!wbuf) fail(std::string("cannot allocate weight buffer: ") + last_error());
        const int fd = ::open(file.path.c_str(), O_RDONLY);
        if (fd < 0) fail("cannot open '" + file.path + "'");
        std::unique_ptr<int, void (*)(int *)> hold(new int(fd), [](int * p) {
            ::close(*p);
            delete p;
        });
        std::vector<uint8_t> staging;
        for (const auto & in : file.tensors) {
            ggml_tensor * t = ggml_get_tensor(wctx, in.name.c_str());
            const size_t n = ggml_nbytes(t);
            staging.resize(n);
            size_t got = 0;
            while (got < n) {
                const ssize_t r = ::pread(fd, staging.data() + got, n - got, (off_t) (file.data_offset + in.offset + got));
                if (r <= 0) fail("short read for tensor " + in.name);
                got += (size_t) r;
            }
            must("upload of tensor " + in.name, [&] { ggml_backend_tensor_set(t, staging.data(), 0, n); });
        }
    }

    void alloc_values() {
        ggml_init_params ip{};
        ip.mem_size = ggml_tensor_overhead() * (prog.values.size() + 1);
        ip.no_alloc = true;
        vctx = ggml_init(ip);
        for (const auto & v : prog.values) {
            ggml_tensor * t = nullptr;
            if (!v.symbolic()) {
                t = ggml_new_tensor_4d(vctx, (ggml_type) v.type, v.ne[0], v.ne[1], v.ne[2], v.ne[3]);
            } else {
                // Room for the largest size over the corners of its symbols' ranges (dims are
                // monotone in each symbol, so a corner holds the maximum).
                std::vector<bool> used(prog.symbols.size(), false);
                for (const auto & d : v.ne_x) d.uses(used);
                std::vector<size_t> idx;
                for (size_t k = 0; k < used.size(); k++)
                    if (used[k]) idx.push_back(k);
                if (idx.size() > 20) fail("value '" + v.name + "' depends on too many symbols");
                int64_t most = 0;
                std::vector<int64_t> b = binding;
                for (size_t mask = 0; mask < ((size_t) 1 << idx.size()); mask++) {
                    for (size_t k = 0; k < idx.size(); k++)
                        b[idx[k]] = (mask >> k) & 1 ? prog.symbols[idx[k]].max : prog.symbols[idx[k]].min;
                    int64_t n = 1;
                    for (const auto & d : v.ne_x) n *= d.eval(b);
                    most = std::max(most, n);
                }
                t = ggml_new_tensor_1d(vctx, (ggml_type) v.type, most);
            }
            if (!t) fail("driver value '" + v.name + "': " + last_error());
            ggml_set_name(t, v.name.c_str());
            store[v.name] = t;
            view[v.name] = t;
            spec[v.name] = &v;
        }
        if (!prog.values.empty()) {
            vbuf = ggml_backend_alloc_ctx_tensors(vctx, backend);
            if (!vbuf) fail(std::string("cannot allocate driver value buffer: ") + last_error());
            must("clearing the driver values", [&] { ggml_backend_buffer_clear(vbuf, 0); });
        }
        for (const auto & e : prog.entries) {
            Entry en;
            en.spec = &e;
            for (const auto & name : e.inputs) {
                if (!spec.count(name)) fail("input '" + name + "' is not a declared value");
                en.inputs.push_back(spec[name]);
                input_set[name] = false;
            }
            for (const auto & name : e.outputs) {
                if (!spec.count(name)) fail("output '" + name + "' is not a declared value");
                en.outputs.push_back(spec[name]);
            }
            entries.push_back(std::move(en));
        }
        for (const auto & name : prog.state)
            if (!spec.count(name)) fail("state '" + name + "' is not a declared value");
    }

    // Views with the binding's shape over the storage of every symbolic value.
    void bind_values() {
        if (bctx) {
            ggml_free(bctx);
            bctx = nullptr;
        }
        size_t n = 0;
        for (const auto & v : prog.values) n += v.symbolic();
        if (n == 0) return;
        ggml_init_params ip{};
        ip.mem_size = ggml_tensor_overhead() * (n + 1);
        ip.no_alloc = true;
        bctx = ggml_init(ip);
        for (const auto & v : prog.values) {
            if (!v.symbolic()) continue;
            const size_t nb1 = ggml_row_size((ggml_type) v.type, v.ne[0]), nb2 = nb1 * (size_t) v.ne[1],
                         nb3 = nb2 * (size_t) v.ne[2];
            ggml_tensor * t = ggml_view_4d(bctx, store.at(v.name), v.ne[0], v.ne[1], v.ne[2], v.ne[3], nb1, nb2, nb3, 0);
            if (!t || ggml_backend_view_init(t) != GGML_STATUS_SUCCESS) fail("cannot view driver value '" + v.name + "'");
            ggml_set_name(t, v.name.c_str());
            view[v.name] = t;
        }
    }

    void rebind() {
        if (binding == built) return;
        prog.bind(binding);
        for (auto * c : slice_ctxs) ggml_free(c);
        slice_ctxs.clear();
        bind_values();
        for (auto & e : prog.entries) build_ops(e.driver);
        built = binding;
    }

    void build_ops(std::vector<DriverOp> & ops) {
        for (auto & d : ops) {
            if (!d.loop) {
                build_call(d);
                continue;
            }
            for (const auto & c : d.carry) {
                ggml_tensor *a = value(c.first), *b = value(c.second);
                if (a->type != b->type || !ggml_are_same_shape(a, b))
                    fail("loop carry '" + c.first + "' does not match its initial value '" + c.second + "'");
            }
            for (const auto & sc : d.scalars)
                if (value(sc.first)->type != GGML_TYPE_F32) fail("loop scalar '" + sc.first + "' must be f32");
            d.slice_rows.clear();
            if (!d.slices.empty()) {
                ggml_init_params ip{};
                ip.mem_size = ggml_tensor_overhead() * (d.slices.size() * (size_t) d.n + 1);
                ip.no_alloc = true;
                ggml_context * vc = ggml_init(ip);
                slice_ctxs.push_back(vc);
                for (const auto & sl : d.slices) {
                    ggml_tensor *a = value(sl.first), *b = value(sl.second);
                    // the source is [n, ...a] in PyTorch order: a's elements n times, outermost
                    if (a->type != b->type || ggml_nelements(b) != ggml_nelements(a) * d.n || !ggml_is_contiguous(b))
                        fail("loop slice '" + sl.first + "' does not match its source '" + sl.second + "'");
                    std::vector<ggml_tensor *> rows;
                    for (int i = 0; i < d.n; i++) {
                        ggml_tensor * r = ggml_view_4d(vc, b, a->ne[0], a->ne[1], a->ne[2], a->ne[3], a->nb[1], a->nb[2],
                                                       a->nb[3], (size_t) i * ggml_nbytes(a));
                        if (!r || ggml_backend_view_init(r) != GGML_STATUS_SUCCESS)
                            fail("cannot view loop slice source '" + sl.second + "'");
                        rows.push_back(r);
                    }
                    d.slice_rows.push_back(std::move(rows));
                }
            }
            build_ops(d.body);
        }
    }

    void build_call(DriverOp & d) {
        if (d.site >= 0) {
            // Rebinding: a stage with static shapes keeps its graph; any other is rebuilt when its
            // site next runs (so one entry never rebuilds another's stages).
            Site & c = sites[d.site];
            if (!c.stage->symbolic) return;
            if (c.ctx) ggml_free(c.ctx);
            c.ctx = nullptr;
            c.gf = nullptr;
            c.stale = true;
            return;
        }
        Site c;
        for (size_t k = 0; k < prog.stages.size(); k++)
            if (prog.stages[k].name == d.stage) {
                c.stage = &prog.stages[k];
                c.stage_index = (int) k;
            }
        if (!c.stage) fail("driver calls unknown stage '" + d.stage + "'");
        d.site = (int) sites.size();
        sites.push_back(c);
        build_site(d);
    }

    void build_site(const DriverOp & d) {
        Site & cs = sites[d.site];
        const StageSpec & st = *cs.stage;
        cs.stale = false;
        if (d.args.size() != st.params.size() || d.out.size() != st.outputs.size())
            fail("call to stage '" + st.name + "' has the wrong number of arguments or results");
        const size_t n_tensors = 8 * st.nodes.size() + 2 * st.outputs.size() + 16;
        const size_t graph_size = n_tensors + st.params.size() + file.tensors.size() + 64;
        ggml_init_params ip{};
        ip.mem_size = ggml_tensor_overhead() * n_tensors + ggml_graph_overhead_custom(graph_size, false);
        ip.no_alloc = true;
        cs.ctx = ggml_init(ip);
        std::unordered_map<std::string, ggml_tensor *> env;
        for (size_t k = 0; k < st.params.size(); k++) {
            ggml_tensor * arg = value(d.args[k]);
            const TensorSpec & p = st.params[k];
            for (int q = 0; q < 4; q++)
                if (arg->ne[q] != p.ne[q] || arg->type != p.type)
                    fail("stage '" + st.name + "' parameter " + p.name + " does not match value '" + d.args[k] + "'");
            env[p.name] = arg;
        }
        std::vector<ggml_tensor *> results;
        auto bf = builders.find(st.name);
        if (bf != builders.end()) {
            ggml_compiler_stage_build b;
            b.ctx = cs.ctx;
            b.backend = backend;
            b.wctx = wctx;
            b.binding = &binding;
            for (const auto & p : st.params) b.params.push_back(env.at(p.name));
            b.outputs.assign(st.outputs.size(), nullptr);
            if (bf->second(&b) != 0 || !b.error.empty())
                fail("builder for stage '" + st.name + "' failed: " + b.error);
            std::unordered_map<std::string, const NodeSpec *> nodes;
            for (const auto & n : st.nodes) nodes[n.id] = &n;
            for (size_t k = 0; k < st.outputs.size(); k++) {
                ggml_tensor * t = b.outputs[k];
                if (!t) fail("builder for stage '" + st.name + "' left output " + std::to_string(k) + " unset");
                auto it = nodes.find(st.outputs[k]);
                if (it != nodes.end()) {
                    bool same = t->type == it->second->type;
                    for (int q = 0; q < 4; q++) same = same && t->ne[q] == it->second->ne[q];
                    if (!same)
                        fail("builder for stage '" + st.name + "' output " + std::to_string(k) +
                             " does not match the program");
                }
                results.push_back(t);
            }
        } else {
            std::vector<ggml_tensor *> src;
            for (const auto & n : st.nodes) {
                src.clear();
                for (const auto & name : n.src) {
                    auto it = env.find(name);
                    if (it != env.end()) {
                        src.push_back(it->second);
                        continue;
                    }
                    ggml_tensor * w = wctx ? ggml_get_tensor(wctx, name.c_str()) : nullptr;
                    if (!w) fail("stage '" + st.name + "' node " + n.id + " reads unknown tensor '" + name + "'");
                    src.push_back(w);
                }
                env[n.id] = emit(cs.ctx, n, src);
            }
            for (const auto & id : st.outputs) {
                auto it = env.find(id);
                if (it == env.end()) fail("stage '" + st.name + "' returns unknown value '" + id + "'");
                results.push_back(it->second);
            }
        }
        cs.gf = ggml_new_graph_custom(cs.ctx, graph_size, false);
        for (ggml_tensor * t : results) ggml_build_forward_expand(cs.gf, t);
        // Copies into the driver values go last, after every read of the stage's arguments.
        for (size_t k = 0; k < results.size(); k++) {
            ggml_tensor *dst = value(d.out[k]), *res = results[k];
            if (res == dst) continue;
            // A result that is its value's memory already (set_rows into the state it read).
            if (res->data && res->data == dst->data && res->type == dst->type && ggml_are_same_shape(res, dst) &&
                ggml_is_contiguous(res))
                continue;
            if (ggml_nelements(res) != ggml_nelements(dst) || res->type != dst->type)
                fail("stage '" + st.name + "' result " + std::to_string(k) + " does not match value '" + d.out[k] + "'");
            ggml_build_forward_expand(cs.gf, ggml_cpy(cs.ctx, res, dst));
        }
        std::string unsupported;
        for (int k = 0; k < ggml_graph_n_nodes(cs.gf); k++) {
            ggml_tensor * t = ggml_graph_node(cs.gf, k);
            if (!ggml_backend_supports_op(backend, t))
                unsupported += std::string("\n  ") + t->name + " (" + ggml_op_desc(t) + "): " + last_error();
        }
        if (!unsupported.empty())
            fail(std::string("backend ") + ggml_backend_name(backend) + " cannot run these nodes of stage '" + st.name +
                 "':" + unsupported);
        if (!cs.ga) cs.ga = ggml_gallocr_new(ggml_backend_get_default_buffer_type(backend));
        if (!ggml_gallocr_alloc_graph(cs.ga, cs.gf))
            fail("cannot allocate compute buffer for stage '" + st.name + "': " + last_error());
    }

    void run_ops(const std::vector<DriverOp> & ops) {
        using clock = std::chrono::steady_clock;
        for (const auto & d : ops) {
            if (!d.loop) {
                if (sites[d.site].stale) build_site(d);
                Site & c = sites[d.site];
                const auto t0 = clock::now();
                const ggml_status status = ggml_backend_graph_compute(backend, c.gf);
                if (status != GGML_STATUS_SUCCESS)
                    fail("stage '" + c.stage->name + "' failed: " + ggml_status_to_string(status) + ": " + last_error());
                auto & st = stage_stats[c.stage_index];
                st.ms += std::chrono::duration<double, std::milli>(clock::now() - t0).count();
                st.calls++;
                last.n_calls++;
                continue;
            }
            for (const auto & c : d.carry)
                must("loop carry '" + c.first + "'", [&] { ggml_backend_tensor_copy(value(c.second), value(c.first)); });
            const int n = d.n_symbol >= 0 ? (int) binding[d.n_symbol] : d.n;
            std::vector<int32_t> starts;
            for (const auto & c : d.counters) {
                int32_t v = 0;
                must("loop counter '" + c.first + "'", [&] { ggml_backend_tensor_get(value(c.second), &v, 0, sizeof v); });
                starts.push_back(v);
            }
            for (const auto & c : d.collect) {
                ggml_tensor * t = store.at(c.first);
                must("loop collect '" + c.first + "'", [&] { ggml_backend_tensor_memset(t, 0, 0, ggml_nbytes(t)); });
            }
            std::vector<float> fill;
            std::vector<int64_t> ext;
            std::vector<char> row;
            for (int i = 0; i < n; i++) {
                for (const auto & sc : d.scalars) {
                    ggml_tensor * t = value(sc.first);
                    fill.assign((size_t) ggml_nelements(t), sc.second[(size_t) i]);
                    must("loop scalar '" + sc.first + "'", [&] { ggml_backend_tensor_set(t, fill.data(), 0, ggml_nbytes(t)); });
                }
                for (size_t k = 0; k < d.slices.size(); k++)
                    must("loop slice '" + d.slices[k].first + "'",
                         [&] { ggml_backend_tensor_copy(d.slice_rows[k][(size_t) i], value(d.slices[k].first)); });
                for (size_t k = 0; k < d.counters.size(); k++) {
                    const int32_t v = starts[k] + i;
                    must("loop counter '" + d.counters[k].first + "'",
                         [&] { ggml_backend_tensor_set(value(d.counters[k].first), &v, 0, sizeof v); });
                }
                if (!d.bind.empty()) {
                    ext = binding;
                    for (int32_t v : starts) ext.push_back(v + i);
                    for (const auto & bnd : d.bind) {
                        const int64_t v = bnd.second.eval(ext);
                        const Symbol & sy = prog.symbols[(size_t) bnd.first];
                        if (v < sy.min || v > sy.max)
                            fail("loop binds " + sy.name + " = " + std::to_string(v) + ", outside its range");
                        binding[(size_t) bnd.first] = v;
                    }
                    rebind();  // a no-op unless a symbol changed
                }
                for (const auto & m : d.masks) {
                    // the causal mask row(s) of position pos: 0 up to pos, -inf after
                    const TensorSpec & v = *spec.at(m.first);
                    const int64_t pos = starts[(size_t) m.second] + i, len = v.ne[0];
                    fill.resize((size_t) (v.ne[0] * v.ne[1] * v.ne[2] * v.ne[3]));
                    for (size_t j = 0; j < fill.size(); j++) fill[j] = (int64_t) (j % (size_t) len) <= pos ? 0.0f : -INFINITY;
                    if (v.type != GGML_TYPE_F32) fail("loop mask '" + m.first + "' must be f32");
                    must("loop mask '" + m.first + "'",
                         [&] { ggml_backend_tensor_set(store.at(m.first), fill.data(), 0, fill.size() * sizeof(float)); });
                }
                run_ops(d.body);
                for (const auto & c : d.collect) {
                    const size_t nb = spec.at(c.second)->nbytes(binding);
                    row.resize(nb);
                    must("loop collect '" + c.first + "'", [&] {
                        ggml_backend_tensor_get(store.at(c.second), row.data(), 0, nb);
                        ggml_backend_tensor_set(store.at(c.first), row.data(), (size_t) i * nb, nb);
                    });
                }
                bool stop = false;
                for (const auto & u : d.until) {
                    int32_t v = 0;
                    must("loop until '" + u.first + "'", [&] { ggml_backend_tensor_get(store.at(u.first), &v, 0, sizeof v); });
                    stop = stop || std::find(u.second.begin(), u.second.end(), v) != u.second.end();
                }
                if (stop) break;
            }
        }
    }
};

// ------------------------------------------------------------------------------------ C API

namespace {

int fill_info(const TensorSpec & v, const std::vector<int64_t> & b, ggml_compiler_tensor_info * info) {
    require(info != nullptr, "info is NULL");
    std::vector<int64_t> shape;
    for (const auto & d : v.shape_x) shape.push_back(d.eval(b));
    switch (v.type) {
        case GGML_TYPE_F32: info->dtype = GGML_COMPILER_DTYPE_F32; break;
        case GGML_TYPE_F16: info->dtype = GGML_COMPILER_DTYPE_F16; break;
        case GGML_TYPE_I32: info->dtype = GGML_COMPILER_DTYPE_I32; break;
        default: fail("value '" + v.name + "' has a type the C API cannot describe");
    }
    require(shape.size() <= GGML_COMPILER_MAX_RANK, "value '" + v.name + "' has rank above GGML_COMPILER_MAX_RANK");
    info->name = v.name.c_str();
    info->ndim = (int) shape.size();
    for (size_t k = 0; k < shape.size(); k++) info->shape[k] = shape[k];
    info->nbytes = v.nbytes(b);
    return 0;
}

// The symbols an input's shape fixes: a dim with one unknown symbol is solved by bisection over
// the symbol's range (dims are monotone in each symbol); then every dim must match.
void solve_shape(ggml_compiler_model * m, const TensorSpec & v, const std::vector<int64_t> & shape) {
    if (shape.size() != v.shape_x.size())
        fail("input '" + v.name + "' has rank " + std::to_string(v.shape_x.size()) + ", got " +
             std::to_string(shape.size()));
    std::vector<int64_t> b = m->binding;
    std::vector<bool> known(b.size(), false);
    for (int pass = 0; pass < 2; pass++) {
        for (size_t i = 0; i < shape.size(); i++) {
            std::vector<bool> used(b.size(), false);
            v.shape_x[i].uses(used);
            int unknown = -1, n_unknown = 0;
            for (size_t k = 0; k < used.size(); k++)
                if (used[k] && !known[k]) {
                    unknown = (int) k;
                    n_unknown++;
                }
            if (n_unknown != 1) continue;
            const Symbol & sy = m->prog.symbols[(size_t) unknown];
            int64_t lo = sy.min, hi = sy.max;
            while (lo < hi) {  // the smallest value whose dim reaches shape[i]
                const int64_t mid = lo + (hi - lo) / 2;
                b[(size_t) unknown] = mid;
                if (v.shape_x[i].eval(b) < shape[i]) lo = mid + 1;
                else hi = mid;
            }
            b[(size_t) unknown] = lo;
            if (v.shape_x[i].eval(b) != shape[i])
                fail("input '" + v.name + "': no " + sy.name + " in [" + std::to_string(sy.min) + ", " +
                     std::to_string(sy.max) + "] gives dim " + std::to_string(i) + " = " + std::to_string(shape[i]));
            known[(size_t) unknown] = true;
        }
    }
    std::vector<int64_t> got;
    for (const auto & d : v.shape_x) got.push_back(d.eval(b));
    if (got != shape) {
        std::string want, have;
        for (auto d : shape) want += (want.empty() ? "" : ", ") + std::to_string(d);
        for (auto d : got) have += (have.empty() ? "" : ", ") + std::to_string(d);
        fail("input '" + v.name + "' cannot have shape [" + want + "] (with the other symbols as bound, it is [" + have +
             "])");
    }
    m->binding = b;
}

// Run f; on an error record the message and return `bad`.
template <class T, class F>
T guarded_value(T bad, F && f) {
    T out = bad;
    if (guarded([&] { out = f(); }) != 0) return bad;
    return out;
}

}  // namespace

extern "C" {

ggml_compiler_model * ggml_compiler_load(const char * path, const ggml_compiler_options * opt) {
    return ggml_compiler_load_with(path, opt, nullptr, 0);
}

ggml_compiler_model * ggml_compiler_load_with(const char * path, const ggml_compiler_options * opt,
                                              const ggml_compiler_builder * builders, int n_builders) {
    const ggml_compiler_options o = opt ? *opt : ggml_compiler_default_options();
    return guarded_value<ggml_compiler_model *>(nullptr, [&]() -> ggml_compiler_model * {
        require(path != nullptr, "path is NULL");
        require(n_builders == 0 || builders != nullptr, "builders is NULL");
        auto m = std::make_unique<ggml_compiler_model>();
        for (int k = 0; k < n_builders; k++) {
            require(builders[k].stage && builders[k].build, "builder " + std::to_string(k) + " is incomplete");
            m->builders[builders[k].stage] = builders[k].build;
        }
        m->load(path, o);
        for (const auto & b : m->builders) {
            bool found = false;
            for (const auto & st : m->prog.stages) found = found || st.name == b.first;
            if (!found) fail("builder for stage '" + b.first + "', which the program does not have");
        }
        return m.release();
    });
}

ggml_context * ggml_compiler_build_ctx(ggml_compiler_stage_build * b) { return b ? b->ctx : nullptr; }

bool ggml_compiler_build_gpu(ggml_compiler_stage_build * b) { return b != nullptr; }  // always a HIP device

bool ggml_compiler_build_supports(ggml_compiler_stage_build * b, const ggml_tensor * t) {
    return b && (!b->backend || ggml_backend_supports_op(b->backend, t));
}

ggml_tensor * ggml_compiler_build_param(ggml_compiler_stage_build * b, int i) {
    if (!b) return nullptr;
    if (i < 0 || i >= (int) b->params.size()) {
        b->error = "parameter index " + std::to_string(i) + " out of range";
        return nullptr;
    }
    return b->params[(size_t) i];
}

ggml_tensor * ggml_compiler_build_weight(ggml_compiler_stage_build * b, const char * name) {
    if (!b) return nullptr;
    ggml_tensor * t = b->wctx && name ? ggml_get_tensor(b->wctx, name) : nullptr;
    if (!t) b->error = std::string("no tensor '") + (name ? name : "(null)") + "' in the GGUF";
    return t;
}

int64_t ggml_compiler_build_symbol(ggml_compiler_stage_build * b, int i) {
    if (!b) return 1;
    if (!b->binding || i < 0 || i >= (int) b->binding->size()) {
        b->error = "symbol index " + std::to_string(i) + " out of range";
        return 1;
    }
    return (*b->binding)[(size_t) i];
}

void ggml_compiler_build_output(ggml_compiler_stage_build * b, int i, ggml_tensor * t) {
    if (!b) return;
    if (i < 0 || i >= (int) b->outputs.size()) {
        b->error = "output index " + std::to_string(i) + " out of range";
        return;
    }
    b->outputs[(size_t) i] = t;
}

const char * ggml_compiler_metadata(const ggml_compiler_model * m, const char * key) {
    if (!m || !key) return nullptr;
    auto it = m->file.strings.find(key);
    return it == m->file.strings.end() ? nullptr : it->second.c_str();
}

void ggml_compiler_free(ggml_compiler_model * m) { delete m; }

const char * ggml_compiler_backend_name(const ggml_compiler_model * m) {
    return m ? ggml_backend_name(m->backend) : nullptr;
}

int ggml_compiler_n_entries(const ggml_compiler_model * m) { return m ? (int) m->entries.size() : -1; }

const char * ggml_compiler_entry_name(const ggml_compiler_model * m, int e) {
    if (!m || e < 0 || e >= (int) m->entries.size()) {
        set_error("entry index out of range");
        return nullptr;
    }
    return m->entries[(size_t) e].spec->name.c_str();
}

int ggml_compiler_entry_n_inputs(const ggml_compiler_model * m, int e) {
    return m && e >= 0 && e < (int) m->entries.size() ? (int) m->entries[(size_t) e].inputs.size() : -1;
}

int ggml_compiler_entry_n_outputs(const ggml_compiler_model * m, int e) {
    return m && e >= 0 && e < (int) m->entries.size() ? (int) m->entries[(size_t) e].outputs.size() : -1;
}

int ggml_compiler_entry_input_info(const ggml_compiler_model * m, int e, int i, ggml_compiler_tensor_info * info) {
    return guarded_value<int>(-1, [&] {
        require(m && e >= 0 && e < (int) m->entries.size() && i >= 0 && i < (int) m->entries[(size_t) e].inputs.size(),
                "input index out of range");
        return fill_info(*m->entries[(size_t) e].inputs[(size_t) i], m->binding, info);
    });
}

int ggml_compiler_entry_output_info(const ggml_compiler_model * m, int e, int i, ggml_compiler_tensor_info * info) {
    return guarded_value<int>(-1, [&] {
        require(m && e >= 0 && e < (int) m->entries.size() && i >= 0 && i < (int) m->entries[(size_t) e].outputs.size(),
                "output index out of range");
        return fill_info(*m->entries[(size_t) e].outputs[(size_t) i], m->binding, info);
    });
}

int ggml_compiler_n_inputs(const ggml_compiler_model * m) { return ggml_compiler_entry_n_inputs(m, 0); }
int ggml_compiler_n_outputs(const ggml_compiler_model * m) { return ggml_compiler_entry_n_outputs(m, 0); }
int ggml_compiler_input_info(const ggml_compiler_model * m, int i, ggml_compiler_tensor_info * info) {
    return ggml_compiler_entry_input_info(m, 0, i, info);
}
int ggml_compiler_output_info(const ggml_compiler_model * m, int i, ggml_compiler_tensor_info * info) {
    return ggml_compiler_entry_output_info(m, 0, i, info);
}

int ggml_compiler_reset(ggml_compiler_model * m) {
    return guarded([&] {
        require(m != nullptr, "model is NULL");
        for (const auto & name : m->prog.state) {
            ggml_tensor * t = m->store.at(name);
            must("reset of '" + name + "'", [&] { ggml_backend_tensor_memset(t, 0, 0, ggml_nbytes(t)); });
        }
    });
}

int ggml_compiler_n_symbols(const ggml_compiler_model * m) { return m ? (int) m->prog.symbols.size() : -1; }

int ggml_compiler_symbol_info(const ggml_compiler_model * m, int i, const char ** name, int64_t * min, int64_t * max,
                              int64_t * value) {
    if (!m || i < 0 || i >= (int) m->prog.symbols.size()) {
        set_error("symbol index out of range");
        return -1;
    }
    const Symbol & sy = m->prog.symbols[(size_t) i];
    if (name) *name = sy.name.c_str();
    if (min) *min = sy.min;
    if (max) *max = sy.max;
    if (value) *value = m->binding[(size_t) i];
    return 0;
}

int ggml_compiler_set_symbol(ggml_compiler_model * m, const char * name, int64_t value) {
    return guarded([&] {
        require(m && name, "NULL argument");
        const int i = m->prog.symbol(name);
        require(i >= 0, "no symbol named '" + std::string(name) + "'");
        const Symbol & sy = m->prog.symbols[(size_t) i];
        require(value >= sy.min && value <= sy.max, "symbol '" + sy.name + "' = " + std::to_string(value) +
                                                        " is outside [" + std::to_string(sy.min) + ", " +
                                                        std::to_string(sy.max) + "]");
        m->binding[(size_t) i] = value;
    });
}

int ggml_compiler_set_input_shape(ggml_compiler_model * m, const char * name, int ndim, const int64_t * shape) {
    return guarded([&] {
        require(m && name && (ndim <= 0 || shape), "NULL argument");
        require(m->input_set.count(name) != 0, "no input named '" + std::string(name) + "'");
        solve_shape(m, *m->spec.at(name), std::vector<int64_t>(shape, shape + std::max(ndim, 0)));
    });
}

int ggml_compiler_set_input(ggml_compiler_model * m, const char * name, const void * data, size_t nbytes) {
    return guarded([&] {
        require(m && name && data, "NULL argument");
        require(m->input_set.count(name) != 0, "no input named '" + std::string(name) + "'");
        const size_t want = m->spec.at(name)->nbytes(m->binding);
        require(nbytes == want, "input '" + std::string(name) + "' needs " + std::to_string(want) + " bytes, got " +
                                    std::to_string(nbytes));
        must("input '" + std::string(name) + "'", [&] { ggml_backend_tensor_set(m->store.at(name), data, 0, nbytes); });
        m->input_set[name] = true;
    });
}

int ggml_compiler_run(ggml_compiler_model * m) {
    if (!m) {
        set_error("model is NULL");
        return -1;
    }
    return ggml_compiler_run_entry(m, m->entries[0].spec->name.c_str());
}

int ggml_compiler_run_entry(ggml_compiler_model * m, const char * entry) {
    return guarded([&] {
        require(m && entry, "NULL argument");
        const ggml_compiler_model::Entry * e = nullptr;
        for (const auto & en : m->entries)
            if (en.spec->name == entry) e = &en;
        require(e != nullptr, "no entry point named '" + std::string(entry) + "'");
        for (const TensorSpec * v : e->inputs)
            require(m->input_set.at(v->name), "input '" + v->name + "' was never set");
        m->rebind();
        for (auto & st : m->stage_stats) st = StageStat{};
        m->last.n_calls = 0;
        const auto t0 = std::chrono::steady_clock::now();
        m->run_ops(e->spec->driver);
        ggml_backend_synchronize(m->backend);
        m->last.ms_total = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    });
}

int ggml_compiler_get_output(ggml_compiler_model * m, const char * name, void * dst, size_t nbytes) {
    return guarded([&] {
        require(m && name && dst, "NULL argument");
        for (const auto & e : m->entries)
            for (const TensorSpec * v : e.outputs) {
                if (v->name != name) continue;
                const size_t have = v->nbytes(m->built);
                require(nbytes == have, "output '" + std::string(name) + "' has " + std::to_string(have) +
                                            " bytes, buffer has " + std::to_string(nbytes));
                must("output '" + std::string(name) + "'", [&] { ggml_backend_tensor_get(m->store.at(name), dst, 0, nbytes); });
                return;
            }
        fail("no output named '" + std::string(name) + "'");
    });
}

int ggml_compiler_last_stats(const ggml_compiler_model * m, ggml_compiler_stats * st) {
    if (!m || !st) {
        set_error("NULL argument");
        return -1;
    }
    *st = m->last;
    return 0;
}

int ggml_compiler_n_stages(const ggml_compiler_model * m) { return m ? (int) m->prog.stages.size() : -1; }

int ggml_compiler_stage_stats(const ggml_compiler_model * m, int i, const char ** name, double * ms, int * n_calls) {
    if (!m || i < 0 || i >= (int) m->prog.stages.size()) {
        set_error("stage index out of range");
        return -1;
    }
    if (name) *name = m->prog.stages[(size_t) i].name.c_str();
    if (ms) *ms = m->stage_stats[(size_t) i].ms;
    if (n_calls) *n_calls = m->stage_stats[(size_t) i].calls;
    return 0;
}

}  // extern "C"
